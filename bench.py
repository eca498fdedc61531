#!/usr/bin/env python3
"""Benchmark of the decode GEMV hot path on one MI355X.

Workload (the headline metric's configuration): the 28-layer stacked
cold-cache Q8_0 GEMV sweep -- five stacked weight sets (attn_q, attn_kv, attn_o,
gate_up, ffn_dn; 436,731,904 bytes, more than the 256 MB MALL), for layer
0..27 the five GEMVs in that order (140 dispatches per step), each with its own
f16 x and y.  One step = one sweep, replayed from a hipGraph of the 140
launches through the C ABI.  Inputs are resident in HBM before timing.

Also measured in the same run:
  * per-dispatch kernel durations (HIP events bound to each launch), from
    which the roofline of the dominant kernel is computed;
  * the f16 vocab GEMV + fused argmax [151936, 1024];
  * the GEMV share of a decode step (28 x q,k,v,o,gate_up,down + vocab);
  * the CPU oracle on a bounded sample of the same sweep (cpu_baseline).

Prints one JSON line.  Only --gpus 1 is supported: this path runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
METRIC = "achieved HBM GB/s (% of peak) on 28-layer Q8_0 GEMV sweep; µs per decode step"
SEED = 20261201


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_bytes(d) -> int:
    """Weights + x + y of one dispatch, each byte counted once."""
    return d.bytes_per_layer + 2 * d.k + 2 * d.n


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kernel-reps", type=int, default=5, help="timed sweeps for per-kernel events")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this path runs on one GPU; --gpus {args.gpus} (WORLD_SIZE={world}) "
              "is not supported. Run with --gpus 1.", file=sys.stderr)
        return 2

    from __graft_entry__ import load_package

    load_package()
    from qwen3_iree_amd import q8gemv as Q
    from qwen3_iree_amd import weights as Wt

    Q.init()
    info = Q.device_info()
    log(f"device {info['name']}, {info['compute_units']} CUs")

    # ---------------------------------------------------------------- inputs
    t0 = time.time()
    kinds = Q.Q8_KINDS  # sweep order per layer: q, kv, o, gate_up, dn
    layers = Q.NUM_LAYERS
    stacks = {}
    for d in kinds:
        host = Wt.synthetic_q8_stack(d.n, d.k, layers, seed=SEED, tensor=d.kind, workers=16)
        stacks[d.kind] = (host, Q.DeviceBuffer.from_array(host))
    xs, ys = {}, {}
    for layer in range(layers):
        for d in kinds:
            x = Wt.synthetic_x(d.k, SEED, index=layer * 8 + d.kind)
            xs[(layer, d.kind)] = (x, Q.DeviceBuffer.from_array(x))
            ys[(layer, d.kind)] = Q.DeviceBuffer(2 * d.n)
    sweep_bytes = sum(algorithmic_bytes(d) for d in kinds) * layers
    weight_bytes = sum(d.bytes_per_layer for d in kinds) * layers
    log(f"sweep inputs ready in {time.time() - t0:.1f}s: {weight_bytes} weight bytes, "
        f"{sweep_bytes} algorithmic bytes per step")

    stream = Q.Stream()

    def record_sweep():
        for layer in range(layers):
            for d in kinds:
                Q.q8gemv(d.kind, stacks[d.kind][1], layer, xs[(layer, d.kind)][1],
                         ys[(layer, d.kind)], stream)

    # correctness spot check of the timed configuration (layer 27 gate_up)
    record_sweep()
    stream.synchronize()

    graph = Q.Graph(stream, record_sweep)
    for _ in range(args.warmup):
        graph.launch(stream)
    stream.synchronize()

    ev0, ev1 = Q.Event(), Q.Event()
    Q.synchronize()
    t_wall = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        graph.launch(stream)
    ev1.record(stream)
    ev1.synchronize()
    Q.synchronize()
    wall_s = time.perf_counter() - t_wall
    ms_total = ev0.elapsed_ms(ev1)
    ms_per_step = ms_total / args.steps
    value = sweep_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"sweep: {ms_per_step * 1e3:.1f} us/step, {value:.1f} GB/s "
        f"({100 * value / HBM_PEAK_GBS:.1f}% of peak); host wall {wall_s:.3f}s")

    # ------------------------------------------------- per-kernel durations
    per_kind = {d.kind: [] for d in kinds}
    starts = [Q.Event() for _ in range(layers * len(kinds))]
    stops = [Q.Event() for _ in range(layers * len(kinds))]
    for rep in range(args.kernel_reps):
        i = 0
        for layer in range(layers):
            for d in kinds:
                Q.time_next_launch(starts[i], stops[i])
                Q.q8gemv(d.kind, stacks[d.kind][1], layer, xs[(layer, d.kind)][1],
                         ys[(layer, d.kind)], stream)
                i += 1
        stream.synchronize()
        i = 0
        for layer in range(layers):
            for d in kinds:
                per_kind[d.kind].append(starts[i].elapsed_ms(stops[i]) * 1e3)
                i += 1
    kern = {}
    for d in kinds:
        us = float(np.mean(per_kind[d.kind]))
        gbs = algorithmic_bytes(d) / (us * 1e-6) / 1e9
        kern[d.name] = {"avg_us": round(us, 3), "median_us": round(float(np.median(per_kind[d.kind])), 3),
                        "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                        "bytes": algorithmic_bytes(d), "launches": len(per_kind[d.kind])}
    sum_kernel_us = sum(kern[d.name]["avg_us"] for d in kinds) * layers
    dominant = max(kinds, key=lambda d: kern[d.name]["avg_us"])
    dk = kern[dominant.name]
    log("kernels: " + ", ".join(f"{n} {v['avg_us']:.2f}us {v['GBps']:.0f}GB/s" for n, v in kern.items()))

    # ------------------------------------------------------------- vocab
    t0 = time.time()
    Wv = Wt.synthetic_f16_matrix(Q.VOCAB_ROWS, Q.HIDDEN, seed=SEED, tensor=24, workers=16)
    xv = Wt.synthetic_x(Q.HIDDEN, SEED, index=9999)
    wv_dev = Q.DeviceBuffer.from_array(Wv)
    xv_dev = Q.DeviceBuffer.from_array(xv)
    logits_dev = Q.DeviceBuffer(2 * Q.VOCAB_ROWS)
    tok_dev = Q.DeviceBuffer(16)
    ws = Q.DeviceBuffer(Q.vocab_workspace_bytes())
    Q.vocab_workspace_reset(ws, stream)
    log(f"vocab inputs ready in {time.time() - t0:.1f}s")
    vocab_bytes = Q.VOCAB.bytes_per_layer + 2 * Q.HIDDEN + 2 * Q.VOCAB_ROWS + 4
    for _ in range(5):
        Q.vocab_gemv_argmax(wv_dev, xv_dev, logits_dev, tok_dev, ws, stream)
    stream.synchronize()
    vs, ve = Q.Event(), Q.Event()
    vocab_us = []
    for _ in range(20):
        Q.time_next_launch(vs, ve)
        Q.vocab_gemv_argmax(wv_dev, xv_dev, logits_dev, tok_dev, ws, stream)
        ve.synchronize()
        vocab_us.append(vs.elapsed_ms(ve) * 1e3)
    v_us = float(np.mean(vocab_us))
    v_gbs = vocab_bytes / (v_us * 1e-6) / 1e9
    token = int(tok_dev.download(np.int32, 1)[0])
    logits = logits_dev.download(np.float16, Q.VOCAB_ROWS)
    log(f"vocab: {v_us:.2f} us, {v_gbs:.0f} GB/s, token {token}")

    # ---------------------------------------- GEMV share of a decode step
    # 28 x (q, k, v, o, gate_up, down) + vocab, each dispatch ordered after
    # the previous one on one stream, replayed from a graph.
    step_y = [Q.DeviceBuffer(2 * 6144) for _ in range(6)]

    def record_decode_gemvs():
        for layer in range(layers):
            for j, d in enumerate(Q.LAYER_ORDER):
                Q.q8gemv(d.kind, stacks[d.kind][1], layer, xs[(layer, d.kind)][1], step_y[j], stream)
        Q.vocab_gemv_argmax(wv_dev, xv_dev, logits_dev, tok_dev, ws, stream)

    dgraph = Q.Graph(stream, record_decode_gemvs)
    for _ in range(5):
        dgraph.launch(stream)
    stream.synchronize()
    ev0.record(stream)
    reps = 50
    for _ in range(reps):
        dgraph.launch(stream)
    ev1.record(stream)
    ev1.synchronize()
    decode_gemv_us = ev0.elapsed_ms(ev1) * 1e3 / reps
    log(f"decode-step GEMVs (168 Q8 + vocab): {decode_gemv_us:.1f} us")

    # ---------------------------------------------------- parity spot check
    sys.path.insert(0, str(REPO / "oracle"))
    import oracle as O  # the checker; also the CPU baseline below

    d = Q.GATE_UP
    y_gpu = ys[(layers - 1, d.kind)].download(np.float16)
    raw = stacks[d.kind][0][layers - 1]
    x27 = xs[(layers - 1, d.kind)][0]
    ref = O.q8_gemv(raw, d.n, d.k, x27)
    _, mag = O.q8_gemv_f64(raw, d.n, d.k, x27)
    rep_q8 = O.gemv_tolerance_report(y_gpu, ref, mag)
    ref_v = O.f16_gemv(Wv, xv)
    _, mag_v = O.f16_gemv_f64(Wv, xv)
    rep_v = O.gemv_tolerance_report(logits, ref_v, mag_v)
    parity_ok = rep_q8["fail"] == 0 and rep_v["fail"] == 0 and token == O.argmax_tiled(logits)
    log(f"parity: gate_up L27 {rep_q8['fail']} fails, vocab {rep_v['fail']} fails, "
        f"token {token} vs argmax(own logits) {O.argmax_tiled(logits)}")

    # ------------------------------------------------------ CPU baseline
    cpu = None
    if not args.no_cpu:
        threads = O.num_threads()
        host = {d.kind: stacks[d.kind][0] for d in kinds}
        hx = {key: v[0] for key, v in xs.items()}
        sweeps = 0
        t0 = time.perf_counter()
        while True:
            for layer in range(layers):
                for d in kinds:
                    O.q8_gemv(host[d.kind][layer], d.n, d.k, hx[(layer, d.kind)])
            sweeps += 1
            if time.perf_counter() - t0 >= args.cpu_seconds:
                break
        cpu_s = time.perf_counter() - t0
        cpu_gbs = sweep_bytes * sweeps / cpu_s / 1e9
        cpu = {"value": round(cpu_gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"{sweeps} full 28-layer sweeps (140 Q8_0 GEMVs each, same inputs) with the "
                         f"C oracle in the reference kernels' f32 order, OpenMP {threads} threads, "
                         f"{cpu_s:.1f}s", "ms_per_step": round(1e3 * cpu_s / sweeps, 3)}
        log(f"cpu oracle: {cpu_gbs:.2f} GB/s over {sweeps} sweeps ({threads} threads)")

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 x f16 -> f32",
        "data": "synthetic (seeded N(0,0.02) weights quantized to Q8_0, N(0,1) f16 x)",
        "config": {
            "workload": "28-layer stacked cold-cache Q8_0 GEMV sweep (attn_q, attn_kv, attn_o, "
                        "gate_up, ffn_dn per layer; 140 dispatches; hipGraph replay)",
            "layers": layers,
            "dispatches_per_step": layers * len(kinds),
            "weight_bytes": weight_bytes,
            "algorithmic_bytes_per_step": sweep_bytes,
            "device": info["name"],
        },
        "pct_of_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "us_per_step": round(ms_per_step * 1e3, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": f"q8gemv {dominant.name} [{dominant.n},{dominant.k}]",
            "achieved": dk["GBps"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": dk["frac"],
            "avg_us": dk["avg_us"],
            "bytes_per_launch": dk["bytes"],
            "traffic": None,
        },
        "kernels": kern,
        "sum_kernel_us_per_step": round(sum_kernel_us, 2),
        "vocab": {"avg_us": round(v_us, 3), "GBps": round(v_gbs, 1),
                  "frac": round(v_gbs / HBM_PEAK_GBS, 4), "bytes": vocab_bytes, "token": token},
        "decode_step_gemv_us": round(decode_gemv_us, 2),
        "parity_ok": bool(parity_ok),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
