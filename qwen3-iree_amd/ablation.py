#!/usr/bin/env python3
"""What each design choice of the Q8_0 GEMV and the vocab GEMV + argmax is
worth, measured on the two headline workloads.

Each variant is a build of csrc/q8gemv_kernels.hip that replaces one choice
with a plain alternative computing the same outputs (the switches are
documented beside their defaults in csrc/q8_device.h); "product" is the
shipped build.  A variant run times, with HIP events on the launch stream:
  * the 28-layer stacked sweep (140 Q8_0 GEMVs, 437,821,440 algorithmic
    bytes) as one batched launch, three identical weight copies taken in turn
    (no launch finds its bytes in the 256 MB MALL);
  * the 151936 x 1024 f16 vocab GEMV + argmax, three matrix copies in turn;
and the product run adds the launch-shape sweeps (workgroups of the batched
launch and of the vocab kernel per compute unit) and the vocab GEMV with the
argmax as a separate pass (the HAL dispatch 24, logits only, then f16_argmax)
instead of fused.  Outputs (every sweep output, the logits, the token) are
saved so --compare can hold each variant to the product build.

    python3 qwen3-iree_amd/ablation.py --build              # lib/ablation/<variant>/
    python3 qwen3-iree_amd/ablation.py --run product --save DIR
    python3 qwen3-iree_amd/ablation.py --run load64 --save DIR
    python3 qwen3-iree_amd/ablation.py --compare DIR

Under rocprofv3 each --run is one traced process: the kernel rows of its
summary (rocprof_summary.py, by kernel and grid) give every variant's and
every launch shape's duration, hence its achieved GB/s.
"""
from __future__ import annotations

import argparse
import json
import shutil
import sys
import time
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
ABL = PKG / "lib" / "ablation"
SEED = 20261201
HBM_PEAK_GBS = 8000.0

# variant -> (hipcc defines, what it replaces)
VARIANTS = {
    "product": ([], "the shipped build"),
    "load64": (["-DQ8_LOAD_BYTES=8"],
               "each lane's 16 weight bytes read as two 64-bit loads, not one 128-bit load"),
    "load32": (["-DQ8_LOAD_BYTES=4"],
               "each lane's 16 weight bytes read as four 32-bit loads"),
    "x_global": (["-DQ8_X_LDS=0"],
                 "x read by every wave from global memory for each unit, not staged once per "
                 "workgroup in LDS"),
    "dequant_scalar": (["-DQ8_DEQUANT_PACKED=0"],
                       "each int8 converted to f32 and multiplied by f32(x), not int8 pairs made "
                       "f16 pairs in registers and multiplied by v_dot2"),
    "reduce_bpermute": (["-DQ8_REDUCE_DPP=0"],
                        "16-lane row sums through ds_bpermute shuffles, not DPP"),
}


def build_all() -> None:
    sys.path.insert(0, str(PKG))
    import build as B

    for name, (defines, _) in VARIANTS.items():
        d = ABL / name
        d.mkdir(parents=True, exist_ok=True)
        B._run([str(B.ROCM / "bin" / "hipcc"), *B.HIPCC_FLAGS, *defines, f"-I{B.CSRC}",
                str(B.CSRC / "q8gemv_kernels.hip"), "-o", str(d / "q8gemv_gfx950.hsaco")])
        for other in ("decode_gfx950.hsaco", "prefill_gfx950.hsaco"):
            shutil.copy(B.LIB / other, d / other)
        print(f"built {name}: {d / 'q8gemv_gfx950.hsaco'}", flush=True)


def timed_us(Q, stream, fn, launches: int) -> float:
    """Untimed launches for 200 ms, then `launches` between two events."""
    t_end = time.perf_counter() + 0.2
    while time.perf_counter() < t_end:
        fn()
        stream.synchronize()
    e0, e1 = Q.Event(), Q.Event()
    e0.record(stream)
    for _ in range(launches):
        fn()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_ms(e1) * 1e3 / launches


def run(name: str, save: Path | None, launches: int, copy_mib: int = 0) -> dict:
    sys.path.insert(0, str(REPO))
    from __graft_entry__ import load_package

    load_package()
    from qwen3_iree_amd import q8gemv as Q
    from qwen3_iree_amd import sweep as SW
    from qwen3_iree_amd import weights as Wt

    co = ABL / name / "q8gemv_gfx950.hsaco"
    if not co.exists():
        raise SystemExit(f"{co} is missing: run --build first")
    Q.init(str(co))
    stream = Q.Stream()
    out = {"variant": name, "replaces": VARIANTS[name][1], "launches": launches}
    if copy_mib:
        # a copy of known size in the same process: what rocprofv3's traffic
        # counters read for it scales theirs (rocprof_summary.py --copy-bytes)
        nbytes = copy_mib << 20
        src, dst = Q.DeviceBuffer(nbytes), Q.DeviceBuffer(nbytes)
        for _ in range(5):
            Q.stream_copy(dst, src, nbytes, stream)
        stream.synchronize()
        src.free()
        dst.free()

    sw = SW.build(SEED, 16, copies=3)
    batches = [sw.batch(c) for c in range(sw.n_copies)]
    turn = [0]

    def sweep_fn():
        batches[turn[0] % len(batches)].launch(stream)
        turn[0] += 1

    us = timed_us(Q, stream, sweep_fn, launches)
    out["sweep_us"] = round(us, 2)
    out["sweep_GBps"] = round(sw.bytes_per_step / us / 1e3, 1)
    out["sweep_frac"] = round(sw.bytes_per_step / us / 1e3 / HBM_PEAK_GBS, 4)
    batches[0].launch(stream)
    stream.synchronize()
    ys = np.concatenate([sw.dev_y[(layer, d.kind)].download(np.uint16) for layer, d in sw.order])

    n, k = Q.VOCAB_ROWS, Q.HIDDEN
    Wv = Wt.synthetic_f16_matrix(n, k, seed=SEED, tensor=24, workers=16)
    xv = Wt.synthetic_x(k, SEED, index=9999)
    wv = [Q.DeviceBuffer.from_array(Wv) for _ in range(3)]
    xd = Q.DeviceBuffer.from_array(xv)
    logits = Q.DeviceBuffer(2 * n)
    tok = Q.DeviceBuffer(16)
    ws = Q.DeviceBuffer(Q.vocab_workspace_bytes())
    Q.vocab_workspace_reset(ws, stream)
    vturn = [0]

    def vocab_fn():
        Q.vocab_gemv_argmax(wv[vturn[0] % 3], xd, logits, tok, ws, stream)
        vturn[0] += 1

    us = timed_us(Q, stream, vocab_fn, launches)
    vbytes = Q.VOCAB.bytes_per_layer + 2 * k + 2 * n + 4
    out["vocab_us"] = round(us, 2)
    out["vocab_GBps"] = round(vbytes / us / 1e3, 1)
    out["vocab_frac"] = round(vbytes / us / 1e3 / HBM_PEAK_GBS, 4)
    Q.vocab_gemv_argmax(wv[0], xd, logits, tok, ws, stream)
    stream.synchronize()
    lg = logits.download(np.uint16)
    token = int(tok.download(np.int32, 1)[0])
    out["token"] = token

    if name == "product":
        cus = Q.device_info()["compute_units"]
        grid = {}
        for per_cu in (1, 2, 4, 6, 8, 10, 12, 16):
            Q.set_batch_workgroups(per_cu * cus)
            grid[per_cu] = round(timed_us(Q, stream, sweep_fn, launches), 2)
        Q.set_batch_workgroups(0)
        out["sweep_us_by_waves_per_cu"] = grid
        vgrid = {}
        for per_cu in (1, 2, 4, 8):
            Q.set_vocab_workgroups(per_cu * cus)
            vgrid[per_cu] = round(timed_us(Q, stream, vocab_fn, launches), 2)
        Q.set_vocab_workgroups(0)
        out["vocab_us_by_workgroups_per_cu"] = vgrid
        # the argmax as its own pass: logits only (HAL dispatch 24 at the vocab
        # kernel's grid), then f16_argmax over them
        b1 = np.zeros(64 + 2 * k, np.uint8)
        b1[64:] = xv.view(np.uint8)
        bind1 = Q.DeviceBuffer.from_array(b1)
        bind2 = Q.DeviceBuffer(2 * n + 64)
        tok2 = Q.DeviceBuffer(16)
        uturn = [0]

        def unfused_fn():
            Q.hal_dispatch(24, wv[uturn[0] % 3], bind1, bind2, [0], stream, cus, 256)
            Q.f16_argmax(bind2, n, tok2, ws, stream)
            uturn[0] += 1

        out["vocab_unfused_us"] = round(timed_us(Q, stream, unfused_fn, launches), 2)
        unfused_fn()
        stream.synchronize()
        out["vocab_unfused_same"] = bool(
            np.array_equal(bind2.download(np.uint16, n), lg)
            and int(tok2.download(np.int32, 1)[0]) == token)
        for b in (bind1, bind2, tok2):
            b.free()

    if save is not None:
        save.mkdir(parents=True, exist_ok=True)
        np.savez(save / f"{name}.npz", sweep_y=ys, logits=lg, token=np.int32(token))
    for b in (*wv, xd, logits, tok, ws):
        b.free()
    for b in batches:
        b.free()
    sw.free()
    return out


def compare(save: Path) -> list:
    ref = np.load(save / "product.npz")
    rows = []
    for name in VARIANTS:
        f = save / f"{name}.npz"
        if name == "product" or not f.exists():
            continue
        v = np.load(f)
        row = {"variant": name}
        for key in ("sweep_y", "logits"):
            a = ref[key].view(np.float16).astype(np.float64)
            b = v[key].view(np.float16).astype(np.float64)
            same = np.array_equal(ref[key], v[key])
            # distance in f16 units of the last place of the product's value
            ulp = np.spacing(np.abs(ref[key].view(np.float16))).astype(np.float64)
            d = np.abs(a - b) / ulp
            row[key] = "bit-identical" if same else f"max {np.nanmax(d):.0f} ulp, {int((d > 0).sum())} differ"
        row["token"] = "same" if int(v["token"]) == int(ref["token"]) else "differs"
        rows.append(row)
    return rows


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--build", action="store_true", help="build every variant's code object")
    ap.add_argument("--run", choices=list(VARIANTS), help="time one variant")
    ap.add_argument("--save", type=Path, default=None, help="directory for the outputs")
    ap.add_argument("--launches", type=int, default=300)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also copy MIB MiB (traffic-counter scale)")
    ap.add_argument("--compare", type=Path, default=None,
                    help="hold every saved variant's outputs to the product's")
    args = ap.parse_args()
    if args.build:
        build_all()
    if args.run:
        print(json.dumps(run(args.run, args.save, args.launches, args.copy_calibration)),
              flush=True)
    if args.compare:
        for row in compare(args.compare):
            print(json.dumps(row), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
