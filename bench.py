#!/usr/bin/env python3
"""Benchmark of the decode GEMV hot path on one MI355X.

Workload (the headline metric's configuration): the 28-layer stacked
cold-cache Q8_0 GEMV sweep -- five stacked weight sets (attn_q, attn_kv, attn_o,
gate_up, ffn_dn; 436,731,904 bytes, more than the 256 MB MALL); for layer
0..27 the five GEMVs in that order, 140 GEMVs per step, each with its own f16 x
and y (qwen3_iree_amd/sweep.py, shared with the parity tests).  Inputs are
resident in HBM before timing.

One step = one sweep executed as a single batched launch (q8gemv_batch: the
140 GEMVs listed in sweep order; waves stream the list in order, so the access
pattern still rotates through the 28 layers).  Measured in the same run:
  * the same sweep as 140 stream-ordered dispatches of the per-GEMV entry
    point (the reference's dispatch granularity), replayed from a hipGraph;
  * the f16 vocab GEMV + fused argmax [151936, 1024];
  * the GEMV share of a decode step: 28 x (one fused q/k/v launch, o,
    gate_up, down) + vocab, stream-ordered, replayed from a hipGraph;
  * the full decode step (qwen3_decode_step: embedding, 28 layers with
    attention over a 1024-position KV cache, final norm, vocab, argmax) on
    random-init Qwen3-0.6B weights, as one launch per step (dec_step) and as
    a hipGraph of 143 per-phase launches, the token fed back on the device,
    checked against the oracle's step;
  * batched prompt ingestion (qwen3_prefill_batched) of 512 tokens, checked
    against the decode-step prompt path;
  * end-to-end generation, the reference's own published measure
    (scripts/benchmark.py:52-81: wall time of one `run` call = prompt
    ingestion + up to 128 greedy tokens with the EOS check after every 4,
    tok/s = tokens generated before EOS / that time), for a chat-sized prompt
    and a 512-token prompt, checked token for token against single steps;
  * parity of all 140 sweep outputs and of the vocab logits/token against the
    CPU oracle;
  * the CPU oracle on a bounded sample of the same sweep (cpu_baseline), at
    every host thread and at one.

Timing: every timed kernel is first run for at least 200 ms (whatever
--warmup says; the GPU clock ramps over the first ~100 ms of sustained work),
then exactly --steps calls are timed with HIP events on the launch stream in
10 blocks: `ms_per_step` / `value` come from the mean over all steps, and the
median over the blocks is reported beside it.

Prints one JSON line.  Only --gpus 1 is supported: this path runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
METRIC = "achieved HBM GB/s (% of peak) on 28-layer Q8_0 GEMV sweep; µs per decode step"
SEED = 20261201
MIN_WARM_MS = 200.0
TIMING_BLOCKS = 10
EOS_TOKEN = 151645   # scripts/benchmark.py:21
MAX_NEW_TOKENS = 128  # scripts/benchmark.py:22
IM_START = 151644     # <|im_start|>; <|im_end|> is EOS_TOKEN
# Lengths of the ten chat prompts of scripts/benchmark.py:8-19 under its template
# `<|im_start|>user\n{text}<|im_end|>\n<|im_start|>assistant\n` (:53): 8 template
# tokens + the text's.  No tokenizer files exist here, so the text counts are
# estimates (one token per word, digit and punctuation mark), and the token ids
# are synthetic.
REFERENCE_PROMPT_TOKENS = (9, 15, 10, 15, 15, 15, 16, 18, 20, 22)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def profiled_traffic(name: str, grid_threads: int) -> dict:
    """HBM bytes per dispatch of kernel `name` at this grid from the committed
    rocprofv3 counter summary (FETCH_SIZE + WRITE_SIZE, each scaled by what it
    reads for a copy kernel of known size), with whether the summary was taken
    on the machine code of that kernel in this tree (per-kernel digest of the
    built code object: edits to other kernels leave it valid)."""
    from qwen3_iree_amd import build as B

    out = {"bytes": None, "code_digest": None, "stale": None}
    path = REPO / "profiles" / "traffic.json"
    if not path.exists():
        return out
    rep = json.loads(path.read_text())
    for k in rep.get("kernels", []):
        if k.get("name") == name and k.get("grid") == grid_threads and k.get("hbm_bytes"):
            out["bytes"] = int(k["hbm_bytes"])
            out["profiled_mean_us"] = round(float(k["mean_us"]), 3)
            out["code_digest"] = k.get("code_digest")
            out["stale"] = k.get("code_digest") != B.kernel_digest(name)
    return out


def warm(stream, fn, n: int, min_ms: float = MIN_WARM_MS) -> int:
    """At least n calls of fn() and at least min_ms of them (host clock)."""
    calls = 0
    t0 = time.perf_counter()
    while calls < n or (time.perf_counter() - t0) * 1e3 < min_ms:
        for _ in range(8):
            fn()
        calls += 8
        stream.synchronize()
    return calls


def timed(Q, stream, fn, reps: int, blocks: int = TIMING_BLOCKS) -> dict:
    """Exactly `reps` back-to-back calls of fn() on `stream`, HIP events on
    that stream between `blocks` blocks of calls.  Mean ms per call over all
    of them, and the median (min, max) of the blocks' means."""
    reps = max(1, int(reps))
    blocks = max(1, min(blocks, reps))
    sizes = [reps // blocks + (1 if i < reps % blocks else 0) for i in range(blocks)]
    ev = [Q.Event() for _ in range(blocks + 1)]
    stream.synchronize()
    ev[0].record(stream)
    for i, n in enumerate(sizes):
        for _ in range(n):
            fn()
        ev[i + 1].record(stream)
    ev[-1].synchronize()
    per = [ev[i].elapsed_ms(ev[i + 1]) / sizes[i] for i in range(blocks)]
    total = ev[0].elapsed_ms(ev[-1])
    for e in ev:
        e.destroy()
    return {"mean_ms": total / reps, "median_ms": statistics.median(per), "min_ms": min(per),
            "max_ms": max(per), "reps": reps, "blocks": blocks}


SCRUB_BYTES = 1 << 30  # per scrub: 1 GiB read, 4x the 256 MB MALL


def bound_launch_us(Q, stream, fn, n: int, scrub=None) -> list[float]:
    """Per-launch times of the kernel fn() launches (HIP events bound to that
    launch, q8rt_time_next_launch), n launches with the stream drained between
    them; with scrub = (src, dst, bytes), each launch follows a copy of that
    many bytes (read only, so no dirty line is left for the kernel to write
    back), which leaves nothing of the kernel's inputs in the MALL."""
    e0, e1 = Q.Event(), Q.Event()
    out = []
    for _ in range(n):
        if scrub is not None:
            Q.stream_read(scrub[0], scrub[1], stream)
        Q.time_next_launch(e0, e1)
        fn()
        e1.synchronize()
        out.append(e0.elapsed_ms(e1) * 1e3)
    e0.destroy()
    e1.destroy()
    return out


def scrub_ab(Q, stream, fn, scrub, n: int = 30) -> dict:
    """The kernel launched by fn() timed alone, A: right after its previous
    launch (the access pattern the benchmark times), B: after a scrub copy,
    both with the same per-launch events.  B / A > 1 would mean part of A's
    bytes came from the memory-side cache (MALL) rather than HBM."""
    warm(stream, fn, 3)
    a = bound_launch_us(Q, stream, fn, n)
    b = bound_launch_us(Q, stream, fn, n, scrub)
    ma, mb = statistics.median(a), statistics.median(b)
    return {"unscrubbed_us": round(ma, 2), "scrubbed_us": round(mb, 2),
            "ratio": round(mb / ma, 4), "launches": n, "scrub_bytes": scrub[1],
            "method": "median of per-launch HIP events bound to the kernel (hipExtModuleLaunchKernel); "
                      f"B launches each follow a read of {scrub[1] >> 20} MiB (4x the 256 MB MALL, "
                      "no writes)"}


def calibration(Q) -> dict:
    """The two measurements the single-launch step's design rests on: what a
    launch of its grid costs (ordinary vs cooperative, empty kernel of the same
    shape and LDS), and what a tagged-word hand-off costs (one producer to one
    consumer, and 128 producers to 192 consumers with 4 replicas: the attn_o
    output feeding the gate/up workgroups)."""
    out = {"launch_cost_us": {}, "handoff_us": {}}
    for coop in (False, True):
        out["launch_cost_us"]["cooperative" if coop else "ordinary"] = round(
            Q.launch_cost(448, 256, 79360, 2000, cooperative=coop), 2)
    for name, (p, c, n, rep) in {"one_to_one_512_words": (1, 1, 512, 1),
                                 "128_to_192_512_words_4_replicas": (128, 192, 512, 4)}.items():
        lat, failed = Q.handoff_latency(p, c, n, rep, rounds=100)
        ok = lat[np.isfinite(lat)]
        out["handoff_us"][name] = {
            "median": round(float(np.median(ok)), 3) if ok.size else None,
            "p10": round(float(np.percentile(ok, 10)), 3) if ok.size else None,
            "p90": round(float(np.percentile(ok, 90)), 3) if ok.size else None,
            "max": round(float(ok.max()), 3) if ok.size else None,
            "samples": int(ok.size), "failed": failed,
            "first_consumer_median": round(float(np.median(np.where(np.isfinite(lat), lat, np.inf)
                                                          .min(axis=1))), 3) if ok.size else None}
    log(f"calibration: launch of the 448 x 256 grid {out['launch_cost_us']['ordinary']} us "
        f"(cooperative {out['launch_cost_us']['cooperative']} us); hand-off 1 -> 1 median "
        f"{out['handoff_us']['one_to_one_512_words']['median']} us, 128 -> 192 median "
        f"{out['handoff_us']['128_to_192_512_words_4_replicas']['median']} us")
    return out


def bench_decode(Q, O, stream, args) -> dict:
    """The full decode step at context args.context: one step checked against
    the oracle's, then steps timed with HIP events (token fed back, position
    kept)."""
    from qwen3_iree_amd import decode as D
    from qwen3_iree_amd import sweep as S

    layers = D.LAYERS
    vocab_bytes = Q.VOCAB.bytes_per_layer + 2 * Q.HIDDEN + 2 * Q.VOCAB_ROWS + 4
    t0 = time.time()
    mhost = D.synthetic_weights(seed=SEED, workers=16)
    model = D.DeviceWeights(mhost)
    ctx = args.context
    max_seq = ctx
    sess = D.DecodeSession(model, max_seq, stream)
    rng = np.random.default_rng(SEED + 5)
    kc = rng.standard_normal((D.LAYERS * max_seq, D.KV_DIM), dtype=np.float32).astype(np.float16)
    vc = (np.float32(0.6) * rng.standard_normal((D.LAYERS * max_seq, D.KV_DIM),
                                                dtype=np.float32)).astype(np.float16)
    sess.k_cache.upload(kc)
    sess.v_cache.upload(vc)
    first_token = 1234
    sess.set_state(first_token, ctx - 1)
    log(f"decode model ready in {time.time() - t0:.1f}s ({model.nbytes} parameter bytes), "
        f"context {ctx}")
    # one checked step: attention over slots 0..ctx-1, position kept (advance = 0)
    sess.step(advance=False, logits=True)
    step_tok, step_pos = sess.get_state()
    step_logits = sess.read_logits()
    # the same step by the CPU oracle (OpenMP over the GEMV rows), timed
    t_cpu = time.perf_counter()
    ref_tok, ref_logits, _ = O.decode_step(mhost, kc, vc, max_seq, first_token, ctx - 1, True)
    cpu_step_us = (time.perf_counter() - t_cpu) * 1e6
    dl = np.abs(step_logits.astype(np.float64) - ref_logits.astype(np.float64))
    srt = np.sort(ref_logits.astype(np.float64))
    margin = float(srt[-1] - srt[-2])
    step_ok = (step_tok == O.argmax_tiled(step_logits) and step_pos == ctx - 1
               and (step_tok == ref_tok or margin <= 2 * dl.max()))
    log(f"decode step parity: token {step_tok} (oracle {ref_tok}, margin {margin:.4f}, "
        f"max |dlogit| {dl.max():.4f})")
    reps = max(50, args.steps // 4)
    # the per-phase step (143 launches) replayed from a hipGraph
    default_mode = D.step_mode()
    D.set_step_mode(0)
    sess.set_state(first_token, ctx - 1)
    if args.no_graph:
        dec_fn = lambda: sess.step(advance=False, logits=False)  # noqa: E731
    else:
        sess.capture(advance=False, logits=False)
        dec_fn = lambda: sess.replay(advance=False, logits=False)  # noqa: E731
    warm(stream, dec_fn, 20)
    tp = timed(Q, stream, dec_fn, reps)
    dec_us = tp["mean_ms"] * 1e3
    norm_bytes = 2 * (D.LAYERS * (2 * D.HIDDEN + 2 * D.HEAD_DIM) + D.HIDDEN)
    kv_bytes = D.LAYERS * ctx * 2 * D.KV_DIM * 2
    dec_bytes = (sum(S.algorithmic_bytes(d) for d in Q.LAYER_ORDER) * layers + vocab_bytes
                 + kv_bytes + norm_bytes + 2 * D.HIDDEN)
    log(f"decode step (context {ctx}, {3 + 5 * layers} launches"
        f"{'' if args.no_graph else ', hipGraph'}): {dec_us:.1f} us/token (median "
        f"{tp['median_ms'] * 1e3:.1f}), {1e6 / dec_us:.0f} tok/s")
    # the same step as one launch (qwen3_set_step_mode(1)), eager
    ts = None
    if args.per_phase_only:
        log("single-launch step: not measured (--per-phase-only)")
    else:
        try:
            D.set_step_mode(1)
        except Q.Q8GemvError as e:
            log(f"single-launch step unavailable: {e}")
        else:
            sess.set_state(first_token, ctx - 1)
            one = lambda: sess.step(advance=False, logits=False)  # noqa: E731
            warm(stream, one, 20)
            ts = timed(Q, stream, one, reps)
            ok1 = sess.get_state()[1] == ctx - 1 and sess.check_status() == 0
            log(f"decode step as one launch: {ts['mean_ms'] * 1e3:.1f} us/token "
                f"(median {ts['median_ms'] * 1e3:.1f}; status ok={ok1})")
    D.set_step_mode(default_mode)
    sess.free()
    model.free()
    cal = None if args.no_calibration else calibration(Q)
    best = ts if ts is not None else tp
    best_us = best["mean_ms"] * 1e3
    best_gbs = dec_bytes / best_us / 1e3
    return {"us": round(best_us, 2), "median_us": round(best["median_ms"] * 1e3, 2),
            "tok_per_s": round(1e6 / best_us, 1), "context": ctx,
            "bytes": dec_bytes, "GBps": round(best_gbs, 1), "frac": round(best_gbs / HBM_PEAK_GBS, 4),
            "launch": "one launch per step (dec_step)" if ts is not None else
                      ("hipGraph of 143 launches" if not args.no_graph else "143 eager launches"),
            "single_launch_us": None if ts is None else round(ts["mean_ms"] * 1e3, 2),
            "per_phase_us": round(dec_us, 2), "per_phase_median_us": round(tp["median_ms"] * 1e3, 2),
            "per_phase_launches": 3 + 5 * layers,
            "per_phase_launch": "eager" if args.no_graph else "hipGraph", "steps_timed": reps,
            "token": step_tok, "oracle_token": ref_tok, "parity_ok": bool(step_ok),
            "calibration": cal,
            "cpu_oracle": {"us": round(cpu_step_us, 1), "threads": O.num_threads(),
                           "kind": "port",
                           "sample": "one step of the C oracle at the same context and inputs "
                                     "(the parity check's step)"}}


def copy_calibration(Q, stream, mib: int) -> dict | None:
    """Five launches of the plain copy kernel (stream_copy_b128) over mib MiB: the
    known-size reference that rocprof_summary.py scales FETCH_SIZE / WRITE_SIZE by."""
    if mib <= 0:
        return None
    nbytes = mib << 20
    src, dst = Q.DeviceBuffer(nbytes), Q.DeviceBuffer(nbytes)
    tc = timed(Q, stream, lambda: Q.stream_copy(dst, src, nbytes, stream), 5, 1)
    copy_ms = tc["mean_ms"]
    log(f"copy calibration: {nbytes} B read + written in {copy_ms * 1e3:.1f} us")
    src.free()
    dst.free()
    return {"bytes_read": nbytes, "bytes_written": nbytes, "us": round(copy_ms * 1e3, 2),
            "GBps_read_plus_write": round(2 * nbytes / (copy_ms * 1e-3) / 1e9, 1)}


def prefill_flops(n: int) -> tuple[int, int]:
    """(GEMM flops, attention flops) of a prompt of n tokens from position 0."""
    per_token = 2 * (2048 * 1024 + 2 * 1024 * 1024 + 1024 * 2048 + 6144 * 1024 + 1024 * 3072)
    gemm = 28 * n * per_token
    attn = 28 * 16 * 128 * 4 * (n * (n + 1) // 2)  # q.k and p.v over positions 0..i
    return gemm, attn


def bench_prefill(Q, stream, args) -> dict:
    """Batched prompt ingestion (qwen3_prefill_batched) of args.prefill_tokens
    tokens from position 0, checked against the decode-step prompt path, then
    timed as whole calls (host wall clock, the call's own position read
    included)."""
    from qwen3_iree_amd import decode as D

    n = args.prefill_tokens
    mhost = D.synthetic_weights(seed=SEED, workers=16)
    model = D.DeviceWeights(mhost)
    sess = D.DecodeSession(model, n, stream)
    rng = np.random.default_rng(SEED + 9)
    prompt = rng.integers(0, D.VOCAB, n).astype(np.int32)
    pbuf = Q.DeviceBuffer.from_array(prompt)
    lib = Q.load_library()
    nbytes = int(lib.qwen3_prefill_workspace_bytes(n))
    ws = Q.DeviceBuffer(nbytes)

    def one(logits=None):
        # the previous call's kernels write the position on `stream`; the call
        # itself waits for the stream anyway (it reads the position first)
        stream.synchronize()
        sess.set_state(0, 0)
        Q._call("qwen3_prefill_batched", model.ref(), sess.k_cache.ptr, sess.v_cache.ptr, n,
                pbuf.ptr, n, sess.token_ptr, sess.pos_ptr, logits, 0, ws.ptr, nbytes,
                sess.scratch.ptr, Q._stream(stream))

    if args.kernels_only:
        # counter runs: three calls over the f16 matrices, then three over the
        # Q8_0 stacks (their GEMM kernels have different names), nothing else
        for f16 in (True, False):
            model.use_prefill_matrices(f16)
            for _ in range(3):
                one()
            stream.synchronize()
        model.use_prefill_matrices(True)
        ws.free()
        pbuf.free()
        sess.free()
        model.free()
        return {"tokens": n, "calls": 6, "parity_ok": True}

    # parity against the decode-step path on the same prompt
    one(sess.logits.ptr)
    stream.synchronize()
    la = sess.read_logits()
    tok_b = sess.get_state()[0]
    ref = D.DecodeSession(model, n, stream)
    ref.set_state(0, 0)
    t0 = time.perf_counter()
    if n > 1:
        ref.prefill(prompt[:-1])
    ref.set_state(int(prompt[-1]), n - 1)
    ref.step(advance=True, logits=True)
    ref.synchronize()
    steps_ms = (time.perf_counter() - t0) * 1e3
    lb = ref.read_logits()
    tok_s = ref.get_state()[0]
    dl = np.abs(la.astype(np.float64) - lb.astype(np.float64))
    rel = float(np.linalg.norm(dl) / np.linalg.norm(lb.astype(np.float64)))
    srt = np.sort(lb.astype(np.float64))
    margin = float(srt[-1] - srt[-2])
    ok = rel < 2e-2 and (tok_b == tok_s or margin <= 2 * dl.max())
    ref.free()
    log(f"prefill parity: token {tok_b} (decode steps {tok_s}, margin {margin:.4f}), logits rel L2 "
        f"{rel:.2e}")
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < MIN_WARM_MS:
        one()
    stream.synchronize()
    reps = max(5, min(50, args.steps // 20))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        one()
        stream.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    ms = statistics.mean(times)
    gemm, attn = prefill_flops(n)
    log(f"prefill of {n} tokens: {ms:.3f} ms (median {statistics.median(times):.3f}) = "
        f"{n / ms * 1e3:.0f} tok/s, {(gemm + attn) / ms / 1e9:.1f} TFLOP/s; as decode steps "
        f"{steps_ms:.1f} ms")
    def mean_ms():
        for _ in range(3):
            one()
        stream.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            one()
        stream.synchronize()
        return (time.perf_counter() - t0) * 1e3 / reps

    for spec in args.prefill_tiling or []:
        rows, split = (int(x) for x in spec.split(":"))
        D.set_prefill_tiling(rows, split)
        log(f"  tiling gemm_rows {rows} attn_split_blocks {split}: {mean_ms():.3f} ms")
    D.set_prefill_tiling(0, 0)
    # the same calls with the GEMMs forming the f16 weights from the Q8_0
    # stacks in registers (no f16 matrices): same bits, for comparison
    model.use_prefill_matrices(False)
    q8_ms = mean_ms()
    model.use_prefill_matrices(True)
    log(f"  GEMMs over the Q8_0 stacks instead of the f16 matrices: {q8_ms:.3f} ms")
    ws.free()
    pbuf.free()
    sess.free()
    model.free()
    return {"tokens": n, "ms": round(ms, 3), "median_ms": round(statistics.median(times), 3),
            "tok_per_s": round(n / ms * 1e3, 1), "q8_stacks_ms": round(q8_ms, 3),
            "gemm_flops": gemm, "attention_flops": attn,
            "TFLOPs": round((gemm + attn) / ms / 1e9, 2),
            "decode_steps_ms": round(steps_ms, 2), "speedup_vs_steps": round(steps_ms / ms, 1),
            "logits_rel_l2_vs_steps": rel, "token": tok_b, "steps_token": tok_s,
            "parity_ok": bool(ok)}


def bench_generate(Q, stream, args) -> dict:
    """End-to-end generation as the reference measures it
    (scripts/benchmark.py:52-81): the wall time of one `run` = a fresh KV
    cache, prompt ingestion (batched, the reference's @prefill), then up to
    128 greedy tokens with the EOS check after every 4 (qwen3_full.mlir:
    2113-2167); tok/s = tokens before EOS / that time.  Prompts: a chat-sized
    one (the reference's prompts with its chat template are ~10-30 tokens) and
    512 tokens.  Parity: the same tokens as the prompt followed by single
    decode steps read back one at a time."""
    from qwen3_iree_amd import decode as D

    mhost = D.synthetic_weights(seed=SEED, workers=16)
    model = D.DeviceWeights(mhost)
    rng = np.random.default_rng(SEED + 13)
    out = {}
    for name, n in (("chat_prompt", args.chat_prompt_tokens), ("prompt_512", 512)):
        prompt = rng.integers(0, D.VOCAB, n).astype(np.int32)
        toks = D.run(model, prompt, MAX_NEW_TOKENS, EOS_TOKEN, stream)  # warm-up + parity
        # parity: prompt, then single steps with the token read back each time
        sess = D.DecodeSession(model, n + MAX_NEW_TOKENS, stream)
        sess.set_state(0, 0)
        sess.prefill_batched(prompt)
        steps = []
        while len(steps) < len(toks):
            sess.step(advance=True, logits=False)
            steps.append(sess.get_state()[0])
        sess.check_status()
        sess.free()
        parity = steps == toks.tolist()
        times = []
        reps = max(3, args.generate_reps)
        t_end = time.perf_counter() + MIN_WARM_MS / 1e3
        while time.perf_counter() < t_end:
            D.run(model, prompt, MAX_NEW_TOKENS, EOS_TOKEN, stream)
        for _ in range(reps):
            t0 = time.perf_counter()
            got = D.run(model, prompt, MAX_NEW_TOKENS, EOS_TOKEN, stream)
            times.append(time.perf_counter() - t0)
        produced = got.tolist()
        n_out = produced.index(EOS_TOKEN) if EOS_TOKEN in produced else len(produced)
        # the token loop alone (qwen3_generate), after the prompt
        sess = D.DecodeSession(model, n + MAX_NEW_TOKENS, stream)
        sess.set_state(0, 0)
        sess.prefill_batched(prompt)
        t0 = time.perf_counter()
        loop = sess.generate(MAX_NEW_TOKENS, EOS_TOKEN)
        loop_s = time.perf_counter() - t0
        sess.free()
        dt = statistics.median(times)
        rec = {"prompt_tokens": n, "max_new_tokens": MAX_NEW_TOKENS, "tokens_out": n_out,
               "run_ms": round(dt * 1e3, 3), "run_ms_mean": round(statistics.mean(times) * 1e3, 3),
               "tok_per_s": round(n_out / dt, 1), "runs": reps,
               "loop_ms_per_token": round(loop_s * 1e3 / max(1, len(loop)), 4),
               "parity_ok": bool(parity and got.tolist() == toks.tolist())}
        log(f"generate ({name}: {n}-token prompt + {MAX_NEW_TOKENS} tokens): run {dt * 1e3:.2f} ms "
            f"-> {rec['tok_per_s']:.0f} tok/s ({n_out} tokens before EOS), token loop "
            f"{rec['loop_ms_per_token']:.4f} ms/token, parity {rec['parity_ok']}")
        out[name] = rec
    out["reference_protocol"] = reference_protocol(D, model, stream, rng)
    model.free()
    out["reference_published"] = {"tok_per_s": 25.52, "where": "Jetson AGX Orin, "
                                  "benchmark.json:71-72 (other hardware)"}
    return out


def reference_protocol(D, model, stream, rng) -> dict:
    """The reference's end-to-end protocol (scripts/benchmark.py:52-81,
    137-155, 203-214): ten chat prompts, one timed `run` each (wall time of
    the call: prompt ingestion + up to 128 tokens with the EOS check every 4),
    tok/s per prompt = tokens before EOS / that time, then the mean and the
    population standard deviation; the record repeats the reference's JSON
    schema {variant: {tps, mean, std, prompts}}.  The prompts are synthetic
    ids in the chat template's shape (im_start, 2 role tokens, the text,
    im_end, newline, im_start, 2 role tokens) at the lengths of
    REFERENCE_PROMPT_TOKENS.  Parity: each timed run gives the tokens of an
    untimed run of the same prompt made before it."""
    prompts = []
    for n in REFERENCE_PROMPT_TOKENS:
        ids = rng.integers(0, D.VOCAB - 2, n).astype(np.int32)
        ids[0] = IM_START
        ids[n - 5] = EOS_TOKEN   # <|im_end|> closes the user turn
        ids[n - 3] = IM_START
        prompts.append(ids)
    want = [D.run(model, p, MAX_NEW_TOKENS, EOS_TOKEN, stream) for p in prompts]
    t_end = time.perf_counter() + MIN_WARM_MS / 1e3
    while time.perf_counter() < t_end:
        D.run(model, prompts[0], MAX_NEW_TOKENS, EOS_TOKEN, stream)
    tps, ms, outs, ok = [], [], [], True
    for p, w in zip(prompts, want):
        t0 = time.perf_counter()
        got = D.run(model, p, MAX_NEW_TOKENS, EOS_TOKEN, stream)
        dt = time.perf_counter() - t0
        toks = got.tolist()
        n_out = toks.index(EOS_TOKEN) if EOS_TOKEN in toks else len(toks)
        ok = ok and toks == w.tolist()
        tps.append(n_out / dt)
        ms.append(round(dt * 1e3, 3))
        outs.append(n_out)
    mean, std = float(np.mean(tps)), float(np.std(tps))
    log(f"generate (reference protocol, 10 chat prompts of {min(REFERENCE_PROMPT_TOKENS)}-"
        f"{max(REFERENCE_PROMPT_TOKENS)} tokens + {MAX_NEW_TOKENS}): {mean:.1f} +- {std:.1f} "
        f"tok/s, parity {ok}")
    return {"mi355x_hip": {"tps": [round(t, 2) for t in tps], "mean": round(mean, 2),
                           "std": round(std, 2),
                           "prompts": [f"synthetic chat prompt, {n} tokens"
                                       for n in REFERENCE_PROMPT_TOKENS]},
            "prompt_tokens": list(REFERENCE_PROMPT_TOKENS), "tokens_out": outs, "run_ms": ms,
            "warm_up_ms": MIN_WARM_MS, "parity_ok": bool(ok),
            "reference_published": {"mean": 25.52, "std": 1.72,
                                    "where": "Jetson AGX Orin, benchmark.json:71-72"}}


def bench_gguf(Q, tmpdir: Path) -> dict:
    """GGUF -> HostWeights -> device: throughput of each stage on the full-size
    synthetic checkpoint (1.09 GB of parameters)."""
    from qwen3_iree_amd import decode as D
    from qwen3_iree_amd import gguf as G

    hw = D.synthetic_weights(seed=SEED, workers=16)
    tmpdir.mkdir(parents=True, exist_ok=True)
    path = tmpdir / "qwen3-0.6b-synthetic-q8_0.gguf"
    t0 = time.perf_counter()
    G.write_qwen3_gguf(hw, path)
    write_s = time.perf_counter() - t0
    size = path.stat().st_size
    reads = []
    for _ in range(3):
        t0 = time.perf_counter()
        got = G.qwen3_host_weights(path, workers=16)
        reads.append(time.perf_counter() - t0)
    same = all(np.array_equal(getattr(got, f).view(np.uint8), getattr(hw, f).view(np.uint8))
               for f in D.WEIGHT_FIELDS)
    t0 = time.perf_counter()
    model = D.DeviceWeights(got)
    Q.synchronize()
    upload_s = time.perf_counter() - t0
    nbytes = model.nbytes
    model.free()
    path.unlink()
    log(f"gguf: {size} B file written in {write_s:.2f}s; read into the device layout in "
        f"{reads[0]:.2f}s (first), {min(reads[1:]):.3f}s (warm cache); upload {upload_s:.2f}s; "
        f"identical={same}")
    return {"file_bytes": size, "param_bytes": nbytes, "write_s": round(write_s, 3),
            "read_first_s": round(reads[0], 3), "read_warm_s": round(min(reads[1:]), 3),
            "read_warm_GBps": round(nbytes / min(reads[1:]) / 1e9, 2),
            "upload_s": round(upload_s, 3), "upload_GBps": round(nbytes / upload_s / 1e9, 2),
            "bit_identical": bool(same)}


def cpu_baseline(O, sw, args) -> dict:
    """The C oracle (reference kernels' f32 order) over whole sweeps of the same
    inputs: at every host thread for ~cpu_seconds, then at one thread for
    ~cpu_seconds / 2."""
    host = {k: v for k, v in sw.host_w.items()}

    def sample(threads: int, budget: float):
        O.set_num_threads(threads)
        sweeps = 0
        t0 = time.perf_counter()
        while True:
            for layer, d in sw.order:
                O.q8_gemv(host[d.kind][layer], d.n, d.k, sw.host_x[(layer, d.kind)])
            sweeps += 1
            if time.perf_counter() - t0 >= budget:
                break
        return sweeps, time.perf_counter() - t0

    # every thread OpenMP is allowed (OMP_NUM_THREADS: the host's share of
    # cores for this GPU), then one
    all_threads = O.num_threads()
    n_all, s_all = sample(all_threads, args.cpu_seconds)
    threads_used = O.num_threads()
    n_one, s_one = sample(1, args.cpu_seconds / 2)
    O.set_num_threads(all_threads)
    gbs_all = sw.bytes_per_step * n_all / s_all / 1e9
    gbs_one = sw.bytes_per_step * n_one / s_one / 1e9
    log(f"cpu oracle: {gbs_all:.2f} GB/s over {n_all} sweeps ({threads_used} threads), "
        f"{gbs_one:.2f} GB/s over {n_one} sweeps (1 thread); {cpu_model()}")
    return {"value": round(gbs_all, 3), "unit": "GB/s", "cores": threads_used, "kind": "port",
            "sample": f"{n_all} full 28-layer sweeps (140 Q8_0 GEMVs each, the same inputs) with the "
                      f"C oracle in the reference kernels' f32 order, OpenMP {threads_used} threads, "
                      f"{s_all:.1f}s; then {n_one} sweeps on 1 thread, {s_one:.1f}s",
            "ms_per_step": round(1e3 * s_all / n_all, 3),
            "single_thread": {"value": round(gbs_one, 3), "unit": "GB/s",
                              "ms_per_step": round(1e3 * s_one / n_one, 3), "cores": 1},
            "cpu_model": cpu_model(), "host_logical_cpus": os.cpu_count()}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=1000,
                    help="untimed steps before timing; at least 200 ms of the timed kernel runs "
                         "whatever this is (the GPU clock ramps over the first ~100 ms)")
    ap.add_argument("--context", type=int, default=1024,
                    help="positions attended by the timed decode step")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the full decode step and print its JSON line")
    ap.add_argument("--sweep-only", action="store_true",
                    help="run only the batched sweep (timed, parity-checked) and print its line")
    ap.add_argument("--kernels-only", action="store_true",
                    help="run only the GEMV kernels (batched sweep, per-dispatch sweep, vocab, the "
                         "decode step's GEMV share) and print the line without the decode step, "
                         "prompt, generation and CPU parts (for counter runs); with "
                         "--prefill-only: three untimed prompt calls over the f16 matrices and "
                         "three over the Q8_0 stacks, no parity check")
    ap.add_argument("--scrub-only", action="store_true",
                    help="run only the MALL-scrub A/B of the batched sweep kernel and the vocab "
                         "kernel (per-launch events; for kernel traces of both cases) and print "
                         "its JSON line")
    ap.add_argument("--scrub-launches", type=int, default=30,
                    help="launches per case of the MALL-scrub A/B")
    ap.add_argument("--generate-only", action="store_true",
                    help="run only end-to-end generation and print its JSON line")
    ap.add_argument("--step-mode", type=int, choices=(0, 1), default=None,
                    help="decode step mode for the whole run (0: per-phase launches, 1: one "
                         "launch per step; default: the library's)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only batched prompt ingestion and print its JSON line")
    ap.add_argument("--prefill-tokens", type=int, default=512,
                    help="prompt length of the batched prompt ingestion measurement")
    ap.add_argument("--prefill-tiling", nargs="*", metavar="ROWS:SPLIT",
                    help="also time the prompt ingestion with these work divisions "
                         "(qwen3_set_prefill_tiling; 0 = by shape)")
    ap.add_argument("--chat-prompt-tokens", type=int, default=24,
                    help="prompt length of the chat-sized generation measurement")
    ap.add_argument("--generate-reps", type=int, default=5, help="timed runs per generation case")
    ap.add_argument("--gguf-ingest", metavar="DIR", default=None,
                    help="only measure GGUF ingestion: write the synthetic model as a Q8_0 GGUF "
                         "under DIR, read it back into the device layout (cold, then warm page "
                         "cache), upload it, check it bit for bit, print one JSON line")
    ap.add_argument("--copies", type=int, default=3,
                    help="identical weight copies the sweep and vocab steps take in turn (the "
                         "MALL holds none of a copy by its next turn)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--per-phase-only", action="store_true",
                    help="decode step: time only the per-phase launches, not the single "
                         "launch (traces of the per-phase kernels alone)")
    ap.add_argument("--no-calibration", action="store_true",
                    help="decode step: skip the launch-cost and hand-off measurements (their "
                         "cooperative launches are kept out of profiler runs)")
    ap.add_argument("--no-graph", action="store_true",
                    help="issue the per-dispatch and decode-step chains eagerly instead of from hipGraphs")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="first run the plain copy kernel over MIB MiB five times (a kernel of known "
                         "traffic for scaling HBM byte counters)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this path runs on one GPU; --gpus {args.gpus} (WORLD_SIZE={world}) "
              "is not supported. Run with --gpus 1.", file=sys.stderr)
        return 2

    from __graft_entry__ import load_package

    load_package()
    from qwen3_iree_amd import q8gemv as Q
    from qwen3_iree_amd import sweep as S

    Q.init()
    info = Q.device_info()
    log(f"device {info['name']}, {info['compute_units']} CUs")
    sys.path.insert(0, str(REPO / "oracle"))
    import oracle as O  # the checker; also the CPU baseline below

    try:
        return run(Q, S, O, info, args)
    finally:
        Q.teardown()


def run(Q, S, O, info, args) -> int:
    if args.step_mode is not None:
        from qwen3_iree_amd import decode as D

        D.set_step_mode(args.step_mode)
    if args.gguf_ingest:
        print(json.dumps({"gguf_ingest": bench_gguf(Q, Path(args.gguf_ingest))}), flush=True)
        return 0
    if args.decode_only:
        stream = Q.Stream()
        copy_calibration(Q, stream, args.copy_calibration)
        print(json.dumps({"decode_step": bench_decode(Q, O, stream, args)}), flush=True)
        return 0
    if args.prefill_only:
        print(json.dumps({"prefill": bench_prefill(Q, Q.Stream(), args)}), flush=True)
        return 0
    if args.generate_only:
        print(json.dumps({"generate": bench_generate(Q, Q.Stream(), args)}), flush=True)
        return 0

    # ---------------------------------------------------------------- inputs
    t0 = time.time()
    sw = S.build(SEED, copies=args.copies)
    layers = S.LAYERS
    sweep_bytes = sw.bytes_per_step
    log(f"sweep inputs ready in {time.time() - t0:.1f}s: {sw.weight_bytes} weight bytes "
        f"(x {sw.n_copies} copies), {sweep_bytes} algorithmic bytes per step")
    stream = Q.Stream()

    copy_cal = copy_calibration(Q, stream, args.copy_calibration)

    # ------------------------------------------- headline: batched sweep
    # Step i reads weight copy i mod copies: the MALL (256 MB) cannot hold a
    # copy until its next turn, (copies - 1) x 437 MB later.
    batches = [sw.batch(c) for c in range(sw.n_copies)]
    turn = [0]

    def launch():
        batches[turn[0] % len(batches)].launch(stream)
        turn[0] += 1

    warm_calls = warm(stream, launch, args.warmup)
    t_wall = time.perf_counter()
    th = timed(Q, stream, launch, args.steps)
    wall_s = time.perf_counter() - t_wall
    ms_per_step = th["mean_ms"]
    value = sweep_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"batched sweep ({sw.n_copies} weight copies in turn): {ms_per_step * 1e3:.2f} us/step "
        f"(median of {th['blocks']} blocks {th['median_ms'] * 1e3:.2f}, after {warm_calls} "
        f"warm-up launches), {value:.1f} GB/s ({100 * value / HBM_PEAK_GBS:.1f}% of peak); host "
        f"wall {wall_s:.3f}s")
    # the same launches always on one copy (each step re-reads what the last
    # one read, 437 MB earlier): what the memory-side cache adds
    batch = batches[0]
    one_copy = lambda: batch.launch(stream)  # noqa: E731
    warm(stream, one_copy, 10)
    t1 = timed(Q, stream, one_copy, max(50, args.steps // 4))
    log(f"  the same on one copy: {t1['mean_ms'] * 1e3:.2f} us/step "
        f"({sweep_bytes / t1['mean_ms'] / 1e6:.1f} GB/s)")

    # the kernel alone after a MALL scrub (A/B with per-launch events)
    launch = one_copy
    scrub = (Q.DeviceBuffer(SCRUB_BYTES), SCRUB_BYTES)
    scrub[0].fill(0)
    sweep_scrub = scrub_ab(Q, stream, launch, scrub, args.scrub_launches)
    log(f"batched sweep kernel alone: {sweep_scrub['unscrubbed_us']} us, after a MALL scrub "
        f"{sweep_scrub['scrubbed_us']} us (ratio {sweep_scrub['ratio']})")

    if args.scrub_only:
        from qwen3_iree_amd import weights as Wt

        for b in batches:
            b.free()
        sw.free()
        Wv = Wt.synthetic_f16_matrix(Q.VOCAB_ROWS, Q.HIDDEN, seed=SEED, tensor=24, workers=16)
        wv_dev = Q.DeviceBuffer.from_array(Wv)
        xv_dev = Q.DeviceBuffer.from_array(Wt.synthetic_x(Q.HIDDEN, SEED, index=9999))
        logits_dev, tok_dev = Q.DeviceBuffer(2 * Q.VOCAB_ROWS), Q.DeviceBuffer(16)
        ws = Q.DeviceBuffer(Q.vocab_workspace_bytes())
        Q.vocab_workspace_reset(ws, stream)
        vocab_scrub = scrub_ab(Q, stream, lambda: Q.vocab_gemv_argmax(
            wv_dev, xv_dev, logits_dev, tok_dev, ws, stream), scrub, args.scrub_launches)
        log(f"vocab GEMV kernel alone: {vocab_scrub['unscrubbed_us']} us, after a MALL scrub "
            f"{vocab_scrub['scrubbed_us']} us (ratio {vocab_scrub['ratio']})")
        for b in (wv_dev, xv_dev, logits_dev, tok_dev, ws, scrub[0]):
            b.free()
        print(json.dumps({"scrub_ab": {"q8gemv_batch_k": sweep_scrub,
                                       "vocab_gemv_argmax_k1024": vocab_scrub}}), flush=True)
        return 0

    # parity of every sweep output (the last timed launch wrote them)
    fails = floor = 0
    for layer, d in sw.order:
        raw = sw.host_w[d.kind][layer]
        x = sw.host_x[(layer, d.kind)]
        rep = O.gemv_tolerance_report(sw.dev_y[(layer, d.kind)].download(np.float16),
                                      O.q8_gemv(raw, d.n, d.k, x), O.q8_gemv_f64(raw, d.n, d.k, x)[1])
        fails += rep["fail"]
        floor += rep["on_floor"]
    log(f"parity: {fails} failing outputs of {sw.outputs} ({floor} on the noise floor)")

    batch_grid = min(batch.total_units, 10 * info["compute_units"]) * 64
    traffic = profiled_traffic("q8gemv_batch_k", batch_grid)
    if traffic["stale"]:
        log("profiles/traffic.json was taken on another build of q8gemv_batch_k (digest "
            f"{traffic['code_digest']}): its traffic figure does not describe this build")
    headline = {
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
            "workload": "28-layer stacked cold-cache Q8_0 GEMV sweep: per layer attn_q, attn_kv, "
                        "attn_o, gate_up, ffn_dn (140 GEMVs), one batched launch per step; "
                        f"steps take {sw.n_copies} identical weight copies in turn, so no step "
                        "finds its weights in the 256 MB MALL",
            "weight_copies": sw.n_copies,
            "layers": layers,
            "gemvs_per_step": len(sw.order),
            "weight_bytes": sw.weight_bytes,
            "algorithmic_bytes_per_step": sweep_bytes,
            "device": info["name"],
        },
        "pct_of_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "us_per_step": round(ms_per_step * 1e3, 2),
        "median_us_per_step": round(th["median_ms"] * 1e3, 2),
        "warmup_launches": warm_calls,
        "roofline": {
            "bound": "hbm",
            "kernel": "q8gemv_batch_k (28-layer sweep, 140 GEMVs)",
            "achieved": round(value, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4),
            "avg_us": round(ms_per_step * 1e3, 2),
            "median_us": round(th["median_ms"] * 1e3, 2),
            "bytes_per_launch": sweep_bytes,
            "traffic": traffic["bytes"],
            "traffic_source": "profiles/traffic.json: rocprofv3 FETCH_SIZE + WRITE_SIZE per dispatch, "
                              "each scaled by its reading for the plain copy kernel of known size",
            "traffic_code_digest": traffic["code_digest"],
            "traffic_stale": traffic["stale"],
            "profiled_mean_us": traffic.get("profiled_mean_us"),
            "scrubbed_us": sweep_scrub["scrubbed_us"],
            "scrub_ab": sweep_scrub,
            "one_copy_us": round(t1["mean_ms"] * 1e3, 2),
            "one_copy_frac": round(sweep_bytes / t1["mean_ms"] / 1e6 / HBM_PEAK_GBS, 4),
        },
        "parity_ok": fails == 0,
        "copy_calibration": copy_cal,
    }
    for b in batches:
        b.free()
    if args.sweep_only:
        print(json.dumps(headline), flush=True)
        sw.free()
        scrub[0].free()
        return 0

    # ------------------------------- the same sweep as 140 dispatches
    # (the weight copies in turn, as above)
    chain_turn = [0]
    if args.no_graph:
        def chain_fn():
            sw.record_dispatches(stream, chain_turn[0] % sw.n_copies)
            chain_turn[0] += 1
    else:
        graphs = [Q.Graph(stream, lambda c=c: sw.record_dispatches(stream, c))
                  for c in range(sw.n_copies)]

        def chain_fn():
            graphs[chain_turn[0] % len(graphs)].launch(stream)
            chain_turn[0] += 1
    warm(stream, chain_fn, 3)
    tc = timed(Q, stream, chain_fn, max(10, args.steps // 4))
    chain_ms = tc["mean_ms"]
    chain_gbs = sweep_bytes / (chain_ms * 1e-3) / 1e9
    log(f"per-dispatch sweep (140 launches{'' if args.no_graph else ', hipGraph'}): "
        f"{chain_ms * 1e3:.1f} us (median {tc['median_ms'] * 1e3:.1f}), {chain_gbs:.1f} GB/s")
    # its floor: 140 stream-ordered empty launches the same way (one workgroup each)
    def record_empty():
        for _ in range(len(sw.order)):
            Q.stream_copy(None, None, 0, stream)

    if args.no_graph:
        floor_fn = record_empty
    else:
        fgraph = Q.Graph(stream, record_empty)
        floor_fn = lambda: fgraph.launch(stream)  # noqa: E731
    warm(stream, floor_fn, 3)
    tf = timed(Q, stream, floor_fn, max(10, args.steps // 4))
    floor_us = tf["mean_ms"] * 1e3
    log(f"  its floor, 140 empty launches the same way: {floor_us:.1f} us")
    # and what each dispatch must wait for before its first weight bytes: one
    # dependent load from HBM (lines evicted from L2 and the MALL first)
    mem = Q.memory_latency(4096)
    bound_us = floor_us + len(sw.order) * mem["hbm_ns"] * 1e-3 + sw.bytes_per_step / HBM_PEAK_GBS / 1e3
    log(f"  dependent load: HBM {mem['hbm_ns']:.0f} ns, MALL {mem['mall_ns']:.0f} ns, L2 "
        f"{mem['l2_ns']:.0f} ns; floor + 140 HBM loads + bytes at 8 TB/s = {bound_us:.1f} us")
    # the same 140 GEMVs through the reference's HAL binding ABI (the kernels an
    # IREE executable substitution would launch), outputs checked against the
    # C-ABI dispatches' bit for bit
    hal_binds = sw.hal_bindings()
    hal_turn = [0]
    if args.no_graph:
        def hal_fn():
            sw.record_hal_dispatches(hal_binds, stream, hal_turn[0] % sw.n_copies)
            hal_turn[0] += 1
    else:
        hgraphs = [Q.Graph(stream, lambda c=c: sw.record_hal_dispatches(hal_binds, stream, c))
                   for c in range(sw.n_copies)]

        def hal_fn():
            hgraphs[hal_turn[0] % len(hgraphs)].launch(stream)
            hal_turn[0] += 1
    warm(stream, hal_fn, 3)
    th = timed(Q, stream, hal_fn, max(10, args.steps // 4))
    hal_us = th["mean_ms"] * 1e3
    sw.record_dispatches(stream)
    stream.synchronize()
    hal_same = all(np.array_equal(
        b2.download(np.uint16, d.n, y_off),
        sw.dev_y[(layer, d.kind)].download(np.uint16, d.n))
        for (layer, d), (_, b2, y_off) in ((k, hal_binds[(k[0], k[1].kind)]) for k in sw.order))
    log(f"  through the HAL binding ABI (q8gemv_hal_dispatch): {hal_us:.1f} us, outputs "
        f"identical to the C ABI's: {hal_same}")
    for b1, b2, _ in hal_binds.values():
        b1.free()
        b2.free()

    # ------------------------------------------------------------- vocab
    from qwen3_iree_amd import weights as Wt

    t0 = time.time()
    Wv = Wt.synthetic_f16_matrix(Q.VOCAB_ROWS, Q.HIDDEN, seed=SEED, tensor=24, workers=16)
    xv = Wt.synthetic_x(Q.HIDDEN, SEED, index=9999)
    wv_devs = [Q.DeviceBuffer.from_array(Wv) for _ in range(args.copies)]  # identical copies
    wv_dev = wv_devs[0]
    xv_dev = Q.DeviceBuffer.from_array(xv)
    logits_dev = Q.DeviceBuffer(2 * Q.VOCAB_ROWS)
    tok_dev = Q.DeviceBuffer(16)
    ws = Q.DeviceBuffer(Q.vocab_workspace_bytes())
    Q.vocab_workspace_reset(ws, stream)
    log(f"vocab inputs ready in {time.time() - t0:.1f}s")
    vocab_bytes = Q.VOCAB.bytes_per_layer + 2 * Q.HIDDEN + 2 * Q.VOCAB_ROWS + 4
    vocab_fn = lambda: Q.vocab_gemv_argmax(wv_dev, xv_dev, logits_dev, tok_dev, ws, stream)  # noqa: E731
    vturn = [0]

    def vocab_turns():  # the copies in turn, as the sweep
        Q.vocab_gemv_argmax(wv_devs[vturn[0] % len(wv_devs)], xv_dev, logits_dev, tok_dev, ws,
                            stream)
        vturn[0] += 1

    warm(stream, vocab_turns, 5)
    tv = timed(Q, stream, vocab_turns, 200)
    warm(stream, vocab_fn, 5)
    tv1 = timed(Q, stream, vocab_fn, 100)
    v_ms = tv["mean_ms"]
    v_gbs = vocab_bytes / (v_ms * 1e-3) / 1e9
    token = int(tok_dev.download(np.int32, 1)[0])
    logits = logits_dev.download(np.float16, Q.VOCAB_ROWS)
    rep_v = O.gemv_tolerance_report(logits, O.f16_gemv(Wv, xv), O.f16_gemv_f64(Wv, xv)[1])
    own = O.argmax_tiled(logits)
    log(f"vocab GEMV + argmax ({len(wv_devs)} matrix copies in turn): {v_ms * 1e3:.2f} us/op "
        f"(median {tv['median_ms'] * 1e3:.2f}), {v_gbs:.0f} GB/s, token {token} (argmax of own "
        f"logits {own}, {rep_v['fail']} failing logits); one copy {tv1['mean_ms'] * 1e3:.2f} us")
    vocab_scrub = scrub_ab(Q, stream, vocab_fn, scrub, args.scrub_launches)
    log(f"vocab GEMV kernel alone: {vocab_scrub['unscrubbed_us']} us, after a MALL scrub "
        f"{vocab_scrub['scrubbed_us']} us (ratio {vocab_scrub['ratio']})")

    # ---------------------------------------- GEMV share of a decode step
    # Separate K and V weights (the attn_kv stack above serves as K).
    v_host = Wt.synthetic_q8_stack(1024, 1024, layers, seed=SEED, tensor=7, workers=16)
    v_dev = Q.DeviceBuffer.from_array(v_host)
    step_y = {name: Q.DeviceBuffer(2 * 6144) for name in ("q", "k", "v", "o", "gu", "dn")}

    def record_decode_gemvs():
        for layer in range(layers):
            Q.q8gemv_qkv(sw.dev_w[Q.ATTN_Q.kind], sw.dev_w[Q.ATTN_KV.kind], v_dev, layer,
                         sw.dev_x[(layer, Q.ATTN_Q.kind)], step_y["q"], step_y["k"], step_y["v"],
                         stream)
            for d, yname in ((Q.ATTN_O, "o"), (Q.GATE_UP, "gu"), (Q.FFN_DN, "dn")):
                Q.q8gemv(d.kind, sw.dev_w[d.kind], layer, sw.dev_x[(layer, d.kind)], step_y[yname],
                         stream)
        vocab_fn()

    if args.no_graph:
        dstep_fn = record_decode_gemvs
    else:
        dgraph = Q.Graph(stream, record_decode_gemvs)
        dstep_fn = lambda: dgraph.launch(stream)  # noqa: E731
    warm(stream, dstep_fn, 3)
    td = timed(Q, stream, dstep_fn, 50)
    decode_gemv_us = td["mean_ms"] * 1e3
    decode_bytes = (sum(S.algorithmic_bytes(d) for d in Q.LAYER_ORDER) * layers + vocab_bytes)
    log(f"decode-step GEMVs (28 x [q8gemv_qkv, o, gate_up, down] + vocab, 114 dispatches): "
        f"{decode_gemv_us:.1f} us, {decode_bytes / decode_gemv_us / 1e3:.0f} GB/s")
    for b in (*wv_devs, xv_dev, logits_dev, tok_dev, ws, v_dev, *step_y.values(), scrub[0]):
        b.free()
    kernels = {
        "per_dispatch_sweep": {"us": round(chain_ms * 1e3, 1),
                               "median_us": round(tc["median_ms"] * 1e3, 1),
                               "GBps": round(chain_gbs, 1),
                               "frac": round(chain_gbs / HBM_PEAK_GBS, 4), "dispatches": 140,
                               "launch": "eager" if args.no_graph else "hipGraph",
                               "floor_us": round(floor_us, 1),
                               "hal_abi_us": round(hal_us, 1),
                               "hal_abi_parity_ok": bool(hal_same),
                               "floor": "140 empty launches (one workgroup each), stream-ordered "
                                        "the same way",
                               "memory_latency": mem,
                               "bound_us": round(bound_us, 1),
                               "bound": "floor_us + 140 x memory_latency.hbm_ns (each dispatch's "
                                        "first weight bytes) + the sweep's bytes at 8 TB/s"},
        "vocab": {"us": round(v_ms * 1e3, 2), "median_us": round(tv["median_ms"] * 1e3, 2),
                  "GBps": round(v_gbs, 1), "frac": round(v_gbs / HBM_PEAK_GBS, 4),
                  "bytes": vocab_bytes, "token": token, "parity_ok": rep_v["fail"] == 0 and token == own,
                  "weight_copies": len(wv_devs), "one_copy_us": round(tv1["mean_ms"] * 1e3, 2),
                  "scrub_ab": vocab_scrub},
        "decode_step_gemv": {"us": round(decode_gemv_us, 2), "bytes": decode_bytes,
                             "GBps": round(decode_bytes / decode_gemv_us / 1e3, 1),
                             "dispatches": 4 * layers + 2,
                             "launch": "eager" if args.no_graph else "hipGraph"},
    }
    if args.kernels_only:
        out = dict(headline)
        out.update(kernels)
        out["parity_ok"] = bool(fails == 0 and rep_v["fail"] == 0 and token == own)
        print(json.dumps(out), flush=True)
        sw.free()
        return 0

    # ------------------------------------------- full decode step (C5)
    dec = bench_decode(Q, O, stream, args)
    pre = bench_prefill(Q, stream, args)
    gen = bench_generate(Q, stream, args)
    gen_ok = all(v.get("parity_ok", True) for v in gen.values() if isinstance(v, dict))

    parity_ok = (fails == 0 and rep_v["fail"] == 0 and token == own and dec["parity_ok"]
                 and pre["parity_ok"] and gen_ok and hal_same)

    # ------------------------------------------------------ CPU baseline
    cpu = None if args.no_cpu else cpu_baseline(O, sw, args)
    sw.free()

    out = dict(headline)
    out.update(kernels)
    out.update({
        "decode_step": dec,
        "prefill": pre,
        "generate": gen,
        "parity_ok": bool(parity_ok),
        "cpu_baseline": cpu,
    })
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
