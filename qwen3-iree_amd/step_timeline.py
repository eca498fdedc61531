#!/usr/bin/env python3
"""Where the single-launch decode step's time goes, phase by phase.

rocprofv3 sees one kernel (dec_step) per step, so this builds the decode code
object with -DDEC_STEP_STAMPS=1 (thread 0 of 16 chosen workgroups reads the
100 MHz real-time counter at every phase boundary, see decode_kernels.hip)
into a temporary directory beside copies of the other code objects, runs
steps at a given context on random-init weights, and prints, per phase, when
it completes relative to the layer's start on workgroup 0, averaged over
layers 1..27, as a markdown report.

    python3 qwen3-iree_amd/step_timeline.py [--context 1024] [--steps 20]

The timestamp build runs the same operations as the product build (the clock
reads add a few instructions per phase), so its step time is printed beside
the product's for comparison.
"""
from __future__ import annotations

import argparse
import shutil
import statistics
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
REPO = PKG.parent

POINTS = {0: "layer start", 1: "A: h ready", 13: "A: x normalised", 2: "A: q/k/v published",
          3: "B: q/k/v ready", 16: "B: head norms + RoPE done", 17: "B: score MFMAs issued",
          18: "B: softmax done", 19: "B: chunk loop done", 20: "B: four waves merged in LDS",
          4: "B: partial published", 5: "merge: partials ready",
          6: "merge: attention published", 14: "C: h rows ready",
          7: "C: attention ready", 8: "C: residual published",
          15: "D: gate/up weights requested", 9: "D: residual ready",
          10: "D: SwiGLU published", 11: "E: SwiGLU ready", 12: "E: h published"}
VOCAB_POINTS = {0: "vocab start", 1: "vocab: h ready", 2: "vocab: key published",
                3: "keys ready (wg 0)", 4: "token written (wg 0)"}
STAMP_WGS = (0, 1, 100, 191, 192, 255, 256, 257, 264, 319, 320, 321, 383, 384, 446, 447)
TICK_US = 0.01  # s_memrealtime: 100 MHz
N_POINTS = 21    # kStampPoints


def build_stamped(dst: Path) -> Path:
    sys.path.insert(0, str(PKG))
    import build as B

    for name in ("q8gemv_gfx950.hsaco", "prefill_gfx950.hsaco"):
        shutil.copy(B.LIB / name, dst / name)
    B._run([str(B.ROCM / "bin" / "hipcc"), *B.HIPCC_FLAGS, "-DDEC_STEP_STAMPS=1", f"-I{B.CSRC}",
            str(B.CSRC / "decode_kernels.hip"), "-o", str(dst / "decode_gfx950.hsaco")])
    return dst / "q8gemv_gfx950.hsaco"


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--context", type=int, default=1024)
    ap.add_argument("--steps", type=int, default=20, help="stamped steps (the last one is read)")
    ap.add_argument("--prebuilt", type=Path, default=None,
                    help="directory holding an already built timestamp build of the three code "
                         "objects (instead of building one)")
    args = ap.parse_args()

    sys.path.insert(0, str(REPO))
    from __graft_entry__ import load_package

    load_package()
    from qwen3_iree_amd import decode as D
    from qwen3_iree_amd import q8gemv as Q

    if args.prebuilt is not None:
        Q.init(str(args.prebuilt / "q8gemv_gfx950.hsaco"))
    else:
        with tempfile.TemporaryDirectory() as td:
            co = build_stamped(Path(td))
            Q.init(co)
    D.set_step_mode(1)
    ctx = args.context
    model = D.DeviceWeights(D.synthetic_weights(seed=20261201, workers=16))
    stream = Q.Stream()
    sess = D.DecodeSession(model, ctx, stream)
    rng = np.random.default_rng(5)
    sess.k_cache.upload(rng.standard_normal((28 * ctx, 1024), dtype=np.float32).astype(np.float16))
    sess.v_cache.upload(rng.standard_normal((28 * ctx, 1024), dtype=np.float32).astype(np.float16))
    sess.set_state(1234, ctx - 1)
    t_end = time.perf_counter() + 0.3
    while time.perf_counter() < t_end:
        sess.step(advance=False, logits=False)
        stream.synchronize()
    e0, e1 = Q.Event(), Q.Event()
    e0.record(stream)
    for _ in range(args.steps):
        sess.step(advance=False, logits=False)
    e1.record(stream)
    e1.synchronize()
    step_us = e0.elapsed_ms(e1) * 1e3 / args.steps
    sess.check_status()
    raw = sess.scratch.download(np.uint32, 16 * 29 * N_POINTS, D.scratch_offset("part"))
    # 32-bit clock reads: unwrap against workgroup 0's first stamp (0 = not reached)
    lo = raw.astype(np.int64).reshape(16, 29, N_POINTS)
    ref = lo[0, 0, 0]
    st = np.where(lo != 0, ref + ((lo - ref + (1 << 31)) % (1 << 32)) - (1 << 31), 0)
    t0 = st[0, 0, 0]

    print(f"# dec_step timeline — context {ctx}, one launch per step\n")
    print("Command (GPU box, repo root):\n\n    python3 qwen3-iree_amd/step_timeline.py "
          f"--context {ctx} --steps {args.steps}\n")
    print(f"Timestamp build: {step_us:.1f} us per step (mean of {args.steps}); times below are "
          "us after the layer's start on workgroup 0 (layers 1..27 averaged; 100 MHz counter, "
          "10 ns ticks).\n")
    layer_len = [(st[0, l + 1, 0] - st[0, l, 0]) * TICK_US for l in range(1, 27)]
    print(f"Layer length on workgroup 0: mean {statistics.mean(layer_len):.2f} us, min "
          f"{min(layer_len):.2f}, max {max(layer_len):.2f}; layers end to end "
          f"{(max(st[:, 27, 12]) - st[0, 0, 0]) * TICK_US:.1f} us; "
          f"vocab phase on workgroup 0 {(st[0, 28, 4] - st[0, 28, 0]) * TICK_US:.1f} us.\n")
    print("| point | " + " | ".join(f"wg {w}" for w in STAMP_WGS) + " |")
    print("|---|" + "---|" * len(STAMP_WGS))
    for k, name in POINTS.items():
        cells = []
        for i in range(len(STAMP_WGS)):
            vals = [(st[i, l, k] - st[0, l, 0]) * TICK_US for l in range(1, 28) if st[i, l, k]]
            cells.append(f"{statistics.mean(vals):.2f}" if vals else "")
        if any(cells):
            print(f"| {k} {name} | " + " | ".join(cells) + " |")
    print()
    print("| vocab point | " + " | ".join(f"wg {w}" for w in STAMP_WGS) + " |")
    print("|---|" + "---|" * len(STAMP_WGS))
    for k, name in VOCAB_POINTS.items():
        cells = [f"{(st[i, 28, k] - st[0, 28, 0]) * TICK_US:.2f}" if st[i, 28, k] else ""
                 for i in range(len(STAMP_WGS))]
        if any(cells):
            print(f"| {k} {name} | " + " | ".join(cells) + " |")
    # the critical path of a layer: each phase's latest completion among the
    # recorded workgroups
    print("\nPer-layer critical path (latest recorded workgroup at each point, layers 1..27):\n")
    prev = 0.0
    for k, name in POINTS.items():
        vals = []
        for l in range(1, 28):
            v = [(st[i, l, k] - st[0, l, 0]) * TICK_US for i in range(len(STAMP_WGS)) if st[i, l, k]]
            if v:
                vals.append(max(v))
        if vals:
            m = statistics.mean(vals)
            print(f"- {name}: {m:.2f} us (+{m - prev:.2f})")
            prev = m
    sess.free()
    model.free()
    stream.destroy()
    Q.teardown()
    return 0


if __name__ == "__main__":
    sys.exit(main())
