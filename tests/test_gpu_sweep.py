"""The benchmark's headline workload under test: the 28-layer stacked
cold-cache Q8_0 GEMV sweep (five stacked weight sets, 140 GEMVs in the
per-layer order q, kv, o, gate_up, dn of model/qwen3_full.mlir:751-864 for
layers 0..27, model/qwen3_full.mlir:1445-1449), built by the same code
bench.py times (qwen3_iree_amd.sweep, the bench's seed).

Every one of the 315,392 outputs of one batched launch is held to the GEMV
rule against the oracle (|gpu - ref| <= 2 f16 ulp or 1e-3 relative, ref in
the reference kernels' f32 order; outputs whose reference cancels to the f32
noise floor may pass on that floor, at most 1 in 2000), one entry of each kind
is bit-identical to the single-GEMV dispatch of the drop-in entry point, and
the 140 stream-ordered dispatches (the reference's granularity) give the same
bits as the batched launch.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BENCH_SEED = 20261201  # bench.py's SEED: the timed workload itself


@pytest.fixture(scope="module")
def sweep(gpu):
    from qwen3_iree_amd import sweep as S

    sw = S.build(BENCH_SEED)
    yield sw
    sw.free()


def test_sweep_table_is_the_configured_workload(gpu, sweep):
    Q = gpu
    assert len(sweep.order) == 140
    assert [d.name for _, d in sweep.order[:5]] == ["attn_q", "attn_kv", "attn_o", "gate_up",
                                                    "ffn_dn"]
    assert [layer for layer, _ in sweep.order[::5]] == list(range(28))
    assert sweep.weight_bytes == 436_731_904
    assert sweep.bytes_per_step == 437_821_440
    assert sweep.outputs == 315_392
    for d in Q.Q8_KINDS:
        assert sweep.host_w[d.kind].shape == (28, d.bytes_per_layer)


def test_batched_sweep_matches_oracle_every_output(gpu, O, sweep):
    Q = gpu
    batch = sweep.batch()
    try:
        for y in sweep.dev_y.values():
            y.fill(0xFF)  # NaN pattern: an output the launch missed cannot pass
        print("batched sweep: one launch of 140 GEMVs", flush=True)
        batch.launch()
        Q.synchronize()
    finally:
        batch.free()
    fails = floor = 0
    worst = []
    for layer, d in sweep.order:
        got = sweep.dev_y[(layer, d.kind)].download(np.float16)
        raw = sweep.host_w[d.kind][layer]
        x = sweep.host_x[(layer, d.kind)]
        rep = O.gemv_tolerance_report(got, O.q8_gemv(raw, d.n, d.k, x),
                                      O.q8_gemv_f64(raw, d.n, d.k, x)[1])
        fails += rep["fail"]
        floor += rep["on_floor"]
        if rep["fail"]:
            worst.append((layer, d.name, rep))
    assert fails == 0, worst[:4]
    assert floor <= sweep.outputs // 2000, floor


def test_batched_sweep_bit_identical_to_single_dispatches(gpu, sweep):
    Q = gpu
    batch = sweep.batch()
    try:
        batch.launch()
        Q.synchronize()
    finally:
        batch.free()
    picks = [(3, Q.ATTN_Q), (11, Q.ATTN_KV), (17, Q.ATTN_O), (24, Q.GATE_UP), (27, Q.FFN_DN)]
    batched = {(l, d.kind): sweep.dev_y[(l, d.kind)].download(np.uint16) for l, d in picks}
    for layer, d in picks:
        y = Q.DeviceBuffer(2 * d.n)
        try:
            print(f"single dispatch {d.export} layer {layer}", flush=True)
            Q.decode_dispatch(d.ordinal, sweep.dev_w[d.kind], layer, sweep.dev_x[(layer, d.kind)], y)
            Q.synchronize()
            assert np.array_equal(y.download(np.uint16), batched[(layer, d.kind)]), (layer, d.name)
        finally:
            y.free()


def test_per_dispatch_sweep_bit_identical_to_batched(gpu, sweep):
    """The 140 dispatches in sweep order, replayed from a hipGraph as the
    benchmark does, leave the same bits as the batched launch."""
    Q = gpu
    batch = sweep.batch()
    try:
        batch.launch()
        Q.synchronize()
    finally:
        batch.free()
    want = {key: y.download(np.uint16) for key, y in sweep.dev_y.items()}
    for y in sweep.dev_y.values():
        y.fill(0xFF)
    stream = Q.Stream()
    graph = Q.Graph(stream, lambda: sweep.record_dispatches(stream))
    try:
        print("per-dispatch sweep: hipGraph of 140 launches, 2 replays", flush=True)
        graph.launch(stream)
        graph.launch(stream)
        stream.synchronize()
    finally:
        graph.destroy()
        stream.destroy()
    for key, y in sweep.dev_y.items():
        assert np.array_equal(y.download(np.uint16), want[key]), key
