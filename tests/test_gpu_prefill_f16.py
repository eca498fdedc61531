"""GPU tests of the f16 layer matrices (qwen3_prefill_matrices_expand) and of
the prompt GEMMs that read them.

- The expanded matrices hold, bit for bit, the oracle's f16 weights of every
  Q8_0 matrix (O.q8_dequant_f16: f16(scale * q), the reference converter's
  values), in the documented row order (q/k/v stacked, gate/up in groups of
  16 gate + 16 up rows).
- The prompt path over the f16 matrices gives the same bits as the prompt
  path over the Q8_0 stacks, in every workspace region and cache row, for
  every tile setting, from one token to past 2048 (where the 128 x 128 tiles
  run) and with attn_o / ffn_down in one, two and many K ranges.  The Q8_0
  route is itself held to the oracle stage by stage in test_gpu_prefill.py,
  so this carries that parity over to the f16 route.
"""
from __future__ import annotations

import numpy as np
import pytest

from test_gpu_decode import fill_cache_layer

pytestmark = pytest.mark.gpu

LAYER_ELEMS = 15_728_640


@pytest.fixture(scope="module")
def D():
    from qwen3_iree_amd import decode

    return decode


@pytest.fixture(scope="module")
def dmodel(gpu, D, model_host):
    m = D.DeviceWeights(model_host, prefill_f16=True)
    yield m
    m.free()


def gu_order(j_rows: int = 3072) -> np.ndarray:
    """Source row (gate 0..3071, up 3072..6143) of each row of the f16
    gate/up matrix."""
    r = np.arange(2 * j_rows)
    grp, within = r // 32, r % 32
    return np.where(within < 16, 16 * grp + within, j_rows + 16 * grp + within - 16)


@pytest.mark.parametrize("layer", [0, 27])
def test_prefill_matrices_are_the_f16_weights(O, gpu, D, dmodel, model_host, layer):
    print(f"prefill matrices layer {layer}", flush=True)
    assert D.prefill_matrices_bytes() == 28 * LAYER_ELEMS * 2
    got = dmodel.prefill_matrices.download(np.float16, LAYER_ELEMS, layer * LAYER_ELEMS * 2)
    hw = model_host
    qkv = np.concatenate([O.q8_dequant_f16(hw.wq[layer], 2048, 1024),
                          O.q8_dequant_f16(hw.wk[layer], 1024, 1024),
                          O.q8_dequant_f16(hw.wv[layer], 1024, 1024)])
    o = O.q8_dequant_f16(hw.wo[layer], 1024, 2048)
    gu = O.q8_dequant_f16(hw.wgu[layer], 6144, 1024)[gu_order()]
    dn = O.q8_dequant_f16(hw.wdn[layer], 1024, 3072)
    want = np.concatenate([qkv.ravel(), o.ravel(), gu.ravel(), dn.ravel()])
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_gu_order_pairs_gate_and_up():
    """Row 32 G + i (i < 16) is gate row 16 G + i and row 32 G + 16 + i the
    up row of the same SwiGLU output."""
    order = gu_order()
    assert sorted(order.tolist()) == list(range(6144))
    for grp in (0, 1, 95):
        for i in (0, 7, 15):
            assert order[32 * grp + i] == 16 * grp + i
            assert order[32 * grp + 16 + i] == 3072 + 16 * grp + i


def run_layer(D, dmodel, sess, n, p0, h_in, f16: bool, rows: int):
    dmodel.use_prefill_matrices(f16)
    D.set_prefill_tiling(rows, 0)
    try:
        g = sess.prefill_layer(5, h_in, p0, False)
    finally:
        D.set_prefill_tiling(0, 0)
        dmodel.use_prefill_matrices(True)
    return g, sess.cache_rows(5, 0, sess.max_seq)


@pytest.mark.parametrize("n,p0", [(1, 0), (45, 3), (300, 0), (600, 0), (1030, 0), (2100, 7)])
def test_prefill_f16_route_bit_identical_to_q8_route(gpu, D, dmodel, n, p0):
    """Every region and cache row: Q8_0 route (default tile) == f16 route at
    tile rows 0 (by shape), 32, 64 and 128."""
    rng = np.random.default_rng(9300 + n)
    max_seq = p0 + n + 8
    sess = D.DecodeSession(dmodel, max_seq)
    try:
        kc = np.zeros((28 * max_seq, 1024), np.float16)
        vc = np.zeros_like(kc)
        fill_cache_layer(sess, 5, p0, rng, kc, vc)
        h_in = (1.5 * rng.standard_normal((n, 1024))).astype(np.float16)
        print(f"prefill q8 route n {n} p0 {p0}", flush=True)
        ref, ref_cache = run_layer(D, dmodel, sess, n, p0, h_in, False, 0)
        for rows in (0, 32, 64, 128):
            print(f"prefill f16 route n {n} p0 {p0} rows {rows}", flush=True)
            got, cache = run_layer(D, dmodel, sess, n, p0, h_in, True, rows)
            for name in ref:
                assert np.array_equal(got[name].view(np.uint16), ref[name].view(np.uint16)), \
                    (rows, name)
            for a, b in zip(cache, ref_cache):
                assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), rows
    finally:
        sess.free()


def test_prefill_batched_f16_route_matches_q8_route(gpu, D, dmodel):
    """A 2100-token prompt from position 0 through all 28 layers: the same
    token, logits and cache on both routes."""
    rng = np.random.default_rng(77)
    n = 2100
    prompt = rng.integers(0, 151936, n, dtype=np.int32)
    res = []
    for f16 in (False, True):
        print(f"prefill batched {n} tokens f16 {f16}", flush=True)
        dmodel.use_prefill_matrices(f16)
        sess = D.DecodeSession(dmodel, n + 4)
        try:
            sess.set_state(0, 0)
            sess.prefill_batched(prompt, logits=True)
            tok, pos = sess.get_state()
            logits = sess.read_logits()
            k, v = sess.cache_rows(27, 0, n)
            res.append((tok, pos, logits, k, v))
        finally:
            sess.free()
            dmodel.use_prefill_matrices(True)
    (ta, pa, la, ka, va), (tb, pb, lb, kb, vb) = res
    assert (ta, pa) == (tb, pb)
    assert pa == n
    for a, b in ((la, lb), (ka, kb), (va, vb)):
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_prefill_matrices_expand_validates(gpu, D, dmodel):
    from qwen3_iree_amd import q8gemv as Q

    buf = dmodel.prefill_matrices
    with pytest.raises(Q.Q8GemvError, match="bytes"):
        Q._call("qwen3_prefill_matrices_expand", dmodel.ref(), buf.ptr,
                D.prefill_matrices_bytes() - 1, None)
    with pytest.raises(Q.Q8GemvError, match="null"):
        Q._call("qwen3_prefill_matrices_expand", dmodel.ref(), None,
                D.prefill_matrices_bytes(), None)
    with pytest.raises(Q.Q8GemvError, match="aligned"):
        Q._call("qwen3_prefill_matrices_expand", dmodel.ref(), buf.ptr + 16,
                D.prefill_matrices_bytes(), None)
