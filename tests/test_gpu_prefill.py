"""GPU parity of the batched prompt path (qwen3_prefill_batched /
qwen3_prefill_layer) against the oracle and against the decode steps.

One layer over n tokens is checked stage by stage, each stage against the
oracle applied to the GPU's own input of that stage (the workspace keeps every
intermediate), with the decode step's tolerances:

  xn, fn        rms_norm per token row         within 1 f16 ulp
  q, k, v       GEMM rows over the f16 weights GEMV rule per row (2 ulp / 1e-3)
                @prefill reads (f16(scale * q))
  q_roped, K    head norm + RoPE at p0 + i     2 ulp + one input ulp
  V slots       raw v                          bit-exact
  attn          causal attention over the GPU  2 ulp + 1e-5
                cache, slots [lo, p0 + i]
  res, h        GEMM + f16 residual add        propagated GEMV rule
  act           gate_up GEMM + SwiGLU          propagated GEMV rule + 4 ulp

(the GEMM references are the oracle's f16 GEMV over O.q8_dequant_f16 of the
layer's Q8_0 matrix: the decode GEMVs scale each block's exact dot instead,
as the reference's decode kernels do, so the two paths differ by the weights'
f16 rounding, well inside the whole-path tolerances below)

then the layer's output against the oracle's decode layer run token by token
(relative L2), and the whole prompt path against the decode-step prompt path
and the oracle's steps (logits, token, every cache row).
"""
from __future__ import annotations

import numpy as np
import pytest

from test_gpu_decode import assert_norm_close, f64, fill_cache_layer, rope_tol, ulp

pytestmark = pytest.mark.gpu

MAX_SEQ = 512


def assert_gemm(O, W16, x, got, what):
    """One GEMM row against the oracle's f16 GEMV of the same f16 weights."""
    ref = O.f16_gemv(W16, x)
    _, mag = O.f16_gemv_f64(W16, x)
    rep = O.gemv_tolerance_report(got, ref, mag)
    assert rep["fail"] == 0, (what, rep)


def assert_gemm_add(O, base, W16, x, got, what):
    """got = f16(base + f16(W x)): the GEMV rule carried through one f16 add."""
    o_ref = O.f16_gemv(W16, x)
    _, mag = O.f16_gemv_f64(W16, x)
    want = O.add_f16(base, o_ref)
    tol = (ulp(O, want) + 2 * ulp(O, o_ref) + 1e-3 * np.abs(f64(o_ref))
           + 8 * 2.0 ** -24 * mag)
    d = np.abs(f64(got) - f64(want))
    assert (d <= tol).all(), (what, np.flatnonzero(d > tol)[:8], d.max())


@pytest.fixture(scope="module")
def D():
    from qwen3_iree_amd import decode

    return decode


@pytest.fixture(scope="module")
def dmodel(gpu, D, model_host):
    m = D.DeviceWeights(model_host)
    yield m
    m.free()


@pytest.mark.parametrize("layer,n,p0,chunk_local", [
    (0, 1, 0, False), (3, 37, 0, False), (11, 64, 5, False), (27, 130, 40, False),
    (7, 20, 9, True), (16, 65, 0, True),
    (20, 500, 0, False)])  # attn_o / ffn_down with K split in two
def test_prefill_layer_stages(O, gpu, D, dmodel, model_host, layer, n, p0, chunk_local):
    w = model_host
    rng = np.random.default_rng(7000 + 100 * layer + n)
    sess = D.DecodeSession(dmodel, MAX_SEQ)
    kc = np.zeros((28 * MAX_SEQ, 1024), np.float16)
    vc = np.zeros_like(kc)
    fill_cache_layer(sess, layer, p0, rng, kc, vc)
    h_in = (1.5 * rng.standard_normal((n, 1024))).astype(np.float16)
    print(f"prefill layer {layer} n {n} p0 {p0} chunk_local {chunk_local}", flush=True)
    g = sess.prefill_layer(layer, h_in, p0, chunk_local)
    k_rows, v_rows = sess.cache_rows(layer, 0, MAX_SEQ)
    lo = p0 if chunk_local else 0
    wq, wk, wv = (O.q8_dequant_f16(m[layer], nr, 1024)
                  for m, nr in ((w.wq, 2048), (w.wk, 1024), (w.wv, 1024)))
    wo = O.q8_dequant_f16(w.wo[layer], 1024, 2048)
    wgu = O.q8_dequant_f16(w.wgu[layer], 6144, 1024)
    wdn = O.q8_dequant_f16(w.wdn[layer], 1024, 3072)

    for i in range(n):
        pos = p0 + i
        assert_norm_close(O, g["xn"][i], O.rmsnorm(h_in[i], w.attn_norm[layer]), ("xn", i))
        assert_gemm(O, wq, g["xn"][i], g["q"][i], ("q", i))
        assert_gemm(O, wk, g["xn"][i], g["k"][i], ("k", i))
        assert_gemm(O, wv, g["xn"][i], g["v"][i], ("v", i))
        qn = O.head_rmsnorm(g["q"][i], w.q_norm[layer])
        q_want = O.rope(qn, pos)
        assert (np.abs(f64(g["q_roped"][i]) - f64(q_want)) <= rope_tol(O, qn, q_want)).all(), i
        kn = O.head_rmsnorm(g["k"][i], w.k_norm[layer])
        k_want = O.rope(kn, pos)
        assert (np.abs(f64(k_rows[pos]) - f64(k_want)) <= rope_tol(O, kn, k_want)).all(), i
        assert np.array_equal(v_rows[pos].view(np.uint16), g["v"][i].view(np.uint16)), i
        a_want = O.attention(g["q_roped"][i], k_rows[lo:pos + 1], v_rows[lo:pos + 1])
        d = np.abs(f64(g["attn"][i]) - f64(a_want))
        assert (d <= 2 * ulp(O, a_want) + 1e-5).all(), (i, d.max())
        assert_gemm_add(O, h_in[i], wo, g["attn"][i], g["res"][i], ("res", i))
        assert_norm_close(O, g["fn"][i], O.rmsnorm(g["res"][i], w.ffn_norm[layer]), ("fn", i))
        gu = O.f16_gemv(wgu, g["fn"][i])
        _, gmag = O.f16_gemv_f64(wgu, g["fn"][i])
        act_want = O.swiglu(gu[:3072], gu[3072:])
        dg = 2 * ulp(O, gu) + 1e-3 * np.abs(f64(gu)) + 8 * 2.0 ** -24 * gmag
        gate, up = f64(gu[:3072]), f64(gu[3072:])
        silu = gate / (1 + np.exp(-gate))
        tol = 1.1 * np.abs(up) * dg[:3072] + np.abs(silu) * dg[3072:] + 4 * ulp(O, act_want)
        d = np.abs(f64(g["act"][i]) - f64(act_want))
        assert (d <= tol).all(), (i, np.flatnonzero(d > tol)[:8], d.max())
        assert_gemm_add(O, g["res"][i], wdn, g["act"][i], g["h"][i], ("h", i))

    # slots outside [p0, p0 + n) untouched
    base = layer * MAX_SEQ
    assert np.array_equal(k_rows[:p0], kc[base:base + p0])
    assert np.array_equal(v_rows[:p0], vc[base:base + p0])
    assert not k_rows[p0 + n:].any() and not v_rows[p0 + n:].any()

    if not chunk_local or p0 == 0:
        # the layer against the oracle's decode layer, token after token
        h_ref = np.empty_like(h_in)
        for i in range(n):
            h_ref[i], _ = O.decode_layer(w, layer, kc, vc, MAX_SEQ, p0 + i, h_in[i])
        rel = np.linalg.norm(f64(g["h"]) - f64(h_ref)) / np.linalg.norm(f64(h_ref))
        assert rel < 5e-3, rel
    sess.free()


def _steps_logits(D, dmodel, prompt, p0_prompt=None):
    """The decode-step path: prompt[:-1] as steps, the last token as a step
    with logits.  Returns (session, logits)."""
    sess = D.DecodeSession(dmodel, MAX_SEQ)
    sess.set_state(0, 0)
    if p0_prompt is not None:
        sess.prefill(p0_prompt)
    start = sess.get_state()[1]
    if len(prompt) > 1:
        sess.prefill(prompt[:-1])
    sess.set_state(int(prompt[-1]), start + len(prompt) - 1)
    sess.step(advance=True, logits=True)
    return sess, sess.read_logits()


def _compare_sessions(a, b, la, lb, n_slots):
    dl = np.abs(f64(la) - f64(lb))
    assert np.linalg.norm(dl) / np.linalg.norm(f64(lb)) < 2e-2
    srt = np.sort(f64(lb))
    ta, tb = a.get_state()[0], b.get_state()[0]
    if srt[-1] - srt[-2] > 2 * dl.max():
        assert ta == tb, (ta, tb, srt[-1] - srt[-2], dl.max())
    assert a.get_state()[1] == b.get_state()[1]
    for layer in range(28):
        ka, va = a.cache_rows(layer, 0, n_slots)
        kb, vb = b.cache_rows(layer, 0, n_slots)
        for x, y in ((ka, kb), (va, vb)):
            rel = np.linalg.norm(f64(x) - f64(y)) / np.linalg.norm(f64(y))
            assert rel < 2e-2, (layer, rel)


@pytest.mark.parametrize("n", [1, 7, 45])
def test_prefill_batched_matches_decode_steps(gpu, D, dmodel, n):
    rng = np.random.default_rng(50 + n)
    prompt = rng.integers(0, D.VOCAB, n).astype(np.int32)
    print(f"prefill batched n {n}", flush=True)
    a = D.DecodeSession(dmodel, MAX_SEQ)
    a.set_state(0, 0)
    a.prefill_batched(prompt, logits=True)
    la = a.read_logits()
    assert a.get_state()[1] == n and a.status() == 0
    # token = lowest index of the maximal f16 logit
    lf = la.astype(np.float32)
    assert a.get_state()[0] == int(np.flatnonzero(lf == lf.max())[0])
    b, lb = _steps_logits(D, dmodel, prompt)
    _compare_sessions(a, b, la, lb, n)
    a.free()
    b.free()


@pytest.mark.parametrize("n", [45, 500, 1100])
def test_prefill_batched_equals_layer_by_layer(gpu, D, dmodel, model_host, n):
    """The whole-prompt call forms each next layer's attention norm inside
    ffn_down's reduce (pf_res_reduce_norm; K split in many ranges at 45
    tokens, in two at 500, one range at 1100); layer by layer
    (qwen3_prefill_layer) runs pf_rmsnorm instead.  Every layer's k/v slots
    depend on that norm, so they must agree bit for bit."""
    rng = np.random.default_rng(900 + n)
    prompt = rng.integers(0, D.VOCAB, n).astype(np.int32)
    print(f"prefill batched vs layers n {n}", flush=True)
    max_seq = max(MAX_SEQ, n)
    a = D.DecodeSession(dmodel, max_seq)
    a.set_state(0, 0)
    a.prefill_batched(prompt)
    b = D.DecodeSession(dmodel, max_seq)
    h = model_host.token_embd[prompt]
    for layer in range(28):
        h = b.prefill_layer(layer, h, 0)["h"]
        ka, va = a.cache_rows(layer, 0, n)
        kb, vb = b.cache_rows(layer, 0, n)
        assert np.array_equal(ka.view(np.uint16), kb.view(np.uint16)), layer
        assert np.array_equal(va.view(np.uint16), vb.view(np.uint16)), layer
    a.free()
    b.free()


def test_prefill_batched_matches_oracle_steps(O, gpu, D, dmodel, model_host):
    w = model_host
    prompt = np.array([151643, 9707, 11, 1879, 0, 151935], np.int32)
    sess = D.DecodeSession(dmodel, MAX_SEQ)
    sess.set_state(0, 0)
    sess.prefill_batched(prompt, logits=True)
    logits = sess.read_logits()
    kc = np.zeros((28 * MAX_SEQ, 1024), np.float16)
    vc = np.zeros_like(kc)
    for i, t in enumerate(prompt):
        ref_tok, ref_logits, _ = O.decode_step(w, kc, vc, MAX_SEQ, int(t), i, True)
    dl = np.abs(f64(logits) - f64(ref_logits))
    assert np.linalg.norm(dl) / np.linalg.norm(f64(ref_logits)) < 2e-2
    srt = np.sort(f64(ref_logits))
    if srt[-1] - srt[-2] > 2 * dl.max():
        assert sess.get_state()[0] == ref_tok
    for layer in (0, 13, 27):
        k, v = sess.cache_rows(layer, 0, len(prompt))
        base = layer * MAX_SEQ
        for x, y in ((k, kc[base:base + len(prompt)]), (v, vc[base:base + len(prompt)])):
            assert np.linalg.norm(f64(x) - f64(y)) / np.linalg.norm(f64(y)) < 2e-2
    sess.free()


def test_prefill_batched_continues_a_sequence(gpu, D, dmodel):
    """A second prompt after a first one attends to the whole cache (the
    decode steps' semantics)."""
    rng = np.random.default_rng(77)
    first = rng.integers(0, D.VOCAB, 10).astype(np.int32)
    second = rng.integers(0, D.VOCAB, 13).astype(np.int32)
    a = D.DecodeSession(dmodel, MAX_SEQ)
    a.set_state(0, 0)
    a.prefill_batched(first)
    a.prefill_batched(second, logits=True)
    la = a.read_logits()
    assert a.get_state()[1] == 23
    b, lb = _steps_logits(D, dmodel, second, p0_prompt=first)
    _compare_sessions(a, b, la, lb, 23)
    a.free()
    b.free()


def test_prefill_batched_chunk_local_ignores_history(gpu, D, dmodel):
    """chunk_local: a prompt at p0 > 0 gives what the same prompt gives at
    position 0 in a fresh cache, up to RoPE's position dependence, which
    cancels in q.k for equal relative offsets: the logits match."""
    rng = np.random.default_rng(78)
    hist = rng.integers(0, D.VOCAB, 9).astype(np.int32)
    prompt = rng.integers(0, D.VOCAB, 11).astype(np.int32)
    a = D.DecodeSession(dmodel, MAX_SEQ)
    a.set_state(0, 0)
    a.prefill_batched(hist)
    a.prefill_batched(prompt, chunk_local=True, logits=True)
    la = a.read_logits()
    b = D.DecodeSession(dmodel, MAX_SEQ)
    b.set_state(0, 0)
    b.prefill_batched(prompt, logits=True)
    lb = b.read_logits()
    rel = np.linalg.norm(f64(la) - f64(lb)) / np.linalg.norm(f64(lb))
    assert rel < 2e-2, rel
    # and it differs from attending to the history
    c = D.DecodeSession(dmodel, MAX_SEQ)
    c.set_state(0, 0)
    c.prefill_batched(hist)
    c.prefill_batched(prompt, logits=True)
    lc = c.read_logits()
    assert np.linalg.norm(f64(lc) - f64(lb)) / np.linalg.norm(f64(lb)) > 2e-2
    for s in (a, b, c):
        s.free()


def test_prefill_batched_cache_edges(gpu, D, dmodel):
    from qwen3_iree_amd import q8gemv as Q

    sess = D.DecodeSession(dmodel, 16)
    sess.set_state(0, 6)
    sess.prefill_batched(np.arange(10, dtype=np.int32))  # fills slots 6..15
    tok, pos = sess.get_state()
    assert pos == 15 and sess.status() & 1 and 0 <= tok < D.VOCAB
    sess.set_state(0, 7)
    with pytest.raises(Q.Q8GemvError, match="exceed max_seq"):
        sess.prefill_batched(np.arange(10, dtype=np.int32))
    sess.free()


@pytest.mark.parametrize("n,p0", [(45, 3), (300, 0), (600, 0), (1030, 0)])
def test_prefill_tile_rows_bit_identical(gpu, D, dmodel, n, p0):
    """The 32- and 64-token GEMM tiles give the same bits in every stage
    (attn_o / ffn_down with K in many ranges at 45 and 300 tokens, in two at
    600, in one range through the reduce at 1030)."""
    rng = np.random.default_rng(9100 + n)
    max_seq = max(MAX_SEQ, p0 + n)
    sess = D.DecodeSession(dmodel, max_seq)
    kc = np.zeros((28 * max_seq, 1024), np.float16)
    vc = np.zeros_like(kc)
    fill_cache_layer(sess, 5, p0, rng, kc, vc)
    h_in = (1.5 * rng.standard_normal((n, 1024))).astype(np.float16)
    outs = []
    try:
        for rows in (32, 64, 0):
            print(f"prefill tile rows {rows} n {n} p0 {p0}", flush=True)
            D.set_prefill_tiling(rows, 0)
            g = sess.prefill_layer(5, h_in, p0, False)
            outs.append((g, sess.cache_rows(5, 0, max_seq)))
    finally:
        D.set_prefill_tiling(0, 0)
    (g32, c32), (g64, c64), (ga, ca) = outs
    for name in g32:
        assert np.array_equal(g32[name].view(np.uint16), g64[name].view(np.uint16)), name
        assert np.array_equal(g32[name].view(np.uint16), ga[name].view(np.uint16)), name
    for a, b in zip(c32, c64):
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    with pytest.raises(Exception):
        D.set_prefill_tiling(48, 0)
    with pytest.raises(Exception):
        D.set_prefill_tiling(0, -1)
    sess.free()


@pytest.mark.parametrize("split", [1, 2, 5, 1000])
def test_prefill_attention_splits(O, gpu, D, dmodel, split):
    """Every division of the cache positions into splits (merged by the last
    split of a query block) gives the attention within its tolerance."""
    n, p0, layer = 100, 50, 9
    rng = np.random.default_rng(9300 + split)
    sess = D.DecodeSession(dmodel, MAX_SEQ)
    kc = np.zeros((28 * MAX_SEQ, 1024), np.float16)
    vc = np.zeros_like(kc)
    fill_cache_layer(sess, layer, p0, rng, kc, vc)
    h_in = (1.5 * rng.standard_normal((n, 1024))).astype(np.float16)
    try:
        for chunk_local in (False, True):
            print(f"prefill attention split {split} chunk_local {chunk_local}", flush=True)
            D.set_prefill_tiling(0, split)
            g = sess.prefill_layer(layer, h_in, p0, chunk_local)
            k_rows, v_rows = sess.cache_rows(layer, 0, MAX_SEQ)
            lo = p0 if chunk_local else 0
            for i in range(n):
                pos = p0 + i
                a_want = O.attention(g["q_roped"][i], k_rows[lo:pos + 1], v_rows[lo:pos + 1])
                d = np.abs(f64(g["attn"][i]) - f64(a_want))
                assert (d <= 2 * ulp(O, a_want) + 1e-5).all(), (chunk_local, i, d.max())
    finally:
        D.set_prefill_tiling(0, 0)
    sess.free()


@pytest.mark.parametrize("chunk_local", [False, True])
def test_prefill_long_history(O, gpu, D, dmodel, chunk_local):
    """Three tokens after 30,000 cached positions: with the default split of
    256 positions a query block would need 118 (block, split) pairs, more
    than the workspace's partial slots hold, so the split is raised; the
    attention still matches the oracle over the whole history."""
    n, p0, layer, max_seq = 3, 30000, 3, 30016
    rng = np.random.default_rng(9400)
    sess = D.DecodeSession(dmodel, max_seq)
    k = rng.standard_normal((p0, 1024)).astype(np.float16)
    v = (0.6 * rng.standard_normal((p0, 1024))).astype(np.float16)
    base = layer * max_seq
    sess.k_cache.upload(k, base * 2048)
    sess.v_cache.upload(v, base * 2048)
    h_in = (1.5 * rng.standard_normal((n, 1024))).astype(np.float16)
    print(f"prefill long history p0 {p0} chunk_local {chunk_local}", flush=True)
    g = sess.prefill_layer(layer, h_in, p0, chunk_local)
    k_rows, v_rows = sess.cache_rows(layer, 0, p0 + n)
    assert np.array_equal(k_rows[:p0], k) and np.array_equal(v_rows[:p0], v)
    lo = p0 if chunk_local else 0
    for i in range(n):
        a_want = O.attention(g["q_roped"][i], k_rows[lo:p0 + i + 1], v_rows[lo:p0 + i + 1])
        d = np.abs(f64(g["attn"][i]) - f64(a_want))
        assert (d <= 2 * ulp(O, a_want) + 1e-5).all(), (i, d.max())
    sess.free()
