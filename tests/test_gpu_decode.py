"""GPU parity of the decode step (include/qwen3_decode.h) against the oracle.

Every stage of a layer is checked against the oracle applied to the GPU's own
input of that stage (the kernels leave their intermediates in the scratch), so
each check isolates one kernel:

  xn, fn, on   rms_norm                    within 1 f16 ulp
  q, k, v      Q8_0 GEMV of the GPU's xn   GEMV rule (2 ulp / 1e-3, noise floor)
  q_roped, K   head norm + RoPE            2 ulp + one input ulp
  V slot       raw v                       bit-exact
  attn         attention over the GPU cache 2 ulp + 1e-5
  res, h_out   GEMV + f16 residual add     propagated GEMV rule
  act          gate_up GEMV + SwiGLU       propagated GEMV rule + 4 ulp
  logits       vocab GEMV of the GPU's on  GEMV rule
  token        argmax of the GPU's logits  bit-exact (lowest index)

The whole layer and the whole step are then compared with the oracle's own
chain: relative L2 error of the hidden state, the logits, and the token
whenever the oracle's top-2 margin exceeds the logit deviation.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAX_SEQ = 1024


@pytest.fixture(scope="module")
def D():
    from qwen3_iree_amd import decode

    return decode


@pytest.fixture(scope="module")
def dmodel(gpu, D, model_host):
    m = D.DeviceWeights(model_host)
    yield m
    m.free()


def ulp(O, v):
    return O.ulp_f16(np.asarray(v, np.float64))


def f64(a):
    return np.asarray(a, np.float64)


def assert_norm_close(O, got, want, what):
    d = np.abs(f64(got) - f64(want))
    ok = d <= ulp(O, want)
    assert ok.all(), (what, np.flatnonzero(~ok)[:8], d.max())


def assert_gemv(O, w_layer, n, k, x, got, what):
    ref = O.q8_gemv(w_layer, n, k, x)
    _, mag = O.q8_gemv_f64(w_layer, n, k, x)
    rep = O.gemv_tolerance_report(got, ref, mag)
    assert rep["fail"] == 0, (what, rep)
    return ref, mag


def assert_gemv_add(O, base, w_layer, n, k, x, got, what):
    """got = f16(base + f16(W x)): the GEMV rule carried through one f16 add."""
    o_ref = O.q8_gemv(w_layer, n, k, x)
    _, mag = O.q8_gemv_f64(w_layer, n, k, x)
    want = O.add_f16(base, o_ref)
    tol = (ulp(O, want) + 2 * ulp(O, o_ref) + 1e-3 * np.abs(f64(o_ref))
           + 8 * 2.0 ** -24 * mag)
    d = np.abs(f64(got) - f64(want))
    assert (d <= tol).all(), (what, np.flatnonzero(d > tol)[:8], d.max())


def rope_tol(O, normed, want):
    """2 ulp of the result plus one ulp of the head's largest input (a 1-ulp
    difference of one normalised input moves the output by at most that)."""
    hmax = np.abs(f64(normed)).reshape(-1, 128).max(axis=1)
    return 2 * ulp(O, want) + np.repeat(ulp(O, hmax), 128)


def rope_tol_far(O, normed, want, pos):
    """rope_tol plus the spread of two correct f32 evaluations of the angle
    at a large position: theta = f32(pos) * powf(1e6, -2i/128) carries up to
    ~2 ulp of powf and 0.5 ulp of the product in each library, so two
    evaluations may differ by about 2^-21 theta (0.01 rad at theta = 2e4),
    which moves an output by up to (|x_d| + |x_d+-64|) times that."""
    x = np.abs(f64(normed)).reshape(-1, 128)
    i = np.arange(128) % 64
    theta = float(pos) * 1e6 ** (-(2.0 * i) / 128.0)
    pair = x + np.concatenate([x[:, 64:], x[:, :64]], axis=1)
    return rope_tol(O, normed, want) + (pair * theta * 2.0 ** -21).reshape(-1)


def fill_cache_layer(sess, layer, n, rng, kc, vc):
    """Random history in slots [0, n) of `layer`, on the device and in the
    host copies kc / vc ([28 * max_seq, 1024])."""
    if n == 0:
        return
    k = rng.standard_normal((n, 1024)).astype(np.float16)
    v = (0.6 * rng.standard_normal((n, 1024))).astype(np.float16)
    base = layer * sess.max_seq
    kc[base:base + n] = k
    vc[base:base + n] = v
    sess.k_cache.upload(k, base * 2048)
    sess.v_cache.upload(v, base * 2048)


def test_layer_attention_long_context(O, gpu, D, dmodel, model_host):
    """One layer at position 20,000 (each of the 32 position splits walks 20
    chunks of 32 cached rows): head norms + RoPE (within the spread of two f32
    evaluations of the angle at that position), the cache write, and the
    attention over the GPU's own cache against the oracle."""
    Q = gpu
    w = model_host
    layer, pos, max_seq = 9, 20000, 20008
    rng = np.random.default_rng(4242)
    sess = D.DecodeSession(dmodel, max_seq)
    k = rng.standard_normal((pos, 1024)).astype(np.float16)
    v = (0.6 * rng.standard_normal((pos, 1024))).astype(np.float16)
    sess.k_cache.upload(k, layer * max_seq * 2048)
    sess.v_cache.upload(v, layer * max_seq * 2048)
    h_in = (1.5 * rng.standard_normal(1024)).astype(np.float16)
    hin, hout = Q.DeviceBuffer.from_array(h_in), Q.DeviceBuffer(2048)
    sess.set_state(0, pos)
    print(f"decode layer {layer} pos {pos}", flush=True)
    sess.layer(layer, hin, hout)
    g = {name: sess.scratch_f16(name, n) for name, n in
         (("q", 2048), ("k", 1024), ("v", 1024), ("q_roped", 2048), ("attn", 2048))}
    k_rows, v_rows = sess.cache_rows(layer, 0, pos + 1)
    assert np.array_equal(k_rows[:pos], k) and np.array_equal(v_rows[:pos], v)
    qn = O.head_rmsnorm(g["q"], w.q_norm[layer])
    q_want = O.rope(qn, pos)
    dq = np.abs(f64(g["q_roped"]) - f64(q_want))
    assert (dq <= rope_tol_far(O, qn, q_want, pos)).all(), dq.max()
    kn = O.head_rmsnorm(g["k"], w.k_norm[layer])
    k_want = O.rope(kn, pos)
    dk = np.abs(f64(k_rows[pos]) - f64(k_want))
    assert (dk <= rope_tol_far(O, kn, k_want, pos)).all(), dk.max()
    assert np.array_equal(v_rows[pos].view(np.uint16), g["v"].view(np.uint16))
    # attention over the GPU's own cache with the GPU's roped q
    a_want = O.attention(g["q_roped"], k_rows, v_rows)
    d = np.abs(f64(g["attn"]) - f64(a_want))
    assert (d <= 2 * ulp(O, a_want) + 1e-5).all(), d.max()
    hin.free()
    hout.free()
    sess.free()


@pytest.mark.parametrize("layer,pos", [(0, 0), (5, 5), (13, 31), (27, 32), (2, 33),
                                       (20, 1023)])
def test_layer_stages(O, gpu, D, dmodel, model_host, layer, pos):
    Q = gpu
    w = model_host
    rng = np.random.default_rng(1000 * layer + pos)
    sess = D.DecodeSession(dmodel, MAX_SEQ)
    kc = np.zeros((28 * MAX_SEQ, 1024), np.float16)
    vc = np.zeros_like(kc)
    fill_cache_layer(sess, layer, pos, rng, kc, vc)
    h_in = (1.5 * rng.standard_normal(1024)).astype(np.float16)
    hin, hout = Q.DeviceBuffer.from_array(h_in), Q.DeviceBuffer(2048)
    sess.set_state(0, pos)
    print(f"decode layer {layer} pos {pos}", flush=True)
    sess.layer(layer, hin, hout)
    g = {name: sess.scratch_f16(name, n) for name, n in
         (("xn", 1024), ("q", 2048), ("k", 1024), ("v", 1024), ("q_roped", 2048),
          ("attn", 2048), ("res", 1024), ("fn", 1024), ("act", 3072))}
    h_out = hout.download(np.float16, 1024)
    k_rows, v_rows = sess.cache_rows(layer, 0, pos + 1)

    # attention norm + q/k/v projections
    assert_norm_close(O, g["xn"], O.rmsnorm(h_in, w.attn_norm[layer]), "xn")
    assert_gemv(O, w.wq[layer], 2048, 1024, g["xn"], g["q"], "q")
    assert_gemv(O, w.wk[layer], 1024, 1024, g["xn"], g["k"], "k")
    assert_gemv(O, w.wv[layer], 1024, 1024, g["xn"], g["v"], "v")
    # head norms + RoPE, the cache write at slot pos
    qn = O.head_rmsnorm(g["q"], w.q_norm[layer])
    q_want = O.rope(qn, pos)
    assert (np.abs(f64(g["q_roped"]) - f64(q_want)) <= rope_tol(O, qn, q_want)).all()
    kn = O.head_rmsnorm(g["k"], w.k_norm[layer])
    k_want = O.rope(kn, pos)
    assert (np.abs(f64(k_rows[pos]) - f64(k_want)) <= rope_tol(O, kn, k_want)).all()
    assert np.array_equal(v_rows[pos].view(np.uint16), g["v"].view(np.uint16))
    # history slots untouched
    assert np.array_equal(k_rows[:pos], kc[layer * MAX_SEQ:layer * MAX_SEQ + pos])
    assert np.array_equal(v_rows[:pos], vc[layer * MAX_SEQ:layer * MAX_SEQ + pos])
    # attention over the GPU's cache with the GPU's roped q
    a_want = O.attention(g["q_roped"], k_rows, v_rows)
    d = np.abs(f64(g["attn"]) - f64(a_want))
    assert (d <= 2 * ulp(O, a_want) + 1e-5).all(), d.max()
    # attn_o + residual, ffn norm, gate_up + SwiGLU, down + residual
    assert_gemv_add(O, h_in, w.wo[layer], 1024, 2048, g["attn"], g["res"], "res")
    assert_norm_close(O, g["fn"], O.rmsnorm(g["res"], w.ffn_norm[layer]), "fn")
    gu = O.q8_gemv(w.wgu[layer], 6144, 1024, g["fn"])
    _, gmag = O.q8_gemv_f64(w.wgu[layer], 6144, 1024, g["fn"])
    act_want = O.swiglu(gu[:3072], gu[3072:])
    dg = 2 * ulp(O, gu) + 1e-3 * np.abs(f64(gu)) + 8 * 2.0 ** -24 * gmag
    gate, up = f64(gu[:3072]), f64(gu[3072:])
    silu = gate / (1 + np.exp(-gate))
    tol = 1.1 * np.abs(up) * dg[:3072] + np.abs(silu) * dg[3072:] + 4 * ulp(O, act_want)
    d = np.abs(f64(g["act"]) - f64(act_want))
    assert (d <= tol).all(), (np.flatnonzero(d > tol)[:8], d.max())
    assert_gemv_add(O, g["res"], w.wdn[layer], 1024, 3072, g["act"], h_out, "h_out")

    # the whole layer against the oracle's own chain
    h_ref, _ = O.decode_layer(w, layer, kc, vc, MAX_SEQ, pos, h_in)
    rel = np.linalg.norm(f64(h_out) - f64(h_ref)) / np.linalg.norm(f64(h_ref))
    assert rel < 5e-3, rel
    for b in (hin, hout):
        b.free()
    sess.free()


def test_embed_rows_and_out_of_range_ids(gpu, D, dmodel, model_host):
    Q = gpu
    sess = D.DecodeSession(dmodel, 4)
    h = Q.DeviceBuffer(2048)
    for tok, row in ((5, 5), (151935, 151935), (-3, 0), (151936, 0)):
        sess.set_state(tok, 0)
        sess.embed(h)
        got = h.download(np.float16, 1024)
        assert np.array_equal(got.view(np.uint16), model_host.token_embd[row].view(np.uint16))
    h.free()
    sess.free()


def _step_checks(O, w, sess, tok_in, pos, kc, vc, O_state):
    """Compare one GPU step with the oracle's; returns the oracle token."""
    tok_gpu, pos_gpu = sess.get_state()
    logits = sess.read_logits()
    on = sess.scratch_f16("on", 1024)
    ref_tok, ref_logits, hl = O.decode_step(w, kc, vc, MAX_SEQ, tok_in, pos, True, True)
    # final norm of the oracle's last hidden state (the GPU's differs slightly)
    on_ref = O.rmsnorm(hl[-1], w.output_norm)
    assert np.linalg.norm(f64(on) - f64(on_ref)) / np.linalg.norm(f64(on_ref)) < 1e-2
    # vocab stage against the GPU's own normalised input
    y_ref = O.f16_gemv(w.output_w, on)
    _, mag = O.f16_gemv_f64(w.output_w, on)
    rep = O.gemv_tolerance_report(logits, y_ref, mag)
    assert rep["fail"] == 0, rep
    # token = lowest index of the maximal f16 logit of the GPU's logits
    lf = logits.astype(np.float32)
    assert tok_gpu == int(np.flatnonzero(lf == lf.max())[0])
    assert tok_gpu == O.argmax_tiled(logits)
    # against the oracle chain
    dl = np.abs(f64(logits) - f64(ref_logits))
    assert np.linalg.norm(dl) / np.linalg.norm(f64(ref_logits)) < 2e-2
    srt = np.sort(ref_logits.astype(np.float64))
    if srt[-1] - srt[-2] > 2 * dl.max():
        assert tok_gpu == ref_tok, (tok_gpu, ref_tok, srt[-1] - srt[-2], dl.max())
    O_state["diffs"].append(float(dl.max()))
    return tok_gpu, pos_gpu


def test_decode_steps_match_oracle(O, gpu, D, dmodel, model_host):
    w = model_host
    sess = D.DecodeSession(dmodel, MAX_SEQ)
    kc = np.zeros((28 * MAX_SEQ, 1024), np.float16)
    vc = np.zeros_like(kc)
    tok, pos = 1234, 0
    sess.set_state(tok, pos)
    state = {"diffs": []}
    for step in range(6):
        print(f"decode step {step}", flush=True)
        sess.step(advance=True, logits=True)
        new_tok, new_pos = _step_checks(O, w, sess, tok, pos, kc, vc, state)
        assert new_pos == pos + 1
        # teacher forcing: the oracle continues from the GPU's token
        tok, pos = new_tok, new_pos
    assert sess.status() == 0
    sess.free()


def test_graph_replay_matches_eager(gpu, D, dmodel):
    Q = gpu
    eager = D.DecodeSession(dmodel, 64)
    eager.set_state(42, 0)
    toks, logits = [], []
    for _ in range(5):
        eager.step(advance=True, logits=True)
        toks.append(eager.get_state())
        logits.append(eager.read_logits())
    eager.free()

    stream = Q.Stream()
    sess = D.DecodeSession(dmodel, 64, stream)
    sess.set_state(42, 0)
    for i in range(5):
        print(f"graph replay {i}", flush=True)
        sess.replay(advance=True, logits=True)
        sess.synchronize()
        assert sess.get_state() == toks[i]
        assert np.array_equal(sess.read_logits().view(np.uint16), logits[i].view(np.uint16))
    sess.free()
    stream.destroy()


def test_cache_full_sets_status_and_keeps_position(gpu, D, dmodel):
    sess = D.DecodeSession(dmodel, 4)
    sess.set_state(9, 3)
    sess.step(advance=True, logits=False)
    tok, pos = sess.get_state()
    assert pos == 3 and sess.status() & 1
    assert 0 <= tok < D.VOCAB
    # an out-of-range position is clamped into the cache, not written past it
    sess.set_state(9, 100)
    sess.step(advance=False, logits=False)
    assert sess.get_state()[1] == 100
    k, v = sess.cache_rows(27, 3, 4)
    assert k.any() and v.any()
    sess.free()
