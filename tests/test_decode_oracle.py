"""Pins the decode-step part of the CPU oracle (oracle/decode_oracle.c).

Each function is checked against something other than its own formula: a
float64 evaluation of the textbook definition (rms_norm, rotate-half RoPE with
base 1e6, softmax attention, SiLU), closed-form known answers (eps placement,
pos = 0 identity, one-position attention = v of the matching kv head, SwiGLU
saturation), exact properties (f16 add, zero weights make a layer the
identity), and the step's own consistency (embedding row, argmax of its
logits, per-layer chaining).
"""
from __future__ import annotations

import types

import numpy as np
import pytest

RNG = np.random.default_rng(8675309)


def f16(a):
    return np.asarray(a, dtype=np.float16)


def within_ulps(got, want64, ulps=1.0, extra=0.0):
    """|got - want| <= ulps * ulp_f16(want) + extra, elementwise."""
    from oracle import ulp_f16

    g = np.asarray(got, np.float64)
    w = np.asarray(want64, np.float64)
    return np.abs(g - w) <= ulps * ulp_f16(w) + extra


# ------------------------------------------------------------- rms_norm ----

@pytest.mark.parametrize("std", [0.02, 1.0, 30.0])
def test_rmsnorm_vs_float64(O, std):
    x = f16(RNG.standard_normal(1024) * std)
    w = f16(1 + 0.1 * RNG.standard_normal(1024))
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 * x64) + O.EPS) * w64
    assert within_ulps(O.rmsnorm(x, w), want, 1.0).all()


def test_rmsnorm_eps_inside_sqrt_known_answer(O):
    # x = 2^-13 everywhere: mean(x^2) = 2^-26 ~ 1.49e-8, so eps = 1e-6
    # dominates: out = 2^-13 / sqrt(2^-26 + 1e-6) = 0.1212...  (eps outside
    # the sqrt or 1e-5 would give 1.0 or 0.0386).
    x = np.full(1024, 2.0 ** -13, np.float16)
    out = O.rmsnorm(x, np.ones(1024, np.float16))
    want = 2.0 ** -13 / np.sqrt(2.0 ** -26 + 9.99999997e-7)
    assert abs(want - 0.12122) < 1e-4
    assert within_ulps(out, np.full(1024, want), 1.0).all()


def test_rmsnorm_zero_vector(O):
    out = O.rmsnorm(np.zeros(1024, np.float16), np.ones(1024, np.float16))
    assert not out.view(np.uint16).any()


def test_head_rmsnorm_per_head_vs_float64(O):
    # heads of very different scale: each is normalised over its own 128 dims
    x = f16(RNG.standard_normal((16, 128)) * np.exp2(RNG.integers(-6, 6, (16, 1))))
    w = f16(1 + 0.1 * RNG.standard_normal(128))
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + O.EPS) * w.astype(np.float64)
    assert within_ulps(O.head_rmsnorm(x, w), want.reshape(-1), 1.0).all()


# ----------------------------------------------------------------- RoPE ----

def rope64(x, pos):
    """Rotate-half RoPE, theta_i = pos * 1e6^(-2i/128), in float64."""
    x = np.asarray(x, np.float64).reshape(-1, 128)
    i = np.arange(64, dtype=np.float64)
    th = pos * 1e6 ** (-(2 * i) / 128)
    c, s = np.cos(th), np.sin(th)
    x1, x2 = x[:, :64], x[:, 64:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=1).reshape(-1)


def test_rope_pos0_identity(O):
    x = f16(RNG.standard_normal(2048))
    assert np.array_equal(O.rope(x, 0).view(np.uint16), x.view(np.uint16))


@pytest.mark.parametrize("pos", [1, 7, 100, 1023, 40000])
def test_rope_vs_float64(O, pos):
    x = f16(RNG.standard_normal(2048))
    # the reference forms theta in f32: |f32(pos*inv) - pos*inv| <= pos * 2^-24
    extra = 2 * pos * 2.0 ** -24 * np.abs(x.astype(np.float64)).reshape(16, 128).max(axis=1)
    extra = np.repeat(extra, 128)
    got = O.rope(x, pos)
    assert within_ulps(got, rope64(x, pos), 1.0, extra + 1e-6).all()


def test_rope_relative_position(O):
    # <rope(q, m), rope(k, n)> depends on m - n only
    q, k = f16(RNG.standard_normal(128)), f16(RNG.standard_normal(128))
    d = [float(np.dot(O.rope(q, m).astype(np.float64), O.rope(k, m - 5).astype(np.float64)))
         for m in (5, 17, 300)]
    assert max(d) - min(d) < 0.05
    d0 = float(np.dot(q.astype(np.float64), O.rope(k, -5 + 5).astype(np.float64)))
    assert abs(d0 - float(np.dot(O.rope(q, 5).astype(np.float64),
                                 O.rope(k, 0).astype(np.float64)))) > 1e-3


# ------------------------------------------------------------ attention ----

def attention64(q, k_rows, v_rows, scale):
    q = np.asarray(q, np.float64).reshape(16, 128)
    k = np.asarray(k_rows, np.float64).reshape(-1, 8, 128)
    v = np.asarray(v_rows, np.float64).reshape(-1, 8, 128)
    out = np.empty((16, 128))
    for h in range(16):
        s = k[:, h // 2, :] @ q[h] * scale
        p = np.exp(s - s.max())
        out[h] = p @ v[:, h // 2, :] / p.sum()
    return out.reshape(-1)


def test_attention_one_position_is_v_of_kv_head(O):
    # softmax over one position is 1: head h returns v of kv head h // 2
    q = f16(RNG.standard_normal(2048))
    k = f16(RNG.standard_normal((1, 8, 128)))
    v = f16(RNG.standard_normal((1, 8, 128)))
    got = O.attention(q, k, v).reshape(16, 128)
    for h in range(16):
        assert np.array_equal(got[h].view(np.uint16), v[0, h // 2].view(np.uint16))


def test_attention_equal_keys_average_values(O):
    ctx = 50
    q = f16(RNG.standard_normal(2048))
    k = np.broadcast_to(f16(RNG.standard_normal((1, 8, 128))), (ctx, 8, 128)).copy()
    v = f16(RNG.standard_normal((ctx, 8, 128)))
    want = np.repeat(v.astype(np.float64).mean(axis=0), 2, axis=0).reshape(-1)
    assert within_ulps(O.attention(q, k, v), want, 2.0, 1e-5).all()


@pytest.mark.parametrize("ctx", [2, 33, 1024])
def test_attention_vs_float64(O, ctx):
    q = f16(RNG.standard_normal(2048) * 1.5)
    k = f16(RNG.standard_normal((ctx, 8, 128)))
    v = f16(RNG.standard_normal((ctx, 8, 128)) * 0.6)
    want = attention64(q, k, v, O.ATTN_SCALE)
    # f32 accumulation over ctx terms of |p v| <= max|v|
    extra = 8 * ctx * 2.0 ** -24 * 4.0
    assert within_ulps(O.attention(q, k, v), want, 2.0, extra).all()


def test_attention_scale_is_rsqrt_head_dim(O):
    assert np.float32(O.ATTN_SCALE).view(np.uint32) == 0x3DB504F3
    assert abs(O.ATTN_SCALE - 128 ** -0.5) < 1e-8


# --------------------------------------------------------------- SwiGLU ----

def test_swiglu_vs_float64(O):
    g = f16(RNG.standard_normal(20000) * 2)
    u = f16(RNG.standard_normal(20000))
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    want = g64 / (1 + np.exp(-g64)) * u64
    # five f16 roundings of the reference's f16 chain: a few ulps of the
    # result (plus the ulp of 1 + e carried through sig)
    extra = np.abs(g64 * u64) * 2.0 ** -11 * 2
    assert within_ulps(O.swiglu(g, u), want, 4.0, extra).all()


def test_swiglu_known_answers(O):
    g = f16([0.0, 10.0, -20.0, 10.0, 1.0])
    u = f16([3.0, 0.5, 2.0, 0.0, 1.0])
    out = O.swiglu(g, u).astype(np.float64)
    assert out[0] == 0.0                   # silu(0) = 0
    assert out[1] == 5.0                   # 1 + e^-10 rounds to 1 in f16: silu(10) = 10
    assert out[2] == 0.0                   # e^20 overflows f16: sig = 0
    assert out[3] == 0.0
    assert abs(out[4] - 1 / (1 + np.exp(-1))) < 2e-3


def test_add_f16_correctly_rounded(O):
    a = f16(RNG.standard_normal(100000) * np.exp2(RNG.integers(-10, 10, 100000)))
    b = f16(RNG.standard_normal(100000) * np.exp2(RNG.integers(-10, 10, 100000)))
    want = (a.astype(np.float64) + b.astype(np.float64)).astype(np.float16)  # exact sum, one RNE
    assert np.array_equal(O.add_f16(a, b).view(np.uint16), want.view(np.uint16))


# --------------------------------------------------------------- layer -----

def _tiny_weights(Wt, layers: int, zero_layers=()):
    """Layer-stacked parameters for `layers` layers (only what a layer reads)."""
    from oracle import HEAD_DIM, HIDDEN, WEIGHT_FIELDS

    shapes = {"wq": (2048, 1024), "wk": (1024, 1024), "wv": (1024, 1024), "wo": (1024, 2048),
              "wgu": (6144, 1024), "wdn": (1024, 3072)}
    ns = types.SimpleNamespace()
    for t, (name, (n, k)) in enumerate(shapes.items()):
        st = Wt.synthetic_q8_stack(n, k, layers, 5, 40 + t)
        for l in zero_layers:
            st[l] = 0  # scale 0: every weight 0
        setattr(ns, name, st)
    r = np.random.default_rng(3)
    ns.attn_norm = f16(1 + 0.1 * r.standard_normal((layers, HIDDEN)))
    ns.ffn_norm = f16(1 + 0.1 * r.standard_normal((layers, HIDDEN)))
    ns.q_norm = f16(1 + 0.1 * r.standard_normal((layers, HEAD_DIM)))
    ns.k_norm = f16(1 + 0.1 * r.standard_normal((layers, HEAD_DIM)))
    ns.token_embd = np.zeros((1, HIDDEN), np.float16)
    ns.output_norm = np.ones(HIDDEN, np.float16)
    ns.output_w = np.zeros((1, HIDDEN), np.float16)
    assert all(hasattr(ns, f) for f in WEIGHT_FIELDS)
    return ns


def _caches(max_seq):
    from oracle import KV_DIM, LAYERS

    return (np.zeros((LAYERS * max_seq, KV_DIM), np.float16),
            np.zeros((LAYERS * max_seq, KV_DIM), np.float16))


def test_layer_with_zero_weights_is_identity_and_strides_layers(O, Wt):
    w = _tiny_weights(Wt, 2, zero_layers=(0,))
    h = f16(RNG.standard_normal(1024))
    kc, vc = _caches(8)
    h0, _ = O.decode_layer(w, 0, kc, vc, 8, 3, h)
    assert np.array_equal(h0.view(np.uint16), h.view(np.uint16))   # o = 0 and down = 0
    h1, _ = O.decode_layer(w, 1, kc, vc, 8, 3, h)
    assert not np.array_equal(h1, h)                                # layer 1 reads its own slice


def test_layer_pos0_and_cache_slot(O, Wt):
    w = _tiny_weights(Wt, 2)
    h = f16(RNG.standard_normal(1024))
    max_seq = 8
    kc, vc = _caches(max_seq)
    _, tr = O.decode_layer(w, 1, kc, vc, max_seq, 0, h)
    # one position: attention output = v of the matching kv head
    att = tr["attn"].reshape(16, 128)
    v = tr["v"].reshape(8, 128)
    for hd in range(16):
        assert np.array_equal(att[hd].view(np.uint16), v[hd // 2].view(np.uint16))
    # the new k (roped) and v land in slot layer * max_seq + pos, nowhere else
    assert np.array_equal(kc[1 * max_seq + 0], tr["k_roped"])
    assert np.array_equal(vc[1 * max_seq + 0], tr["v"])
    assert np.count_nonzero(kc.view(np.uint16).any(axis=1)) == 1
    # at pos 0 RoPE is the identity: k_roped = head_rmsnorm(k)
    _, tr5 = O.decode_layer(w, 1, kc, vc, max_seq, 5, h)
    assert np.array_equal(kc[1 * max_seq + 5], tr5["k_roped"])
    assert not np.array_equal(tr5["k_roped"], tr["k_roped"])


# ---------------------------------------------------------------- step -----

def test_step_consistency(O, model_host):
    w = model_host
    max_seq = 16
    kc, vc = _caches(max_seq)
    kc2, vc2 = _caches(max_seq)
    tok, logits, hl = O.decode_step(w, kc, vc, max_seq, 777, 0, True, True)
    assert np.array_equal(hl[0], w.token_embd[777])
    # the 28 layers chain through decode_layer with the same caches
    h = hl[0]
    for l in range(O.LAYERS):
        h, _ = O.decode_layer(w, l, kc2, vc2, max_seq, 0, h)
        assert np.array_equal(h.view(np.uint16), hl[l + 1].view(np.uint16)), l
    assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2)
    # logits = output_w . rms_norm(h_28, output_norm); token = lowest index of the max
    normed = O.rmsnorm(hl[O.LAYERS], w.output_norm)
    assert np.array_equal(logits.view(np.uint16), O.f16_gemv(w.output_w, normed).view(np.uint16))
    lf = logits.astype(np.float32)
    assert tok == int(np.flatnonzero(lf == lf.max())[0])
    # and the logits are the float64 product within the GEMV tolerance
    y64, mag = O.f16_gemv_f64(w.output_w, normed)
    rep = O.gemv_tolerance_report(logits, y64, mag)
    assert rep["fail"] == 0, rep
