"""Pins the CPU oracle (oracle/q8_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something other than its own formula:
numpy's binary16 conversion, hand-built known-answer blocks, one-hot inputs that
reduce a GEMV to a single exactly-representable product, an independent float64
matmul, exact power-of-two linearity, and brute-force argmax.
"""
from __future__ import annotations

import numpy as np
import pytest

RNG = np.random.default_rng(20261201)


# ----------------------------------------------------------------- f16 -----

def test_f16_to_f32_all_halves(O):
    h = np.arange(65536, dtype=np.uint16).view(np.float16)
    got, want = O.f16_to_f32(h), h.astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_f32_to_f16_matches_numpy(O):
    bits = RNG.integers(0, 2**32, size=1_000_000, dtype=np.uint64).astype(np.uint32)
    scaled = (RNG.standard_normal(1_000_000) * np.exp2(RNG.integers(-30, 18, 1_000_000)))
    hv = np.arange(0, 0x7BFF, dtype=np.uint16).view(np.float16).astype(np.float64)
    nxt = np.nextafter(hv.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    halfway = (hv + nxt) / 2  # exact ties: must round to even
    for f in (bits.view(np.float32), scaled.astype(np.float32), halfway.astype(np.float32),
              -halfway.astype(np.float32)):
        with np.errstate(over="ignore"):
            want = f.astype(np.float16)
        got = O.f32_to_f16(f)
        same = (got.view(np.uint16) == want.view(np.uint16)) | (np.isnan(got) & np.isnan(want))
        assert same.all()


# ------------------------------------------------------------ quantizer -----

def _block_bytes(scale_f16: float, q: np.ndarray) -> np.ndarray:
    return np.concatenate([np.array([scale_f16], np.float16).view(np.uint8),
                           np.asarray(q, np.int8).view(np.uint8)])


def test_quantize_known_answer_round_half_even(O):
    # max|w| = 127 -> scale exactly 1.0, so q = round(w): ties must go to even.
    w = np.zeros(32, np.float32)
    w[:12] = [127, -127, 63.5, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.49, -3.51, 126.5]
    want_q = np.zeros(32, np.int8)
    want_q[:12] = [127, -127, 64, 0, 2, 2, 0, -2, -2, 3, -4, 126]
    assert np.array_equal(O.q8_quantize(w), _block_bytes(1.0, want_q))


def test_quantize_zero_block_scale_one(O):
    out = O.q8_quantize(np.zeros(64, np.float32))
    assert np.array_equal(out[:2], np.array([0x00, 0x3C], np.uint8))  # f16 1.0, LE
    assert not out[2:34].any() and np.array_equal(out[34:36], [0x00, 0x3C])


def test_quantize_scale_is_f16_of_f32_division(O):
    blk = np.zeros(32, np.float32)
    blk[5] = np.float32(0.0317)
    scale32 = np.float32(0.0317) / np.float32(127.0)
    out = O.q8_quantize(blk)
    assert out[:2].view(np.float16)[0] == np.float16(scale32)
    assert out[2 + 5].astype(np.int8) == 127


def test_quantize_invariants_random(O):
    w = (RNG.standard_normal(32 * 4096) * 0.02).astype(np.float32)
    w[:32] = 0.0
    raw = O.q8_quantize(w).reshape(-1, 34)
    q = raw[:, 2:].view(np.int8).astype(np.int32)
    s16 = raw[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
    nz = np.any(w.reshape(-1, 32) != 0, axis=1)
    assert np.all(np.abs(q[nz]).max(axis=1) == 127)
    assert np.all(q[~nz] == 0) and np.all(s16[~nz] == 1.0)
    s32 = (np.abs(w.reshape(-1, 32)).max(axis=1) / np.float32(127)).astype(np.float64)
    err = np.abs(q * s16[:, None] - w.reshape(-1, 32))
    bound = 127 * np.abs(s16 - s32) + s32 / 2 * (1 + 1e-6)
    assert np.all(err[nz] <= bound[nz, None] + 1e-12)


def test_quantize_agrees_with_product_weight_prep(O, Wt):
    w = (RNG.standard_normal(32 * 2048) * 0.02).astype(np.float32)
    w[64:96] = 0
    w[96:128] = np.linspace(-3, 3, 32, dtype=np.float32)
    assert np.array_equal(O.q8_quantize(w), Wt.quantize_q8_0(w))


def test_dequant_known_answer(O):
    q = np.arange(-128, 128, dtype=np.int32).reshape(8, 32)
    raw = np.concatenate([_block_bytes(1.0 if i % 2 == 0 else 2.0, q[i]) for i in range(8)])
    got = O.q8_dequant(raw).reshape(8, 32)
    want = q * np.where(np.arange(8) % 2 == 0, 1.0, 2.0)[:, None]
    assert np.array_equal(got, want.astype(np.float32))


def test_dequant_f16_rounds_each_exact_product_once(O):
    """The prompt path's f16 weights: f16(scale * q), one rounding of the exact
    product.  Checked against float64 products (exact: 11 x 8 bits) converted
    by numpy's correctly rounded float64 -> float16, with scales whose products
    need rounding (1/3, 0.0123), that land on f16 subnormals (2^-20) and that
    make every product exact (powers of two)."""
    q = RNG.integers(-128, 128, (6, 32)).astype(np.int32)
    q[0, :3] = (-128, 127, 0)
    scales = [1.0 / 3.0, 0.0123, 2.0 ** -20, 0.5, 4.0, -0.7]
    raw = np.concatenate([_block_bytes(sc, q[i]) for i, sc in enumerate(scales)])
    got = O.q8_dequant_f16(raw, 6, 32)
    s16 = np.array(scales, np.float16).astype(np.float64)
    want = (s16[:, None] * q).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    # powers of two: no rounding at all
    assert np.array_equal(got[3:5].astype(np.float64), s16[3:5, None] * q[3:5])
    # f16(1/3) * 3 = 1 - 2^-12 exactly: a tie between 1 - 2^-11 and 1, which
    # round-to-nearest-even sends to 1; f16(1/3) * -3 likewise to -1
    third = _block_bytes(1.0 / 3.0, np.array([3, -3] * 16))
    got = O.q8_dequant_f16(third, 1, 32)[0, :2]
    assert float(np.float16(1.0 / 3.0)) * 3 == 1 - 2.0 ** -12
    assert got[0] == np.float16(1.0) and got[1] == np.float16(-1.0)


# ---------------------------------------------------------------- GEMV ------

def _q8_layer(n, k, seed):
    from qwen3_iree_amd import weights

    return weights.synthetic_q8_layer(n, k, seed, 0, 0)


@pytest.mark.parametrize("k", [1024, 2048, 3072])
def test_q8_gemv_one_hot_is_exact(O, k):
    n = 64
    raw = _q8_layer(n, k, 3 + k)
    blocks = raw.reshape(n, k // 32, 34)
    for col in (0, 1, 31, 32, 33, 1023, k - 1, k // 2 + 5):
        x = np.zeros(k, np.float16)
        x[col] = 1.0
        y = O.q8_gemv(raw, n, k, x)
        scale = blocks[:, col // 32, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
        q = blocks[:, col // 32, 2 + col % 32].view(np.int8).astype(np.float32)
        assert np.array_equal(y.view(np.uint16), (scale * q).astype(np.float16).view(np.uint16)), col


@pytest.mark.parametrize("k", [1024, 2048, 3072])
def test_q8_gemv_matches_float64_matmul(O, k):
    n = 256
    raw = _q8_layer(n, k, 11 + k)
    x = (RNG.standard_normal(k)).astype(np.float16)
    W = O.q8_dequant(raw).reshape(n, k).astype(np.float64)  # s*q exact in f32
    y64 = W @ x.astype(np.float64)
    y64_o, mag = O.q8_gemv_f64(raw, n, k, x)
    assert np.allclose(y64_o, y64, rtol=1e-12, atol=1e-12)
    assert np.allclose(mag, np.abs(W) @ np.abs(x.astype(np.float64)), rtol=1e-12)
    rep = O.gemv_tolerance_report(O.q8_gemv(raw, n, k, x), y64.astype(np.float16), mag)
    assert rep["fail"] == 0, rep
    assert rep["on_floor"] <= 2, rep


def test_q8_gemv_power_of_two_linearity_and_zero(O):
    n, k = 128, 2048
    raw = _q8_layer(n, k, 5)
    x = (RNG.standard_normal(k) * 0.5).astype(np.float16)
    y1 = O.q8_gemv(raw, n, k, x).astype(np.float32)
    y2 = O.q8_gemv(raw, n, k, (x.astype(np.float32) * 2).astype(np.float16)).astype(np.float32)
    normal = np.abs(y1) >= 2.0 ** -14
    assert np.array_equal(y2[normal], 2 * y1[normal])
    y0 = O.q8_gemv(raw, n, k, np.zeros(k, np.float16))
    assert np.all(y0.view(np.uint16) == 0)


def test_f16_gemv_one_hot_and_float64(O):
    n, k = 512, 1024
    W = (RNG.standard_normal((n, k)) * 0.02).astype(np.float16)
    for col in (0, 31, 32, 1023):
        x = np.zeros(k, np.float16)
        x[col] = 1.0
        assert np.array_equal(O.f16_gemv(W, x).view(np.uint16), W[:, col].view(np.uint16))
    x = RNG.standard_normal(k).astype(np.float16)
    y64 = W.astype(np.float64) @ x.astype(np.float64)
    y64_o, mag = O.f16_gemv_f64(W, x)
    assert np.allclose(y64_o, y64, rtol=1e-12, atol=1e-15)
    rep = O.gemv_tolerance_report(O.f16_gemv(W, x), y64.astype(np.float16), mag)
    assert rep["fail"] == 0 and rep["on_floor"] <= 2, rep


def test_tolerance_report_flags_planted_errors(O):
    n, k = 256, 1024
    raw = _q8_layer(n, k, 9)
    x = RNG.standard_normal(k).astype(np.float16)
    ref = O.q8_gemv(raw, n, k, x)
    _, mag = O.q8_gemv_f64(raw, n, k, x)
    big = int(np.argmax(np.abs(ref.astype(np.float32))))
    bad = ref.copy()
    bad[big] = np.float16(ref[big].astype(np.float32) * (1 + 4e-3))  # a 0.4% error
    assert O.gemv_tolerance_report(bad, ref, mag)["fail"] == 1
    # a dropped term (block 0 of every row ignored) fails broadly
    raw2 = raw.copy().reshape(n, -1, 34)
    raw2[:, 0, 2:] = 0
    dropped = O.q8_gemv(raw2.reshape(-1), n, k, x)
    assert O.gemv_tolerance_report(dropped, ref, mag)["fail"] > n // 2


# -------------------------------------------------------------- argmax ------

def brute_argmax(v: np.ndarray) -> int:
    f = v.astype(np.float32)
    ok = ~np.isnan(f) & (f > -np.inf)
    if not ok.any():
        return -1
    m = f[ok].max()
    return int(np.nonzero(ok & (f == m))[0][0])


def _tie_cases():
    n = 151936
    base = (RNG.standard_normal(n) * 0.64).astype(np.float16)
    cases = []
    v = base.copy(); v[255] = v[256] = 9.0; cases.append(("tile boundary tie", v))
    v = base.copy(); v[0] = 9.0; cases.append(("max at 0", v))
    v = base.copy(); v[n - 1] = 9.0; cases.append(("max in padded last tile", v))
    v = base.copy(); v[70000] = v[151935] = v[151000] = 9.0; cases.append(("3-way tie", v))
    v = base.copy(); v[:] = -5.0; v[100] = -0.0; v[50] = 0.0; cases.append(("-0/+0 tie", v))
    v = base.copy(); v[3] = np.nan; v[4] = 9.0; v[5] = np.nan; cases.append(("nan around max", v))
    v = np.full(n, np.nan, np.float16); cases.append(("all nan", v))
    v = np.full(n, -np.inf, np.float16); cases.append(("all -inf", v))
    v = np.full(n, -np.inf, np.float16); v[77] = np.nan; v[99] = -65504; cases.append(("one finite", v))
    v = base.copy(); v[1234] = np.inf; v[99999] = np.inf; cases.append(("+inf tie", v))
    cases.append(("n=1", np.array([1.5], np.float16)))
    cases.append(("n=300", base[:300].copy()))
    return cases


@pytest.mark.parametrize("name,v", _tie_cases(), ids=lambda c: c if isinstance(c, str) else "")
def test_argmax_tiled_known_cases(O, name, v):
    assert O.argmax_tiled(v) == brute_argmax(v), name


def test_argmax_tiled_random_vs_brute_force(O):
    for trial in range(20):
        n = int(RNG.integers(1, 5000))
        v = RNG.integers(-8, 8, n).astype(np.float16)  # many ties
        assert O.argmax_tiled(v) == brute_argmax(v)
        assert O.argmax_tiled(v, 7) == brute_argmax(v)
