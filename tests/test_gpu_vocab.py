"""GPU parity of the fused f16 vocab GEMV + argmax against the oracle.

Logits: the GEMV tolerance rule (2 f16 ulp / 1e-3 relative, f32 noise floor
bounded per test).  Token: bit-exact -- it must equal the oracle's two-phase
tiled argmax (model/qwen3_full.mlir:1469-1511) of the GPU's own f16 logits
on every input, and the oracle's argmax of the oracle logits whenever the
top-2 oracle logits differ by more than the logit tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED = 99
N = 151936
K = 1024


@pytest.fixture(scope="module")
def vocab_w(Wt):
    return Wt.synthetic_f16_matrix(N, K, seed=SEED, tensor=24)


@pytest.fixture(scope="module")
def dev(gpu, vocab_w):
    Q = gpu
    bufs = {
        "w": Q.DeviceBuffer.from_array(vocab_w),
        "x": Q.DeviceBuffer(2 * K),
        "logits": Q.DeviceBuffer(2 * N),
        "token": Q.DeviceBuffer(16),
        "ws": Q.DeviceBuffer(Q.vocab_workspace_bytes()),
    }
    Q.vocab_workspace_reset(bufs["ws"])
    yield bufs
    for b in bufs.values():
        b.free()


def run(Q, dev, x, w=None, n=N, logits=True):
    dev["x"].upload(x)
    wbuf = w if w is not None else dev["w"]
    lg = dev["logits"] if logits else None
    if n == N:
        Q.vocab_gemv_argmax(wbuf, dev["x"], lg, dev["token"], dev["ws"])
    else:
        Q.f16_gemv_argmax_rows(wbuf, n, dev["x"], lg, dev["token"], dev["ws"])
    Q.synchronize()
    tok = int(dev["token"].download(np.int32, 1)[0])
    return (dev["logits"].download(np.float16, n) if logits else None), tok


def check_token(O, W, x, logits, tok, max_floor=30):
    ref = O.f16_gemv(W, x)
    _, mag = O.f16_gemv_f64(W, x)
    rep = O.gemv_tolerance_report(logits, ref, mag)
    assert rep["fail"] == 0, rep
    assert rep["on_floor"] <= max_floor, rep
    assert tok == O.argmax_tiled(logits), (tok, O.argmax_tiled(logits))
    ref_tok = O.argmax_tiled(ref)
    if tok != ref_tok:
        # only acceptable when the oracle's own top values are within tolerance
        a, b = float(ref[tok]), float(ref[ref_tok])
        assert abs(a - b) <= 2 * O.ulp_f16(np.array([b]))[0] + 1e-3 * abs(b), (tok, ref_tok, a, b)
    return rep


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_vocab_logits_and_token_random(gpu, O, Wt, vocab_w, dev, seed):
    x = Wt.synthetic_x(K, SEED, seed)
    logits, tok = run(gpu, dev, x)
    check_token(O, vocab_w, x, logits, tok)


def test_reference_named_entry_point_and_null_logits(gpu, O, Wt, vocab_w, dev):
    Q = gpu
    x = Wt.synthetic_x(K, SEED, 7)
    logits, tok = run(Q, dev, x)
    _, tok2 = run(Q, dev, x, logits=False)
    assert tok2 == tok
    dev["x"].upload(x)
    Q.decode_dispatch(24, dev["w"], dev["x"], dev["logits"], dev["token"], dev["ws"])
    Q.synchronize()
    assert int(dev["token"].download(np.int32, 1)[0]) == tok
    assert np.array_equal(dev["logits"].download(np.uint16, N), logits.view(np.uint16))


@pytest.mark.parametrize("rows", [[255, 256], [0, 151935], [147, 148, 149, 75968],
                                  [151935, 151934], [40000, 3, 120000]])
def test_exact_ties_pick_lowest_index(gpu, O, Wt, vocab_w, dev, rows):
    """Identical rows give bit-identical logits; the winner must be the lowest
    index however the ties straddle waves, workgroups and the padded tail."""
    Q = gpu
    x = Wt.synthetic_x(K, SEED, 11)
    hot = (np.sign(x.astype(np.float32)) * 0.05).astype(np.float16)  # logit ~ 0.05 * sum|x|
    W = vocab_w.copy()
    for r in rows:
        W[r] = hot
    with Q.DeviceBuffer.from_array(W) as wdev:
        logits, tok = run(Q, dev, x, w=wdev)
    assert tok == min(rows)
    assert len({int(logits.view(np.uint16)[r]) for r in rows}) == 1
    check_token(O, W, x, logits, tok)


def test_signed_zero_tie_and_negative_logits(gpu, O, Wt, dev):
    """All logits <= 0 with a +0 / -0 tie at the top: -0 == +0, lowest index wins."""
    Q = gpu
    n = 4096
    x = np.ones(K, np.float16)
    W = np.full((n, K), np.float16(-0.01), np.float16)
    W[1000] = 0.0          # logit +0
    W[700] = -0.0          # logit: sum of -0 * 1 -> -0 or +0; either ties with +0
    with Q.DeviceBuffer.from_array(W) as wdev:
        logits, tok = run(Q, dev, x, w=wdev, n=n)
    assert tok == 700
    assert tok == O.argmax_tiled(logits)


@pytest.mark.parametrize("case", ["nan_x", "inf_x", "all_neg_inf"])
def test_non_finite_inputs(gpu, O, Wt, dev, case):
    Q = gpu
    n = 5000
    W = Wt.synthetic_f16_matrix(n, K, seed=SEED, tensor=77)
    x = Wt.synthetic_x(K, SEED, 13)
    if case == "nan_x":
        x[17] = np.nan           # every logit NaN: no winner
    elif case == "inf_x":
        x[5] = np.inf            # logits +-inf or NaN (0 * inf)
    else:
        W[:] = np.float16(-60000.0)
        x[:] = np.float16(60000.0)  # every logit overflows to -inf
    with Q.DeviceBuffer.from_array(W) as wdev:
        logits, tok = run(Q, dev, x, w=wdev, n=n)
    assert tok == O.argmax_tiled(logits)
    if case in ("nan_x", "all_neg_inf"):
        assert tok == -1
    else:
        ref = O.f16_gemv(W, x)
        assert tok == O.argmax_tiled(ref)


@pytest.mark.parametrize("n", [1, 2, 63, 64, 65, 1000, 4095, 4096, 4097, 20000])
def test_ragged_row_counts(gpu, O, Wt, dev, n):
    Q = gpu
    W = Wt.synthetic_f16_matrix(n, K, seed=SEED, tensor=1000 + n)
    x = Wt.synthetic_x(K, SEED, n)
    with Q.DeviceBuffer.from_array(W) as wdev:
        dev["logits"].fill(0x55)
        logits, tok = run(Q, dev, x, w=wdev, n=n)
        tail = dev["logits"].download(np.uint8, 64, offset=2 * n)
    check_token(O, W, x, logits, tok, max_floor=5)
    assert np.all(tail == 0x55)


@pytest.mark.parametrize("wgs", [1, 7, 256, 1000, 4096])
def test_workgroup_counts_agree(gpu, O, Wt, vocab_w, dev, wgs):
    Q = gpu
    x = Wt.synthetic_x(K, SEED, 21)
    base_logits, base_tok = run(Q, dev, x)
    old = Q.get_vocab_workgroups()
    try:
        Q.set_vocab_workgroups(wgs)
        logits, tok = run(Q, dev, x)
    finally:
        Q.set_vocab_workgroups(0)
    assert Q.get_vocab_workgroups() == old
    assert tok == base_tok
    assert np.array_equal(logits.view(np.uint16), base_logits.view(np.uint16))


def test_workspace_counter_resets_between_launches(gpu, O, Wt, vocab_w, dev):
    """Back-to-back launches on one stream reuse the workspace; each must see
    a zero counter (left by the previous launch) and produce its own token."""
    Q = gpu
    xs = [Wt.synthetic_x(K, SEED, 100 + i) for i in range(4)]
    xbuf = Q.DeviceBuffer.from_array(np.stack(xs))
    toks = Q.DeviceBuffer(16)
    try:
        for i in range(4):
            Q.vocab_gemv_argmax(dev["w"], xbuf.ptr + 2 * K * i, None, toks.ptr + 4 * i, dev["ws"])
        Q.synchronize()
        got = toks.download(np.int32, 4)
        counter = dev["ws"].download(np.uint32, 1)[0]
    finally:
        xbuf.free()
        toks.free()
    assert counter == 0
    for i in range(4):
        _, tok = run(Q, dev, xs[i])
        assert got[i] == tok


def test_graph_replay_matches_eager(gpu, O, Wt, vocab_w, dev):
    Q = gpu
    x = Wt.synthetic_x(K, SEED, 31)
    logits, tok = run(Q, dev, x)
    s = Q.Stream()
    try:
        g = Q.Graph(s, lambda: Q.vocab_gemv_argmax(dev["w"], dev["x"], dev["logits"],
                                                   dev["token"], dev["ws"], s))
        for rep in range(3):
            dev["token"].fill(0)
            dev["logits"].fill(0)
            g.launch(s)
            s.synchronize()
            assert int(dev["token"].download(np.int32, 1)[0]) == tok, rep
            assert np.array_equal(dev["logits"].download(np.uint16, N), logits.view(np.uint16))
            run(Q, dev, x)  # eager work between replays
        g.destroy()
    finally:
        s.destroy()
