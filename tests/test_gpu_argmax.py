"""The tiled argmax as its own pass (f16_argmax): the token of n f16 values
already in device memory must equal the oracle's two-phase tiled argmax
(model/qwen3_full.mlir:1469-1511) bit for bit -- the lowest index of the
maximal value, NaN never winning, -1 when nothing wins -- on random vectors,
every ragged length around the kernel's 8-value pieces and 2048-value
workgroup shares, and constructed ties.  With the HAL vocab dispatch (which
writes logits only) it reproduces the fused vocab kernel's token."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def run(Q, v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, np.float16)
    with Q.DeviceBuffer.from_array(v) as d, Q.DeviceBuffer(16) as tok, \
            Q.DeviceBuffer(Q.vocab_workspace_bytes()) as ws:
        Q.vocab_workspace_reset(ws)
        print(f"f16_argmax n={v.size}", flush=True)
        Q.f16_argmax(d, v.size, tok, ws)
        Q.synchronize()
        t = int(tok.download(np.int32, 1)[0])
        assert int(ws.download(np.uint64, 1)[0]) == 0  # left zero for the next call
    return t


@pytest.mark.parametrize("n", [1, 7, 8, 9, 255, 256, 257, 2047, 2048, 2049, 151936, 600001])
def test_random_lengths(gpu, O, n):
    rng = np.random.default_rng(n)
    v = rng.standard_normal(n).astype(np.float16)
    assert run(gpu, v) == O.argmax_tiled(v)


@pytest.mark.parametrize("pos", [[0, 5], [255, 256], [2047, 2048], [151934, 151935],
                                 [3, 70000, 151935]])
def test_exact_ties_pick_lowest_index(gpu, O, pos):
    rng = np.random.default_rng(7)
    v = (rng.standard_normal(151936) * 0.1).astype(np.float16)
    for p in pos:
        v[p] = np.float16(3.5)
    assert run(gpu, v) == O.argmax_tiled(v) == min(pos)


@pytest.mark.parametrize("case", ["nan_around_max", "all_nan", "all_neg_inf", "pos_inf_ties",
                                  "signed_zero", "negative_only"])
def test_special_values(gpu, O, case):
    n = 5000
    rng = np.random.default_rng(11)
    v = (-np.abs(rng.standard_normal(n)) - 1.0).astype(np.float16)
    if case == "nan_around_max":
        v[100] = 2.0
        v[99] = v[101] = v[4000] = np.nan
    elif case == "all_nan":
        v[:] = np.nan
    elif case == "all_neg_inf":
        v[:] = -np.inf
    elif case == "pos_inf_ties":
        v[2049] = v[17] = np.inf
    elif case == "signed_zero":
        v[300] = np.float16(-0.0)
        v[200] = np.float16(0.0)
        v[4095] = np.float16(-0.0)
    want = O.argmax_tiled(v)
    assert run(gpu, v) == want
    if case in ("all_nan", "all_neg_inf"):
        assert want == -1


def test_hal_vocab_then_argmax_matches_fused(gpu, Wt):
    """decode_dispatch_24 through the HAL ABI (logits only) followed by
    f16_argmax gives the fused vocab kernel's token and logits."""
    Q = gpu
    n, k = Q.VOCAB_ROWS, Q.HIDDEN
    W = Wt.synthetic_f16_matrix(n, k, seed=31, tensor=24)
    x = Wt.synthetic_x(k, 31, 24)
    b1 = np.zeros(64 + 2 * k, np.uint8)
    b1[64:] = x.view(np.uint8)
    with Q.DeviceBuffer.from_array(W) as w, Q.DeviceBuffer.from_array(b1) as bind1, \
            Q.DeviceBuffer(2 * n + 64) as bind2, Q.DeviceBuffer.from_array(x) as xd, \
            Q.DeviceBuffer(2 * n) as ld, Q.DeviceBuffer(16) as td, Q.DeviceBuffer(16) as td2, \
            Q.DeviceBuffer(Q.vocab_workspace_bytes()) as ws:
        Q.vocab_workspace_reset(ws)
        Q.hal_dispatch(24, w, bind1, bind2, [0])
        Q.f16_argmax(bind2, n, td2, ws)
        Q.vocab_gemv_argmax(w, xd, ld, td, ws)
        Q.synchronize()
        assert np.array_equal(bind2.download(np.uint16, n), ld.download(np.uint16))
        assert int(td2.download(np.int32, 1)[0]) == int(td.download(np.int32, 1)[0])
