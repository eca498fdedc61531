"""Golden fixtures (tests/golden/golden_vectors.npz, written by make_golden.py
from an independent float64 computation) checked against the oracle on the
CPU and against the HIP kernels on the GPU."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden" / "golden_vectors.npz"


@pytest.fixture(scope="module")
def G():
    return np.load(GOLDEN)


@pytest.mark.parametrize("k", [1024, 2048, 3072])
def test_oracle_q8_gemv_matches_golden(O, G, k):
    w, x = G[f"q8_k{k}_w"], G[f"q8_k{k}_x"]
    n = G[f"q8_k{k}_y"].size
    y64, mag = O.q8_gemv_f64(w, n, k, x)
    assert np.allclose(y64, G[f"q8_k{k}_y64"], rtol=1e-12, atol=1e-12)
    assert np.allclose(mag, G[f"q8_k{k}_sumabs"], rtol=1e-12)
    rep = O.gemv_tolerance_report(O.q8_gemv(w, n, k, x), G[f"q8_k{k}_y"], mag)
    assert rep["fail"] == 0 and rep["on_floor"] == 0, rep


def test_oracle_f16_gemv_and_argmax_match_golden(O, G):
    W, x = G["f16_w"], G["f16_x"]
    y64, mag = O.f16_gemv_f64(W, x)
    assert np.allclose(y64, G["f16_y64"], rtol=1e-12, atol=1e-15)
    y = O.f16_gemv(W, x)
    rep = O.gemv_tolerance_report(y, G["f16_y"], mag)
    assert rep["fail"] == 0 and rep["on_floor"] == 0, rep
    assert O.argmax_tiled(y) == int(G["f16_token"][0])
    for i in range(4):
        assert O.argmax_tiled(G[f"argmax_{i}_v"]) == int(G[f"argmax_{i}_token"][0]), i


@pytest.mark.gpu
@pytest.mark.parametrize("k", [1024, 2048, 3072])
def test_gpu_q8_gemv_matches_golden(gpu, O, G, k):
    Q = gpu
    w, x = G[f"q8_k{k}_w"], G[f"q8_k{k}_x"]
    n = G[f"q8_k{k}_y"].size
    with Q.DeviceBuffer.from_array(w) as wd, Q.DeviceBuffer.from_array(x) as xd, \
            Q.DeviceBuffer(2 * n) as yd:
        Q.q8gemv_rows(wd, n, k, xd, yd)
        Q.synchronize()
        y = yd.download(np.float16)
    rep = O.gemv_tolerance_report(y, G[f"q8_k{k}_y"], G[f"q8_k{k}_sumabs"])
    assert rep["fail"] == 0 and rep["on_floor"] == 0, rep


@pytest.mark.gpu
def test_gpu_f16_gemv_argmax_matches_golden(gpu, O, G):
    Q = gpu
    W, x = G["f16_w"], G["f16_x"]
    n = W.shape[0]
    with Q.DeviceBuffer.from_array(W) as wd, Q.DeviceBuffer.from_array(x) as xd, \
            Q.DeviceBuffer(2 * n) as ld, Q.DeviceBuffer(16) as td, \
            Q.DeviceBuffer(Q.vocab_workspace_bytes()) as ws:
        Q.vocab_workspace_reset(ws)
        Q.f16_gemv_argmax_rows(wd, n, xd, ld, td, ws)
        Q.synchronize()
        logits = ld.download(np.float16)
        tok = int(td.download(np.int32, 1)[0])
    rep = O.gemv_tolerance_report(logits, G["f16_y"], G["f16_sumabs"])
    assert rep["fail"] == 0 and rep["on_floor"] == 0, rep
    assert tok == int(G["f16_token"][0])
