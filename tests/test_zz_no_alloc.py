"""The allocation-free entry point f16_gemv_argmax_rows_noalloc against the
workspace form f16_gemv_argmax_rows, through the C ABI: the same logits bit
for bit and the same token, on two calls in a row (the second over fewer rows
than the first call's winning row, so a key left over from the first call
would show), interleaved with workspace calls, and under stream capture."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED = 777


def _pair(Q, w, n, x, ws):
    """(logits, token) of the workspace form and of the allocation-free form."""
    out = []
    for noalloc in (False, True):
        logits = Q.DeviceBuffer(2 * n + 64)
        tok = Q.DeviceBuffer(16)
        logits.fill(0xFF)
        tok.fill(0xFF)
        print(f"f16 argmax rows={n} noalloc={noalloc}", flush=True)
        if noalloc:
            Q.f16_gemv_argmax_rows_noalloc(w, n, x, logits, tok)
        else:
            Q.f16_gemv_argmax_rows(w, n, x, logits, tok, ws)
        Q.synchronize()
        out.append((logits.download(np.uint16, n), int(tok.download(np.int32, 1)[0])))
        logits.free()
        tok.free()
    return out


def test_noalloc_matches_workspace_form_two_calls(gpu, O, Wt):
    Q = gpu
    rows = Q.VOCAB_ROWS
    W = Wt.synthetic_f16_matrix(rows, 1024, seed=SEED, tensor=1)
    x1 = Wt.synthetic_x(1024, SEED, 1)
    x2 = Wt.synthetic_x(1024, SEED, 2)
    with Q.DeviceBuffer.from_array(W) as w, Q.DeviceBuffer.from_array(x1) as xb1, \
            Q.DeviceBuffer.from_array(x2) as xb2, \
            Q.DeviceBuffer(Q.vocab_workspace_bytes()) as ws:
        Q.vocab_workspace_reset(ws)
        (la, ta), (lb, tb) = _pair(Q, w, rows, xb1, ws)
        assert np.array_equal(la, lb) and ta == tb
        assert ta == O.argmax_tiled(la.view(np.float16))
        # second call: fewer rows than the first winner's index
        n2 = max(1, ta // 2) if ta > 1 else 1000
        (la2, ta2), (lb2, tb2) = _pair(Q, w, n2, xb2, ws)
        assert np.array_equal(la2, lb2) and ta2 == tb2
        assert 0 <= tb2 < n2
        assert tb2 == O.argmax_tiled(lb2.view(np.float16))
        # a repeat of the first input after the smaller call
        (la3, ta3), (lb3, tb3) = _pair(Q, w, rows, xb1, ws)
        assert np.array_equal(lb3, la) and tb3 == ta


def test_noalloc_under_graph_capture(gpu, Wt):
    """Captured in a hipGraph (no allocation inside the capture) and replayed
    three times with eager calls between the replays; each replay matches the
    eager result."""
    Q = gpu
    n = 40000
    W = Wt.synthetic_f16_matrix(n, 1024, seed=SEED, tensor=3)
    x = Wt.synthetic_x(1024, SEED, 3)
    stream = Q.Stream()
    with Q.DeviceBuffer.from_array(W) as w, Q.DeviceBuffer.from_array(x) as xb, \
            Q.DeviceBuffer(2 * n) as lg, Q.DeviceBuffer(16) as tk, \
            Q.DeviceBuffer(2 * n) as lg_e, Q.DeviceBuffer(16) as tk_e:
        Q.f16_gemv_argmax_rows_noalloc(w, n, xb, lg_e, tk_e, stream)
        stream.synchronize()
        want_l, want_t = lg_e.download(np.uint16), int(tk_e.download(np.int32, 1)[0])
        graph = Q.Graph(stream, lambda: Q.f16_gemv_argmax_rows_noalloc(w, n, xb, lg, tk, stream))
        try:
            for i in range(3):
                lg.fill(0)
                tk.fill(0xFF)
                print(f"graph replay {i}", flush=True)
                graph.launch(stream)
                stream.synchronize()
                assert np.array_equal(lg.download(np.uint16), want_l), i
                assert int(tk.download(np.int32, 1)[0]) == want_t, i
                Q.f16_gemv_argmax_rows_noalloc(w, n // 2, xb, lg_e, tk_e, stream)
                stream.synchronize()
        finally:
            graph.destroy()
            stream.destroy()


def test_noalloc_validates_before_launch(gpu):
    Q = gpu
    L = Q.load_library()
    assert L.f16_gemv_argmax_rows_noalloc(None, 10, 0x10000, None, 0x10000, None) == \
        Q.Q8_ERR_NULL_POINTER
    assert L.f16_gemv_argmax_rows_noalloc(0x10000, 0, 0x10000, None, 0x10000, None) == \
        Q.Q8_ERR_BAD_SHAPE
    assert L.f16_gemv_argmax_rows_noalloc(0x10000, 1 << 31, 0x10000, None, 0x10000, None) == \
        Q.Q8_ERR_BAD_SHAPE
    assert "n_rows" in Q.last_error()
