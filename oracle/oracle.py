"""numpy-facing wrapper of the CPU oracle (oracle/q8_oracle.c).

TEST INFRASTRUCTURE ONLY.  The oracle is the checker for the HIP kernels:
only tests/, the smoke check and the benchmark's CPU-baseline leg import this
module.  The product never calls it.

Each function restates the reference arithmetic; the C source cites the
reference file:line for each one.  Half-precision arrays are numpy float16
(their raw bits are what the C side reads).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "liboracle.so"

_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def build() -> Path:
    """Compile liboracle.so with the Makefile next to this file."""
    import subprocess

    subprocess.run(["make", "-s", "-B", "-C", str(_HERE), "liboracle.so"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle library not built: {LIB_PATH} (run oracle.build())")
        L = ctypes.CDLL(str(LIB_PATH))
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f16_to_f32_array.argtypes = [_P, _P, _I64]
        L.oracle_f32_to_f16_array.argtypes = [_P, _P, _I64]
        L.oracle_q8_quantize.argtypes = [_P, _I64, _P]
        L.oracle_q8_quantize.restype = ctypes.c_int
        L.oracle_q8_dequant.argtypes = [_P, _I64, _P]
        L.oracle_q8_gemv.argtypes = [_P, _I64, _I64, _P, _P]
        L.oracle_q8_gemv_f64.argtypes = [_P, _I64, _I64, _P, _P, _P]
        L.oracle_f16_gemv.argtypes = [_P, _I64, _I64, _P, _P]
        L.oracle_f16_gemv_f64.argtypes = [_P, _I64, _I64, _P, _P, _P]
        L.oracle_argmax_tiled.argtypes = [_P, _I64, _I64]
        L.oracle_argmax_tiled.restype = ctypes.c_int64
        L.oracle_num_threads.restype = ctypes.c_int
        L.oracle_set_num_threads.argtypes = [ctypes.c_int]
        L.oracle_set_num_threads.restype = None
        # decode_oracle.c
        L.oracle_rmsnorm.argtypes = [_P, _P, ctypes.c_int, ctypes.c_float, _P]
        L.oracle_head_rmsnorm.argtypes = [_P, ctypes.c_int, _P, ctypes.c_float, _P]
        L.oracle_rope.argtypes = [_P, ctypes.c_int, ctypes.c_int32, _P]
        L.oracle_attention.argtypes = [_P, _P, _P, ctypes.c_int, ctypes.c_float, _P]
        L.oracle_swiglu.argtypes = [_P, _P, ctypes.c_int, _P]
        L.oracle_add_f16.argtypes = [_P, _P, ctypes.c_int, _P]
        L.oracle_decode_layer.argtypes = [_P, ctypes.c_int, _P, _P, _I64, ctypes.c_int32, _P, _P,
                                          _P]
        L.oracle_decode_step.argtypes = [_P, _P, _P, _I64, ctypes.c_int32, ctypes.c_int32, _P, _P]
        L.oracle_decode_step.restype = ctypes.c_int64
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle needs contiguous arrays"
    return a.ctypes.data


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.float16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.float16)
    lib().oracle_f32_to_f16_array(_ptr(f), _ptr(out), f.size)
    return out


def q8_quantize(w: np.ndarray) -> np.ndarray:
    """Q8_0 bytes (uint8, n/32*34) of a float32 array; create_q8_irpa.py:103-118."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    if w.size % 32:
        raise ValueError("element count must be a multiple of 32")
    out = np.empty(w.size // 32 * 34, np.uint8)
    rc = lib().oracle_q8_quantize(_ptr(w), w.size, _ptr(out))
    assert rc == 0
    return out


def q8_dequant(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    nb = blocks.size // 34
    out = np.empty(nb * 32, np.float32)
    lib().oracle_q8_dequant(_ptr(blocks), nb, _ptr(out))
    return out


def q8_dequant_f16(w_layer: np.ndarray, N: int, K: int) -> np.ndarray:
    """The f16 [N, K] matrix the reference's @prefill reads for a Q8_0 layer
    matrix: each weight f32(scale) * f32(q), exact in f32, rounded once to f16
    (tools/convert_gguf_to_irpa.py:28-44 dequant_q8_0, then .astype(np.float16)
    at :178 and :197-198)."""
    w_layer = np.ascontiguousarray(w_layer, dtype=np.uint8).reshape(-1)
    assert w_layer.size >= N * K // 32 * 34 and K % 32 == 0
    return f32_to_f16(q8_dequant(w_layer[:N * K // 32 * 34])).reshape(N, K)


def q8_gemv(w_layer: np.ndarray, N: int, K: int, x: np.ndarray) -> np.ndarray:
    """f16 y[N] in the reference MLIR kernels' f32 order."""
    w_layer = np.ascontiguousarray(w_layer, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float16)
    assert w_layer.size >= N * K // 32 * 34 and x.size >= K and K % 32 == 0
    y = np.empty(N, np.float16)
    lib().oracle_q8_gemv(_ptr(w_layer), N, K, _ptr(x), _ptr(y))
    return y


def q8_gemv_f64(w_layer: np.ndarray, N: int, K: int, x: np.ndarray):
    """(y_f64, sum_abs) for the same GEMV computed in float64."""
    w_layer = np.ascontiguousarray(w_layer, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float16)
    assert w_layer.size >= N * K // 32 * 34 and x.size >= K and K % 32 == 0
    y = np.empty(N, np.float64)
    mag = np.empty(N, np.float64)
    lib().oracle_q8_gemv_f64(_ptr(w_layer), N, K, _ptr(x), _ptr(y), _ptr(mag))
    return y, mag


def f16_gemv(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.float16)
    x = np.ascontiguousarray(x, dtype=np.float16)
    N, K = W.shape
    assert x.size == K
    y = np.empty(N, np.float16)
    lib().oracle_f16_gemv(_ptr(W), N, K, _ptr(x), _ptr(y))
    return y


def f16_gemv_f64(W: np.ndarray, x: np.ndarray):
    W = np.ascontiguousarray(W, dtype=np.float16)
    x = np.ascontiguousarray(x, dtype=np.float16)
    N, K = W.shape
    y = np.empty(N, np.float64)
    mag = np.empty(N, np.float64)
    lib().oracle_f16_gemv_f64(_ptr(W), N, K, _ptr(x), _ptr(y), _ptr(mag))
    return y, mag


def argmax_tiled(v: np.ndarray, tile: int = 256) -> int:
    v = np.ascontiguousarray(v, dtype=np.float16).reshape(-1)
    return int(lib().oracle_argmax_tiled(_ptr(v), v.size, tile))


def num_threads() -> int:
    return int(lib().oracle_num_threads())


def set_num_threads(n: int) -> None:
    """OpenMP threads of the oracle's following calls."""
    lib().oracle_set_num_threads(int(n))


# ---------------------------------------------------------- decode step ----
# Qwen3-0.6B shapes (model/qwen3_full.mlir:29-64).
LAYERS, HIDDEN, Q_HEADS, KV_HEADS, HEAD_DIM, FFN, VOCAB = 28, 1024, 16, 8, 128, 3072, 151936
Q_DIM, KV_DIM = Q_HEADS * HEAD_DIM, KV_HEADS * HEAD_DIM
EPS = float(np.float32(9.99999997e-7))
ATTN_SCALE = float(np.float32(1.0 / 11.313708498984761))
WEIGHT_FIELDS = ("token_embd", "attn_norm", "ffn_norm", "q_norm", "k_norm", "wq", "wk", "wv",
                 "wo", "wgu", "wdn", "output_norm", "output_w")


class _Weights(ctypes.Structure):
    _fields_ = [(f, _P) for f in WEIGHT_FIELDS]


class _Trace(ctypes.Structure):
    _fields_ = [("q_roped", ctypes.c_uint16 * Q_DIM), ("k_roped", ctypes.c_uint16 * KV_DIM),
                ("v", ctypes.c_uint16 * KV_DIM), ("attn", ctypes.c_uint16 * Q_DIM),
                ("res1", ctypes.c_uint16 * HIDDEN), ("act", ctypes.c_uint16 * FFN)]


def _f16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float16)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = EPS) -> np.ndarray:
    x, w = _f16(x).reshape(-1), _f16(w).reshape(-1)
    assert x.size == w.size
    out = np.empty_like(x)
    lib().oracle_rmsnorm(_ptr(x), _ptr(w), x.size, eps, _ptr(out))
    return out


def head_rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = EPS) -> np.ndarray:
    x, w = _f16(x).reshape(-1), _f16(w).reshape(-1)
    assert w.size == HEAD_DIM and x.size % HEAD_DIM == 0
    out = np.empty_like(x)
    lib().oracle_head_rmsnorm(_ptr(x), x.size // HEAD_DIM, _ptr(w), eps, _ptr(out))
    return out


def rope(x: np.ndarray, pos: int) -> np.ndarray:
    x = _f16(x).reshape(-1)
    assert x.size % HEAD_DIM == 0
    out = np.empty_like(x)
    lib().oracle_rope(_ptr(x), x.size // HEAD_DIM, int(pos), _ptr(out))
    return out


def attention(q: np.ndarray, k_rows: np.ndarray, v_rows: np.ndarray,
              scale: float = ATTN_SCALE) -> np.ndarray:
    """q f16[2048]; k_rows, v_rows f16[ctx, 8, 128] -> f16[2048]."""
    q = _f16(q).reshape(-1)
    k_rows, v_rows = _f16(k_rows).reshape(-1, KV_DIM), _f16(v_rows).reshape(-1, KV_DIM)
    assert q.size == Q_DIM and k_rows.shape == v_rows.shape
    out = np.empty(Q_DIM, np.float16)
    lib().oracle_attention(_ptr(q), _ptr(k_rows), _ptr(v_rows), k_rows.shape[0], scale, _ptr(out))
    return out


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    gate, up = _f16(gate).reshape(-1), _f16(up).reshape(-1)
    assert gate.size == up.size
    out = np.empty_like(gate)
    lib().oracle_swiglu(_ptr(gate), _ptr(up), gate.size, _ptr(out))
    return out


def add_f16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a, b = _f16(a).reshape(-1), _f16(b).reshape(-1)
    out = np.empty_like(a)
    lib().oracle_add_f16(_ptr(a), _ptr(b), a.size, _ptr(out))
    return out


def _weights_struct(w) -> _Weights:
    """w: an object with the WEIGHT_FIELDS attributes as contiguous numpy arrays."""
    ptrs = []
    for f in WEIGHT_FIELDS:
        a = getattr(w, f)
        assert a.flags["C_CONTIGUOUS"], f
        ptrs.append(a.ctypes.data)
    return _Weights(*ptrs)


def decode_layer(w, layer: int, k_cache: np.ndarray, v_cache: np.ndarray, max_seq: int,
                 pos: int, h_in: np.ndarray) -> tuple[np.ndarray, dict]:
    """One layer at position pos; updates k_cache / v_cache ([28*max_seq, 1024]
    f16) in place.  Returns (h_out, trace dict of intermediates)."""
    assert k_cache.dtype == np.float16 and k_cache.flags["C_CONTIGUOUS"]
    assert v_cache.dtype == np.float16 and v_cache.flags["C_CONTIGUOUS"]
    assert k_cache.size == LAYERS * max_seq * KV_DIM == v_cache.size
    h_in = _f16(h_in).reshape(-1)
    h_out = np.empty(HIDDEN, np.float16)
    tr = _Trace()
    ws = _weights_struct(w)
    lib().oracle_decode_layer(ctypes.byref(ws), int(layer), _ptr(k_cache), _ptr(v_cache),
                              int(max_seq), int(pos), _ptr(h_in), _ptr(h_out), ctypes.byref(tr))
    trace = {name: np.frombuffer(bytes(getattr(tr, name)), np.float16).copy()
             for name, _ in _Trace._fields_}
    return h_out, trace


def decode_step(w, k_cache: np.ndarray, v_cache: np.ndarray, max_seq: int, token: int,
                pos: int, want_logits: bool = True, want_hidden: bool = False):
    """One token; updates the caches in place.  Returns (token, logits | None,
    h_layers [29, 1024] | None)."""
    assert k_cache.size == LAYERS * max_seq * KV_DIM == v_cache.size
    logits = np.empty(VOCAB, np.float16) if want_logits else None
    hl = np.empty((LAYERS + 1, HIDDEN), np.float16) if want_hidden else None
    ws = _weights_struct(w)
    tok = lib().oracle_decode_step(ctypes.byref(ws), _ptr(k_cache), _ptr(v_cache), int(max_seq),
                                   int(token), int(pos),
                                   _ptr(logits) if logits is not None else None,
                                   _ptr(hl) if hl is not None else None)
    return int(tok), logits, hl


# ------------------------------------------------------ generation loop ----

def generate_control(step, first_token: int, start_pos: int, max_new: int, eos_id: int,
                     batch: int = 4):
    """@generate's control flow (qwen3_full.mlir:1396-1534) around
    step(token, pos) -> next token.

    out = zeros(max_new); batches of min(4, remaining) steps (:1412, 1419-1420),
    each writing its token to out[idx] and advancing pos (:1512-1523); after a
    batch the last token is compared with eos (:1528-1531).  The first token
    is an input only (:1427).  Returns (out int64 [max_new], count).
    """
    out = np.zeros(max_new, np.int64)
    tok, pos, idx, not_eos = int(first_token), int(start_pos), 0, True
    while idx < max_new and not_eos:
        for _ in range(min(batch, max_new - idx)):
            tok = int(step(tok, pos))
            out[idx] = tok
            idx += 1
            pos += 1
        not_eos = tok != eos_id
    return out, idx


def run_control(step_logits, step, prompt, max_gen: int, eos_id: int):
    """@run (qwen3_full.mlir:2113-2167) with prompt ingestion as per-token
    decode steps (@prefill_all, :1541-1561): step_logits(token, pos) -> f16
    logits for each prompt token at positions 0..n-1; the first token is the
    lowest-index argmax of the last logits; then @generate from position n."""
    prompt = [int(t) for t in prompt]
    logits = None
    for i, t in enumerate(prompt):
        logits = step_logits(t, i)
    first = argmax_tiled(logits)
    return generate_control(step, first, len(prompt), max_gen, eos_id)


# ------------------------------------------------------------ tolerance ----

def ulp_f16(v: np.ndarray) -> np.ndarray:
    """Spacing of binary16 at |v| (2^-24 in the subnormal range)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    a = np.where(np.isfinite(a), a, 65504.0)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return np.exp2(e - 10.0)


def gemv_tolerance_report(got: np.ndarray, ref: np.ndarray, sum_abs: np.ndarray,
                          rel: float = 1e-3, ulps: float = 2.0,
                          noise_mult: float = 8.0) -> dict:
    """Check f16 GEMV outputs against the reference-order f16 outputs.

    Primary rule: |got - ref| <= 2 ulp_f16(ref)  or  <= 1e-3 * |ref|.
    Noise floor: two f32 summation orders of the same K-term dot product may
    each differ from the exact value by a few units of 2^-24 * sum|terms|; where
    cancellation makes |ref| tiny that exceeds 2 f16 ulp.  Outputs within
    noise_mult * 2^-24 * sum|terms| pass on the floor; the report counts them so
    a test can bound how many outputs rely on it.
    """
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    d = np.abs(g - r)
    both_nan = np.isnan(g) & np.isnan(r)
    same_inf = np.isinf(g) & np.isinf(r) & (np.sign(g) == np.sign(r))
    d = np.where(both_nan | same_inf, 0.0, d)
    primary = (d <= ulps * ulp_f16(r)) | (d <= rel * np.abs(r))
    floor = noise_mult * 2.0 ** -24 * np.asarray(sum_abs, dtype=np.float64)
    on_floor = (~primary) & (d <= floor)
    fail = ~(primary | on_floor)
    return {
        "n": int(g.size),
        "fail": int(fail.sum()),
        "on_floor": int(on_floor.sum()),
        "max_abs_diff": float(np.nanmax(d)) if d.size else 0.0,
        "fail_idx": np.nonzero(fail)[0][:16].tolist(),
    }
