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
