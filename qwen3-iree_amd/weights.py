"""Weight preparation for the decode GEMV path (host side, numpy).

The reference converts GGUF tensors offline (tools/create_q8_irpa.py): Q8_0
weights stay as raw 34-byte blocks in GGUF's native [N, K] row order and are
stacked per layer into [28, BPL] byte tensors (create_q8_irpa.py:185-207), with
gate and up concatenated byte-wise into one [6144, 1024] weight
(create_q8_irpa.py:209-224).  This module produces exactly those byte layouts
from float weights, and the seeded synthetic inputs the benchmarks and tests
use (no checkpoint is available offline).
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np

BLOCK_ELEMS = 32
BLOCK_BYTES = 34
WEIGHT_STD = 0.02


def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """Q8_0 bytes of a float array, tools/create_q8_irpa.py:103-118.

    Per 32-element block: scale = max|w| / 127 in f32 (0 -> 1.0),
    q = round-half-even(w / scale) clipped to [-128, 127], then the scale
    stored as f16 little-endian (bytes 0-1) followed by the 32 int8 q.
    """
    flat = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    if flat.size % BLOCK_ELEMS:
        raise ValueError(f"element count {flat.size} is not a multiple of {BLOCK_ELEMS}")
    blocks = flat.reshape(-1, BLOCK_ELEMS)
    scale = (np.max(np.abs(blocks), axis=1, keepdims=True) / np.float32(127.0)).astype(np.float32)
    scale = np.where(scale == 0, np.float32(1.0), scale)
    q = np.clip(np.round(blocks / scale), -128, 127).astype(np.int8)
    out = np.empty((blocks.shape[0], BLOCK_BYTES), np.uint8)
    out[:, :2] = scale.astype(np.float16).view(np.uint8)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def dequant_q8_0(raw: np.ndarray) -> np.ndarray:
    """f32 values of Q8_0 bytes, tools/create_q8_irpa.py:121-129."""
    r = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, BLOCK_BYTES)
    scale = r[:, :2].copy().view(np.float16).astype(np.float32)
    return (scale * r[:, 2:].view(np.int8).astype(np.float32)).reshape(-1)


def concat_gate_up(gate_q8: np.ndarray, up_q8: np.ndarray) -> np.ndarray:
    """gate_up layer bytes: gate rows then up rows (create_q8_irpa.py:213-221)."""
    return np.concatenate([np.asarray(gate_q8, np.uint8).reshape(-1),
                           np.asarray(up_q8, np.uint8).reshape(-1)])


def stack_layers(layers: list[np.ndarray]) -> np.ndarray:
    """[L, BPL] stacked byte tensor (create_q8_irpa.py:199-204)."""
    return np.stack([np.asarray(l, np.uint8).reshape(-1) for l in layers])


def _rng(*key: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence(list(key))))


def synthetic_q8_layer(n: int, k: int, seed: int, layer: int, tensor: int) -> np.ndarray:
    """One layer's Q8_0 bytes for W ~ N(0, 0.02) of shape [n, k]."""
    w = _rng(seed, tensor, layer).standard_normal((n, k), dtype=np.float32)
    w *= np.float32(WEIGHT_STD)
    return quantize_q8_0(w)


def synthetic_q8_stack(n: int, k: int, layers: int, seed: int, tensor: int,
                       workers: int = 8) -> np.ndarray:
    """[layers, n*k/32*34] stacked Q8_0 bytes, one independent seed per layer."""
    bpl = n * k // BLOCK_ELEMS * BLOCK_BYTES
    out = np.empty((layers, bpl), np.uint8)

    def one(l: int) -> None:
        out[l] = synthetic_q8_layer(n, k, seed, l, tensor)

    with ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        list(ex.map(one, range(layers)))
    return out


def synthetic_f16_matrix(n: int, k: int, seed: int, tensor: int, workers: int = 8) -> np.ndarray:
    """f16(N(0, 0.02)) of shape [n, k], generated in row chunks."""
    out = np.empty((n, k), np.float16)
    chunk = 8192
    starts = list(range(0, n, chunk))

    def one(i: int) -> None:
        s = starts[i]
        e = min(n, s + chunk)
        w = _rng(seed, tensor, i).standard_normal((e - s, k), dtype=np.float32)
        w *= np.float32(WEIGHT_STD)
        out[s:e] = w.astype(np.float16)

    with ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        list(ex.map(one, range(len(starts))))
    return out


def synthetic_x(k: int, seed: int, index: int = 0) -> np.ndarray:
    """x = f16(N(0, 1)) of length k."""
    return _rng(seed, 1_000_003, index).standard_normal(k, dtype=np.float32).astype(np.float16)
