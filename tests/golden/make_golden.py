#!/usr/bin/env python3
"""Writes the golden fixtures in this directory (golden_vectors.npz).

The reference ships no test vectors, so these are computed independently of
both the oracle and the kernels: Q8_0 blocks are built directly from random
f16 scales and int8 values (no quantizer involved), the expected GEMV outputs
are float64 sums rounded once to f16 by numpy, and the expected tokens come
from a brute-force argmax over those f16 logits.  Deterministic: rerunning
reproduces the file bit for bit.

    python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "golden_vectors.npz"


def q8_rows(rng, n, k):
    nb = n * k // 32
    scale = (rng.uniform(0.0002, 0.0008, nb)).astype(np.float16)
    q = rng.integers(-128, 128, (nb, 32)).astype(np.int8)
    q[::7, rng.integers(0, 32)] = 127
    raw = np.concatenate([scale.view(np.uint8).reshape(nb, 2), q.view(np.uint8)], axis=1)
    w = scale.astype(np.float64)[:, None] * q.astype(np.float64)
    return raw.reshape(-1), w.reshape(n, k)


def first_max(v16):
    f = v16.astype(np.float64)
    ok = ~np.isnan(f) & (f > -np.inf)
    if not ok.any():
        return -1
    return int(np.nonzero(ok & (f == f[ok].max()))[0][0])


def main():
    rng = np.random.default_rng(777)
    out = {}
    for k in (1024, 2048, 3072):
        n = 8
        raw, w = q8_rows(rng, n, k)
        x = rng.standard_normal(k).astype(np.float16)
        y64 = w @ x.astype(np.float64)
        out[f"q8_k{k}_w"] = raw
        out[f"q8_k{k}_x"] = x
        out[f"q8_k{k}_y"] = y64.astype(np.float16)
        out[f"q8_k{k}_y64"] = y64
        out[f"q8_k{k}_sumabs"] = np.abs(w) @ np.abs(x.astype(np.float64))
    # vocab-shaped f16 GEMV (K = 1024) with an exact tie between rows 5 and 29
    n = 32
    W = (rng.standard_normal((n, 1024)) * 0.02).astype(np.float16)
    x = rng.standard_normal(1024).astype(np.float16)
    hot = (np.sign(x.astype(np.float32)) * 0.03).astype(np.float16)
    W[5] = hot
    W[29] = hot
    y64 = W.astype(np.float64) @ x.astype(np.float64)
    logits = y64.astype(np.float16)
    out["f16_w"] = W
    out["f16_x"] = x
    out["f16_y"] = logits
    out["f16_y64"] = y64
    out["f16_sumabs"] = np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64))
    out["f16_token"] = np.array([first_max(logits)], np.int64)
    # argmax vectors (f16) with their expected tokens
    cases = []
    v = rng.integers(-50, 50, 700).astype(np.float16); v[[255, 256, 600]] = 60; cases.append(v)
    v = np.full(513, -np.inf, np.float16); v[[3, 400]] = np.nan; cases.append(v)
    v = np.zeros(257, np.float16); v[::2] = -0.0; cases.append(v)
    v = rng.standard_normal(1000).astype(np.float16); v[999] = np.inf; v[10] = np.nan; cases.append(v)
    for i, v in enumerate(cases):
        out[f"argmax_{i}_v"] = v
        out[f"argmax_{i}_token"] = np.array([first_max(v)], np.int64)
    np.savez_compressed(OUT, **out)
    print(OUT, OUT.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
