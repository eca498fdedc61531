"""The full decode step at the configured context (Qwen3-0.6B, batch 1,
context 1024: max_seq 1024, position 1023 over a seeded history in every
layer's 1023 cached slots) against the oracle's own step, in both step modes
(one launch; one launch per phase).  The reference's step is
@generate's inner loop, model/qwen3_full.mlir:1431-1526.

Checks, as for the short-context steps:
  * the vocab stage against the oracle applied to the GPU's own final norm:
    every logit under the GEMV rule;
  * the token = the lowest index of the GPU's maximal f16 logit (bit-exact);
  * against the oracle's whole chain: logits within 2e-2 relative L2, and the
    same token whenever the oracle's top-2 margin exceeds 2 max|dlogit|;
  * the new position's K/V slots of every layer written, the history intact;
  * both modes give the same bits (logits, token, caches).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAX_SEQ = 1024
POS = 1023
TOKEN = 1234


@pytest.fixture(scope="module")
def D():
    from qwen3_iree_amd import decode

    return decode


@pytest.fixture(scope="module")
def dmodel(gpu, D, model_host):
    m = D.DeviceWeights(model_host)
    yield m
    m.free()


@pytest.fixture(scope="module")
def history(D):
    rng = np.random.default_rng(20261202)
    k = rng.standard_normal((D.LAYERS * MAX_SEQ, D.KV_DIM), dtype=np.float32).astype(np.float16)
    v = (np.float32(0.6) * rng.standard_normal((D.LAYERS * MAX_SEQ, D.KV_DIM),
                                               dtype=np.float32)).astype(np.float16)
    return k, v


@pytest.fixture(scope="module")
def oracle_step(O, model_host, history):
    kc, vc = history[0].copy(), history[1].copy()
    tok, logits, hl = O.decode_step(model_host, kc, vc, MAX_SEQ, TOKEN, POS, True, True)
    return tok, logits, hl, kc, vc


def f64(a):
    return np.asarray(a, np.float64)


def run_mode(D, dmodel, history, mode):
    before = D.step_mode()
    D.set_step_mode(mode)
    try:
        s = D.DecodeSession(dmodel, MAX_SEQ)
        s.k_cache.upload(history[0])
        s.v_cache.upload(history[1])
        s.set_state(TOKEN, POS)
        print(f"mode {mode}: step at position {POS} of {MAX_SEQ}", flush=True)
        s.step(advance=False, logits=True)
        status = s.check_status()
        out = {"state": s.get_state(), "logits": s.read_logits(),
               "on": s.scratch_f16("on", 1024), "status": status,
               "k": s.k_cache.download(np.float16).reshape(-1, D.KV_DIM),
               "v": s.v_cache.download(np.float16).reshape(-1, D.KV_DIM)}
        s.free()
        return out
    finally:
        D.set_step_mode(before)


@pytest.fixture(scope="module")
def gpu_steps(D, dmodel, history):
    return {mode: run_mode(D, dmodel, history, mode) for mode in (1, 0)}


@pytest.mark.parametrize("mode", [1, 0], ids=["single_launch", "per_phase"])
def test_full_step_context_1024_matches_oracle(O, D, model_host, history, oracle_step,
                                               gpu_steps, mode):
    w = model_host
    g = gpu_steps[mode]
    ref_tok, ref_logits, hl, kc_ref, vc_ref = oracle_step
    tok, pos = g["state"]
    logits = g["logits"]
    assert pos == POS and g["status"] == 0
    # final norm close to the oracle's (its input differs slightly)
    on_ref = O.rmsnorm(hl[-1], w.output_norm)
    assert np.linalg.norm(f64(g["on"]) - f64(on_ref)) / np.linalg.norm(f64(on_ref)) < 1e-2
    # vocab stage against the GPU's own normalised input: the GEMV rule
    y_ref = O.f16_gemv(w.output_w, g["on"])
    _, mag = O.f16_gemv_f64(w.output_w, g["on"])
    rep = O.gemv_tolerance_report(logits, y_ref, mag)
    assert rep["fail"] == 0, rep
    # token: lowest index of the GPU's maximal f16 logit
    lf = logits.astype(np.float32)
    assert tok == int(np.flatnonzero(lf == lf.max())[0]) == O.argmax_tiled(logits)
    # the oracle's whole chain
    dl = np.abs(f64(logits) - f64(ref_logits))
    rel = np.linalg.norm(dl) / np.linalg.norm(f64(ref_logits))
    assert rel < 2e-2, rel
    srt = np.sort(f64(ref_logits))
    margin = srt[-1] - srt[-2]
    if margin > 2 * dl.max():
        assert tok == ref_tok, (tok, ref_tok, margin, dl.max())
    print(f"mode {mode}: token {tok} (oracle {ref_tok}), logits rel L2 {rel:.2e}, margin "
          f"{margin:.4f}, max |dlogit| {dl.max():.4f}", flush=True)
    # caches: history untouched, slot POS of every layer written and close to
    # the oracle's (the K slot is RoPE'd, the V slot the raw projection)
    slots = np.arange(D.LAYERS) * MAX_SEQ + POS
    hist = np.ones(D.LAYERS * MAX_SEQ, bool)
    hist[slots] = False
    assert np.array_equal(g["k"][hist], history[0][hist])
    assert np.array_equal(g["v"][hist], history[1][hist])
    for got, want in ((g["k"][slots], kc_ref[slots]), (g["v"][slots], vc_ref[slots])):
        assert np.isfinite(got.astype(np.float32)).all()
        assert np.linalg.norm(f64(got) - f64(want)) / np.linalg.norm(f64(want)) < 2e-2


def test_full_step_context_1024_modes_bit_identical(gpu_steps):
    a, b = gpu_steps[1], gpu_steps[0]
    assert a["state"] == b["state"]
    assert np.array_equal(a["logits"].view(np.uint16), b["logits"].view(np.uint16))
    assert np.array_equal(a["k"].view(np.uint16), b["k"].view(np.uint16))
    assert np.array_equal(a["v"].view(np.uint16), b["v"].view(np.uint16))
