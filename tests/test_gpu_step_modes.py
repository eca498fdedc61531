"""The single-launch decode step (qwen3_set_step_mode(1): one
launch, phases handing activations over through tagged words) against the
launch-per-phase step (mode 0, itself checked stage by stage against the
oracle).  Both run the same operations in the same order, so logits, tokens,
positions and the KV cache must agree bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


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
def single(gpu, D, dmodel):
    before = D.step_mode()
    D.set_step_mode(1)  # raises if the device cannot run the single-launch step
    yield
    D.set_step_mode(before)


def run_steps(D, dmodel, mode, max_seq, token, pos, n, history=None):
    D.set_step_mode(mode)
    s = D.DecodeSession(dmodel, max_seq)
    if history is not None:
        s.k_cache.upload(history[0])
        s.v_cache.upload(history[1])
    s.set_state(token, pos)
    out = []
    for i in range(n):
        print(f"mode {mode} step {i}", flush=True)
        s.step(advance=True, logits=True)
        out.append((s.get_state(), s.read_logits(), s.status()))
    k, v = s.cache_rows(27, 0, max_seq)
    k0, v0 = s.cache_rows(0, 0, max_seq)
    s.free()
    return out, (k, v, k0, v0)


@pytest.mark.parametrize("max_seq,pos,n", [(16, 0, 5), (1024, 1020, 3), (40, 7, 2),
                                           (20000, 19998, 2)])
def test_single_launch_matches_per_phase(D, dmodel, single, max_seq, pos, n):
    rng = np.random.default_rng(max_seq + pos)
    hist = None
    if pos > 0:
        size = 28 * max_seq * 1024
        base = min(size, 1 << 22)  # long caches: a random block repeated
        k = rng.standard_normal(base, dtype=np.float32).astype(np.float16)
        v = (0.6 * rng.standard_normal(base, dtype=np.float32)).astype(np.float16)
        hist = (np.resize(k, size), np.resize(v, size))
    a, ca = run_steps(D, dmodel, 0, max_seq, 4321, pos, n, hist)
    b, cb = run_steps(D, dmodel, 1, max_seq, 4321, pos, n, hist)
    for i, ((sa, la, st_a), (sb, lb, st_b)) in enumerate(zip(a, b)):
        assert sa == sb, (i, sa, sb)
        assert st_a == st_b, (i, st_a, st_b)
        assert np.array_equal(la.view(np.uint16), lb.view(np.uint16)), i
    for x, y in zip(ca, cb):
        assert np.array_equal(x.view(np.uint16), y.view(np.uint16))


def test_single_launch_generate_and_prefill(D, dmodel, single):
    prompt = [17, 4, 151935, 99, 0, 12]
    res = {}
    for mode in (0, 1):
        D.set_step_mode(mode)
        s = D.DecodeSession(dmodel, 32)
        s.set_state(-1, 0)
        print(f"mode {mode}: prefill + generate", flush=True)
        s.prefill(prompt)
        st = s.get_state()
        toks = s.generate(9, eos_id=-3)
        res[mode] = (st, toks.tolist(), s.get_state(), s.status())
        s.free()
    assert res[0] == res[1]
    assert res[1][2][1] == len(prompt) + 9


def test_single_launch_repeated_steps_keep_sequence(D, dmodel, single):
    """Many launches on one scratch: every step's tags differ from the last."""
    D.set_step_mode(1)
    s = D.DecodeSession(dmodel, 64)
    s.set_state(5, 0)
    for i in range(40):
        s.step(advance=True, logits=False)
    tok, pos = s.get_state()
    assert pos == 40 and s.status() == 0 and 0 <= tok < D.VOCAB
    s.free()


def test_single_launch_abort_is_reported_and_recoverable(gpu, D, dmodel, single):
    """A poll limit of one round makes the step's bounded waits give up (the
    host forces the condition; every workgroup still exits normally): status
    bit 1 is set and the position is not advanced; qwen3_check_status,
    qwen3_decode_step_checked and qwen3_generate report Q8_ERR_STEP_ABORTED;
    a step launched on the scratch while bit 1 is set does nothing (token and
    position stay); a scratch reset clears the status and the step then gives
    the bits of a fresh session's step."""
    Q = gpu
    ref = D.DecodeSession(dmodel, 64)
    ref.set_state(77, 5)
    ref.step(advance=False, logits=True)
    want_state, want_logits = ref.get_state(), ref.read_logits()
    ref.free()

    s = D.DecodeSession(dmodel, 64)
    s.set_state(77, 5)
    D.set_step_spin_limit(1)
    try:
        print("single-launch step with a one-round poll limit", flush=True)
        s.step(advance=True, logits=True)
        s.synchronize()
    finally:
        D.set_step_spin_limit(0)
    assert s.status() & 2
    assert s.get_state() == (77, 5)
    with pytest.raises(Q.Q8GemvError) as e:
        s.check_status()
    assert e.value.code == Q.Q8_ERR_STEP_ABORTED
    with pytest.raises(Q.Q8GemvError) as e:
        s.step_checked()
    assert e.value.code == Q.Q8_ERR_STEP_ABORTED
    with pytest.raises(Q.Q8GemvError) as e:
        s.generate(4, eos_id=-1)
    assert e.value.code == Q.Q8_ERR_STEP_ABORTED

    print("steps behind the aborted one", flush=True)
    for _ in range(3):
        s.step(advance=True, logits=True)
    s.synchronize()
    assert s.get_state() == (77, 5)
    assert s.status() & 2  # sticky until the scratch is reset

    s.reset_scratch()
    assert s.check_status() == 0
    s.step(advance=False, logits=True)
    assert s.get_state() == want_state
    assert np.array_equal(s.read_logits().view(np.uint16), want_logits.view(np.uint16))
    toks = s.generate(4, eos_id=-1)
    assert len(toks) == 4 and s.get_state()[1] == 9 and s.check_status() == 0
    s.free()


def per_phase_generate(D, dmodel, token, pos, n, max_seq=64):
    before = D.step_mode()
    D.set_step_mode(0)
    try:
        s = D.DecodeSession(dmodel, max_seq)
        s.set_state(token, pos)
        toks = s.generate(n, eos_id=-1)
        out = (toks.tolist(), s.get_state(), s.status())
        s.free()
    finally:
        D.set_step_mode(before)
    return out


def test_generate_falls_back_when_every_launch_gives_up(gpu, D, dmodel, single):
    """A one-round poll limit (set from the host; every workgroup still exits
    normally) makes the first single launch give up: qwen3_generate re-runs
    the batch from that step with the per-phase launches and finishes the
    loop in that mode, returning the per-phase loop's tokens and state with
    status bit 2 (fallback) instead of bit 1."""
    want_toks, want_state, _ = per_phase_generate(D, dmodel, 77, 5, 8)
    s = D.DecodeSession(dmodel, 64)
    s.set_state(77, 5)
    n0 = D.step_fallback_count()
    D.set_step_spin_limit(1)
    try:
        print("generate 8 with a one-round poll limit", flush=True)
        toks = s.generate(8, eos_id=-1)
        s.synchronize()
    finally:
        D.set_step_spin_limit(0)
    assert toks.tolist() == want_toks
    assert s.get_state() == want_state
    st = s.check_status()
    assert st & 4 and not st & 2
    assert D.step_fallback_count() == n0 + 1
    s.free()

