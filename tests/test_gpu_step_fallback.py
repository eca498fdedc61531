"""The single-launch decode step on a device it does not have to itself.

A single launch gives up (status bit 1) when a wait cannot complete; the host
forces that here with the library's test hook (qwen3_debug_force_step_abort:
the chosen launch's workgroup 0 gives up at its start, every workgroup still
exits normally) instead of provoking a real stall.  What must hold:
  * launches queued behind the one that gave up do nothing (token, position
    and out_tokens slots stay as the last completed step left them);
  * qwen3_generate, qwen3_prefill and qwen3_decode_step_checked re-run the
    steps that did nothing with the per-phase launches and return the tokens,
    positions, logits and cache rows of a per-phase run, bit for bit, with
    status bit 2 and the process-wide fallback count recording it;
  * single-launch steps of two sessions on two streams, enqueued interleaved,
    are ordered by the library and give each session's bits.
"""
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
    D.force_step_abort(-1)
    D.set_step_mode(before)


def in_mode(D, mode, fn):
    before = D.step_mode()
    D.set_step_mode(mode)
    try:
        return fn()
    finally:
        D.set_step_mode(before)


def session_result(s, layers=(0, 27)):
    rows = [s.cache_rows(l, 0, s.max_seq) for l in layers]
    return s.get_state(), [r.view(np.uint16).copy() for kv in rows for r in kv]


def same_cache(a, b):
    return all(np.array_equal(x, y) for x, y in zip(a, b))


@pytest.mark.parametrize("after", [0, 2, 3, 5])
def test_generate_resumes_mid_batch(D, dmodel, single, after):
    """The single launch `after` steps into qwen3_generate gives up (the first
    step of a batch, its middle, its last one, a later batch's): the loop
    re-runs from there per phase, with the per-phase loop's tokens, state and
    cache."""
    def run():
        s = D.DecodeSession(dmodel, 48)
        s.set_state(321, 3)
        toks = s.generate(10, eos_id=-1).tolist()
        st, cache = session_result(s)
        status = s.check_status()
        s.free()
        return toks, st, cache, status

    want = in_mode(D, 0, run)
    n0 = D.step_fallback_count()
    D.force_step_abort(after)
    print(f"generate 10, launch {after} forced to give up", flush=True)
    got = run()
    D.force_step_abort(-1)
    assert got[0] == want[0]
    assert got[1] == want[1] == (want[0][-1], 13)
    assert same_cache(got[2], want[2])
    assert got[3] & 4 and not got[3] & 2
    assert D.step_fallback_count() == n0 + 1


def test_launches_behind_an_abort_do_nothing(gpu, D, dmodel, single):
    """Three steps enqueued with no check between them, the second forced to
    give up: the first completes, the second and third leave token, position
    and their output untouched (status bit 1 makes them return at their
    start)."""
    s = D.DecodeSession(dmodel, 32)
    s.set_state(11, 4)
    D.force_step_abort(1)
    print("three steps, the second forced to give up", flush=True)
    s.step(advance=True, logits=False)
    s.step(advance=True, logits=False)
    s.step(advance=True, logits=False)
    s.synchronize()
    D.force_step_abort(-1)
    tok, pos = s.get_state()
    assert pos == 5 and s.status() & 2

    ref = D.DecodeSession(dmodel, 32)
    ref.set_state(11, 4)
    ref.step(advance=True, logits=False)
    assert ref.get_state() == (tok, pos)
    ref.free()
    s.free()


def test_prefill_resumes_after_an_abort(D, dmodel, single):
    prompt = [5, 151935, 17, 0, 42, 9, 1000]

    def run():
        s = D.DecodeSession(dmodel, 24)
        s.set_state(-1, 2)
        s.prefill(prompt)
        st, cache = session_result(s)
        status = s.check_status()
        s.free()
        return st, cache, status

    want = in_mode(D, 0, run)
    n0 = D.step_fallback_count()
    D.force_step_abort(4)
    print("prefill of 7 tokens, launch 4 forced to give up", flush=True)
    got = run()
    D.force_step_abort(-1)
    assert got[0] == want[0] and got[0][1] == 2 + len(prompt)
    assert same_cache(got[1], want[1])
    assert got[2] & 4 and not got[2] & 2
    assert D.step_fallback_count() == n0 + 1


def test_step_checked_reruns_per_phase(D, dmodel, single):
    def run(force):
        s = D.DecodeSession(dmodel, 40)
        s.set_state(999, 20)
        if force:
            D.force_step_abort(0)
        s.step_checked(advance=True, logits=True)
        D.force_step_abort(-1)
        out = (s.get_state(), s.read_logits().view(np.uint16).copy(), s.check_status())
        s.free()
        return out

    want = in_mode(D, 0, lambda: run(False))
    plain = run(False)
    assert plain[0] == want[0] and np.array_equal(plain[1], want[1]) and plain[2] == 0
    n0 = D.step_fallback_count()
    print("checked step, forced to give up", flush=True)
    got = run(True)
    assert got[0] == want[0] and got[0][1] == 21
    assert np.array_equal(got[1], want[1])
    assert got[2] & 4 and not got[2] & 2
    assert D.step_fallback_count() == n0 + 1


def test_two_streams_interleaved(gpu, D, dmodel, single):
    """Two sessions on two streams, single-launch steps enqueued alternately
    with no synchronization between them: the library orders them, every
    step completes (status 0) and each session ends with the tokens, position
    and cache of the same steps run alone."""
    Q = gpu

    def alone(token, pos):
        s = D.DecodeSession(dmodel, 64)
        s.set_state(token, pos)
        for _ in range(6):
            s.step(advance=True, logits=False)
        out = session_result(s)
        s.free()
        return out

    want_a, want_b = alone(1234, 10), alone(4321, 30)
    st_a, st_b = Q.Stream(), Q.Stream()
    a = D.DecodeSession(dmodel, 64, st_a)
    b = D.DecodeSession(dmodel, 64, st_b)
    a.set_state(1234, 10)
    b.set_state(4321, 30)
    print("12 single-launch steps on two streams, interleaved", flush=True)
    for _ in range(6):
        a.step(advance=True, logits=False)
        b.step(advance=True, logits=False)
    st_a.synchronize()
    st_b.synchronize()
    assert a.check_status() == 0 and b.check_status() == 0
    got_a, got_b = session_result(a), session_result(b)
    assert got_a[0] == want_a[0] and same_cache(got_a[1], want_a[1])
    assert got_b[0] == want_b[0] and same_cache(got_b[1], want_b[1])
    a.free()
    b.free()
    st_a.destroy()
    st_b.destroy()
