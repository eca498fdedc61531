"""GPU prompt ingestion (qwen3_prefill) and generation loop (qwen3_generate,
run) against the oracle's restatement of @prefill_all / @generate / @run
control flow driven by single GPU decode steps.

The loop runs the same kernels as a single step, so its tokens must equal the
step-by-step ones bit for bit; the control flow (batches of 4, EOS checked on
a batch's last token, the first token not output) comes from the oracle.
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


def step_fn(sess):
    """One eager GPU decode step at an explicit (token, pos)."""
    def step(tok, pos):
        sess.set_state(tok, pos)
        sess.step(advance=False, logits=False)
        return sess.get_state()[0]
    return step


def step_logits_fn(sess):
    def step(tok, pos):
        sess.set_state(tok, pos)
        sess.step(advance=False, logits=True)
        return sess.read_logits()
    return step


def test_generate_matches_steps_without_eos(O, D, dmodel):
    max_seq = 32
    ref = D.DecodeSession(dmodel, max_seq)
    want, n_want = O.generate_control(step_fn(ref), 1234, 3, 10, eos_id=-7)
    ref.free()
    sess = D.DecodeSession(dmodel, max_seq)
    sess.set_state(1234, 3)
    print("generate 10 from pos 3", flush=True)
    got = sess.generate(10, eos_id=-7)
    assert n_want == 10 and got.tolist() == want.tolist()
    assert sess.get_state() == (int(want[-1]), 13)
    sess.free()


@pytest.mark.parametrize("eos_index", [3, 5])
def test_generate_eos_after_batch(O, D, dmodel, eos_index):
    max_seq = 32
    ref = D.DecodeSession(dmodel, max_seq)
    free_run, _ = O.generate_control(step_fn(ref), 77, 0, 12, eos_id=-7)
    ref.free()
    eos = int(free_run[eos_index])
    ref = D.DecodeSession(dmodel, max_seq)
    want, n_want = O.generate_control(step_fn(ref), 77, 0, 12, eos_id=eos)
    ref.free()
    sess = D.DecodeSession(dmodel, max_seq)
    sess.set_state(77, 0)
    print(f"generate with eos {eos} (index {eos_index})", flush=True)
    got = sess.generate(12, eos_id=eos)
    assert got.size == n_want and got.tolist() == want[:n_want].tolist()
    # the batch queued behind the EOS batch was undone: the state is the one
    # the loop stopped with
    assert sess.get_state() == (int(want[n_want - 1]), n_want)
    assert sess.status() == 0
    sess.free()


def test_prefill_matches_steps(O, D, dmodel):
    prompt = [11, 151935, 0, 4242, 99]
    max_seq = 16
    ref = D.DecodeSession(dmodel, max_seq)
    for i, t in enumerate(prompt):
        ref.set_state(t, i)
        ref.step(advance=False, logits=False)
    ref_tok = ref.get_state()[0]
    ref_k, ref_v = ref.cache_rows(13, 0, len(prompt))
    ref.free()
    sess = D.DecodeSession(dmodel, max_seq)
    sess.set_state(-1, 0)
    print("prefill 5 tokens", flush=True)
    sess.prefill(prompt)
    assert sess.get_state() == (ref_tok, len(prompt))
    k, v = sess.cache_rows(13, 0, len(prompt))
    assert np.array_equal(k, ref_k) and np.array_equal(v, ref_v)
    sess.free()


def test_run_matches_control_flow(O, D, dmodel):
    prompt = [3, 1, 4, 1, 5]
    ref = D.DecodeSession(dmodel, len(prompt) + 7)
    want, n_want = O.run_control(step_logits_fn(ref), step_fn(ref), prompt, 7, eos_id=-7)
    ref.free()
    print("run: 5 prompt tokens, 7 new", flush=True)
    got = D.run(dmodel, prompt, 7, eos_id=-7)
    assert got.tolist() == want[:n_want].tolist()


def test_generate_rejects_overflowing_positions(gpu, D, dmodel):
    Q = gpu
    sess = D.DecodeSession(dmodel, 8)
    sess.set_state(5, 6)
    with pytest.raises(Q.Q8GemvError) as e:
        sess.generate(3, eos_id=-1)
    assert e.value.code == Q.Q8_ERR_BAD_SHAPE
    got = sess.generate(2, eos_id=-1)  # exactly fills the cache
    assert got.size == 2 and sess.status() & 1  # the second step asked to advance past slot 7
    sess.free()
