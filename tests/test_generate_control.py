"""The oracle's restatement of @generate / @run control flow
(qwen3_full.mlir:1396-1534, 2113-2167), pinned with step functions whose
outputs are known in closed form."""
from __future__ import annotations

import numpy as np
import pytest


def pos_step(t, p):
    return 100 + p  # the token a step emits names its position


def test_no_eos_runs_max_new_and_skips_first_token(O):
    out, n = O.generate_control(pos_step, first_token=7, start_pos=5, max_new=6, eos_id=-5)
    assert n == 6
    assert out.tolist() == [105, 106, 107, 108, 109, 110]  # 7 itself is never output


@pytest.mark.parametrize("eos_index,count", [(0, 9), (1, 9), (2, 9), (3, 4), (4, 9), (7, 8),
                                             (8, 9)])
def test_eos_is_checked_after_each_batch_of_four(O, eos_index, count):
    # eos = the token of output index eos_index (each token is unique here).
    # Only a batch's last token (indices 3, 7, then 8 of the short batch) is
    # compared with eos, so an eos elsewhere does not stop the loop.
    out, n = O.generate_control(pos_step, 0, 0, 9, 100 + eos_index)
    assert n == count
    assert out[:n].tolist() == [100 + i for i in range(n)]
    assert not out[n:].any()


def test_eos_on_every_token_stops_after_first_batch(O):
    out, n = O.generate_control(lambda t, p: 2, 2, 0, 10, 2)  # first token == eos is not checked
    assert n == 4 and out.tolist() == [2, 2, 2, 2, 0, 0, 0, 0, 0, 0]


def test_short_last_batch_and_zero(O):
    out, n = O.generate_control(lambda t, p: 1 if p == 5 else 0, 0, 0, 6, 1)
    assert n == 6 and out[5] == 1          # batches of 4 then 2; the last one ends on eos
    out, n = O.generate_control(pos_step, 0, 0, 0, 1)
    assert n == 0 and out.size == 0


def test_run_feeds_prompt_positions_and_argmax(O):
    seen = []

    def step_logits(t, p):
        seen.append((t, p))
        lg = np.zeros(151936, np.float16)
        lg[[17, 42]] = 3.0  # tie: the lowest index wins
        return lg

    out, n = O.run_control(step_logits, pos_step, [5, 6, 7], 4, eos_id=-1)
    assert seen == [(5, 0), (6, 1), (7, 2)]
    assert n == 4 and out.tolist() == [103, 104, 105, 106]
