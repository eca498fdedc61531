"""The measurement tools behind the single-launch decode step's design
(q8rt_launch_cost, q8rt_handoff_latency): they run to completion on the
device and return physically sensible figures.  (The figures themselves are
recorded by bench.py; the tests only bound them loosely.)"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_launch_cost_of_the_step_grid(gpu):
    Q = gpu
    ordinary = Q.launch_cost(448, 256, 79360, launches=200)
    coop = Q.launch_cost(448, 256, 79360, launches=200, cooperative=True)
    print(f"empty 448 x 256 launch: ordinary {ordinary:.2f} us, cooperative {coop:.2f} us",
          flush=True)
    assert 0.1 < ordinary < 200.0
    assert 0.1 < coop < 500.0


@pytest.mark.parametrize("producers,consumers,n_words,replicas",
                         [(1, 1, 512, 1), (128, 192, 512, 4), (4, 8, 64, 2)])
def test_handoff_latency(gpu, producers, consumers, n_words, replicas):
    Q = gpu
    lat, failed = Q.handoff_latency(producers, consumers, n_words, replicas, rounds=20)
    print(f"hand-off {producers} -> {consumers}, {n_words} words x {replicas}: median "
          f"{np.median(lat):.3f} us, max {lat.max():.3f} us, failed {failed}", flush=True)
    assert lat.shape == (20, consumers)
    assert failed == 0 and np.isfinite(lat).all()
    # a consumer cannot hold the vector before the last producer stored it
    # (up to the clock's 10 ns tick), and no hand-off takes anywhere near the
    # 20 us between rounds
    assert lat.min() >= -0.05 and np.median(lat) < 15.0
