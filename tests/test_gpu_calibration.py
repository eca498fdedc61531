"""The measurement tools behind the single-launch decode step's design
(q8rt_launch_cost, q8rt_handoff_latency, q8rt_memory_latency): they run to completion on the
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


def test_memory_latency_by_level(gpu):
    Q = gpu
    r = Q.memory_latency(2048)
    print(f"dependent load: HBM {r['hbm_ns']:.0f} ns, MALL {r['mall_ns']:.0f} ns, "
          f"L2 {r['l2_ns']:.0f} ns (XCDs {r['xcds']})", flush=True)
    assert 0 <= r["xcds"][0] < 8 and r["xcds"][1] == (r["xcds"][0] + 1) % 8
    for k in ("hbm_ns", "mall_ns", "l2_ns"):
        assert np.isfinite(r[k]) and 20.0 < r[k] < 20000.0, (k, r[k])
    # a line from this XCD's L2 comes back sooner than one from the memory side
    assert r["l2_ns"] < r["mall_ns"] and r["l2_ns"] < r["hbm_ns"]
