"""Activation observer oracle (oracle/observer.py) pinned on the CPU.

- MT19937 against the C++ standard's known answer;
- the reference's own ActivationObserver (src/quant/observer.cpp compiled
  from source into oracle/_ref) fed the same values: every percentile
  bit-equal, across fills, replacements, several calls and several sites;
- the reference's observer tests (tests/cpp/test_observer.cpp:19-87)
  restated on the oracle, with numpy-drawn uniform inputs in place of the
  test's std::mt19937(0xfade) stream (its bound, 9.99 +- 0.2, holds for any
  uniform [0, 10] sample).
"""
import numpy as np
import pytest

from conftest import rng
from observer import MT19937, RESERVOIR_SIZE, ActivationObserver, uniform_index

PCTS = [0.0, 0.1, 1.0, 10.0, 25.0, 50.0, 75.0, 90.0, 99.0, 99.9, 99.99, 100.0, -5.0, 150.0]


def test_mt19937_known_answer():
    # C++ [rand.predef]: the 10000th invocation of a default-constructed
    # std::mt19937 produces 4123659995.
    g = MT19937()
    for _ in range(9999):
        g()
    assert g() == 4123659995


def test_uniform_index_stays_in_range_and_is_uniform():
    g = MT19937(7)
    draws = np.array([uniform_index(g, 9) for _ in range(20000)])
    assert draws.min() == 0 and draws.max() == 9
    counts = np.bincount(draws, minlength=10)
    assert np.all(np.abs(counts - 2000) < 200)
    assert uniform_index(MT19937(1), 0) == 0


def _same(a, b):
    assert a.keys() == b.keys()
    for k in a:
        assert np.float32(a[k]) == np.float32(b[k]), (k, a[k], b[k])


@pytest.mark.parametrize("sizes", [[1000], [RESERVOIR_SIZE], [RESERVOIR_SIZE + 1], [150000],
                                   [30000, 50000, 70000], [RESERVOIR_SIZE - 3, 7, 90000]])
def test_oracle_matches_reference_observer(ref, sizes):
    r = rng(sum(sizes))
    mine, theirs = ActivationObserver(), ref.observer()
    try:
        for n in sizes:
            v = (r.standard_normal(n) * r.uniform(0.5, 3.0)).astype(np.float32)
            mine.observe("site", v)
            theirs.observe("site", v)
        for p in PCTS:
            _same(mine.percentile(p), theirs.percentile(p))
    finally:
        theirs.free()


def test_oracle_matches_reference_observer_sites_and_clear(ref):
    r = rng(3)
    mine, theirs = ActivationObserver(), ref.observer()
    try:
        for site, n in [("a", 70000), ("b", 100), ("a", 5000), ("c", 0), ("b", 80000)]:
            v = r.standard_normal(n).astype(np.float32)
            mine.observe(site, v)
            theirs.observe(site, v)
        assert theirs.site_count() == 2 and sorted(mine.sites) == ["a", "b"]
        for p in PCTS:
            _same(mine.percentile(p), theirs.percentile(p))
        mine.clear()
        theirs.clear()
        assert mine.percentile(50.0) == {} and theirs.site_count() == 0
    finally:
        theirs.free()


def test_percentile_index_closed_form():
    # Samples 0..n-1: the p-th percentile is floor(p/100 * (n - 1)).
    obs = ActivationObserver()
    n = 1001
    obs.observe("s", np.arange(n, dtype=np.float32)[::-1])
    for p in [0.0, 12.5, 50.0, 99.9, 100.0]:
        assert obs.percentile(p)["s"] == np.floor(np.float32(p / 100) * np.float32(n - 1))


# --- the reference's observer tests (tests/cpp/test_observer.cpp), restated


def test_uniform_input_produces_999_pctile_near_analytic_bound():
    v = rng(0xFADE).uniform(0.0, 10.0, 200000).astype(np.float32)
    obs = ActivationObserver()
    obs.observe("site_a", v)
    stats = obs.percentile(99.9)
    assert abs(stats["site_a"] - 9.99) <= 0.2


def test_negative_values_use_absolute_magnitude():
    v = np.ones(10000, np.float32)
    v[[100, 200, 300]] = [-50.0, -49.0, -48.0]
    obs = ActivationObserver()
    obs.observe("site_neg", v)
    s = obs.percentile(99.9)["site_neg"]
    assert 1.0 <= s <= 50.0


def test_multiple_sites_tracked_independently():
    obs = ActivationObserver()
    obs.observe("small", np.full(1000, 0.5, np.float32))
    obs.observe("large", np.full(1000, 5.0, np.float32))
    s = obs.percentile(99.9)
    assert abs(s["small"] - 0.5) <= 1e-4 and abs(s["large"] - 5.0) <= 1e-4


def test_clear_resets_state():
    obs = ActivationObserver()
    obs.observe("a", np.ones(100, np.float32))
    assert obs.percentile(99.9)
    obs.clear()
    assert not obs.percentile(99.9)


def test_multiple_observe_calls_accumulate():
    obs = ActivationObserver()
    obs.observe("site", np.full(1000, 0.1, np.float32))
    obs.observe("site", np.full(1000, 10.0, np.float32))
    assert abs(obs.percentile(99.9)["site"] - 10.0) <= 1e-4


def test_empty_observe_is_noop():
    obs = ActivationObserver()
    obs.observe("nothing", np.zeros(0, np.float32))
    assert not obs.percentile(99.9)
