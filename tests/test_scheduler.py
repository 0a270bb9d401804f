"""PlanBatches (reference src/sched/scheduler.cpp:54-75) through the C ABI's
host-only esm_gfx950_plan_batches.

* The reference's own unit tests (tests/cpp/test_scheduler.cpp:24-80):
  uniform lengths stay one batch, imbalanced lengths split, max_batch_size
  chunks, every index is covered exactly once.
* Exact agreement with the reference's PlanBatches compiled from its source
  (oracle/_ref) on random length lists, ties included (the split sorts with
  std::sort, so equal lengths must land in the same order).
"""
import numpy as np
import pytest

import esm_gfx950 as eg


def test_single_batch_when_lengths_are_uniform():
    plan = eg.plan_batches([100] * 16, max_batch_size=64, imbalance_threshold=1.2)
    assert len(plan) == 1 and len(plan[0]) == 16


def test_splits_when_lengths_are_imbalanced():
    lengths = [50] * 8 + [500] * 8  # max/mean = 1.82 > 1.2
    plan = eg.plan_batches(lengths, max_batch_size=64, imbalance_threshold=1.2)
    assert len(plan) >= 2
    assert sum(len(b) for b in plan) == 16


def test_chunks_on_max_batch_size():
    plan = eg.plan_batches([100] * 10, max_batch_size=4, imbalance_threshold=1.2)
    assert len(plan) >= 3
    assert all(len(b) <= 4 for b in plan)
    assert sum(len(b) for b in plan) == 10


def test_preserves_indices_covering_every_input():
    lengths = [50 + i * 30 for i in range(17)]
    plan = eg.plan_batches(lengths, max_batch_size=8, imbalance_threshold=1.2)
    assert sorted(i for b in plan for i in b) == list(range(17))


def test_empty_and_invalid():
    assert eg.plan_batches([]) == []
    with pytest.raises(eg.Gfx950Error):
        eg.plan_batches([3, -1, 4])


def test_no_chunk_limit_when_max_batch_size_is_not_positive():
    plan = eg.plan_batches([100] * 300, max_batch_size=0)
    assert plan == [list(range(300))]


@pytest.mark.parametrize("seed", range(12))
def test_matches_reference_plan(ref, seed):
    r = np.random.default_rng(seed)
    n = int(r.integers(1, 700))
    if seed % 3 == 0:
        lengths = r.integers(0, 6, n) * 50  # many ties, some zero-length
    else:
        lengths = np.exp(r.uniform(np.log(20), np.log(1100), n)).astype(np.int32)
    max_batch = [0, 1, 3, 64, 256][seed % 5]
    thr = [1.2, 1.05, 2.0, 1.0][seed % 4]
    got = eg.plan_batches(lengths, max_batch_size=max_batch, imbalance_threshold=thr)
    want = ref.plan_batches(lengths, max_batch_size=max_batch, imbalance_threshold=thr)
    assert got == want
