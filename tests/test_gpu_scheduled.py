"""Scheduled forward (esm_gfx950_forward_scheduled; reference
Model::ForwardScheduled, src/model.cpp:1298-1421) against the serial forward,
mirroring tests/python/test_forward_scheduled.py:35-100:

* scheduled == serial within 1e-4 (:35-50), single sequence within 1e-5
  (:75-80), empty input (:83-84), max_batch_size changes nothing (:87-100);
* outputs come back in input order when the length-bucket split reorders
  the work (:53-72);
* the W8A8 per-token model: the scheduled groups give the same logits as one
  packed forward of every sequence, also with concurrent sequence groups.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import esm_gfx950 as eg
from esm_gfx950 import synthetic as syn


@pytest.fixture(scope="module")
def m8(dev):
    w = syn.make_weights(syn.ESM2_8M, seed=20261201 + 1, int8=False)
    m = eg.Model(dev, w, int8=False)
    yield m
    m.free()


def seqs(lengths, seed):
    b = syn.batch_from_lengths(lengths, seed=seed)
    return [b.ids[b.cu[i]:b.cu[i + 1]].copy() for i in range(len(lengths))]


def serial(m, ids_list):
    return [m.forward_packed(x, np.array([0, len(x)], np.int32)) for x in ids_list]


def test_scheduled_matches_serial(m8):
    ids = seqs([20, 31, 16, 16], seed=1)
    got = m8.forward_scheduled(ids)
    want = serial(m8, ids)
    assert len(got) == len(want)
    for i, (g, w) in enumerate(zip(got, want)):
        np.testing.assert_allclose(g, w, rtol=1e-4, atol=1e-4, err_msg=f"seq {i}")


def test_scheduled_preserves_input_order(m8):
    lengths = [5, 113, 5, 113, 5, 113, 5, 113]  # max/mean far above 1.2: the split fires
    ids = seqs(lengths, seed=2)
    assert len(eg.plan_batches(lengths)) > 1
    got = m8.forward_scheduled(ids)
    want = serial(m8, ids)
    for i, (g, w, L) in enumerate(zip(got, want, lengths)):
        assert g.shape == (L, 33), f"position {i}"
        np.testing.assert_allclose(g, w, rtol=1e-4, atol=1e-4, err_msg=f"seq {i}")


def test_scheduled_single_sequence(m8):
    ids = seqs([20], seed=3)
    got = m8.forward_scheduled(ids)
    np.testing.assert_allclose(got[0], serial(m8, ids)[0], rtol=1e-5, atol=1e-5)


def test_scheduled_empty_input(m8):
    assert m8.forward_scheduled([]) == []


def test_scheduled_max_batch_size_keeps_numerics(m8):
    ids = seqs([27] * 8, seed=4)
    a = m8.forward_scheduled(ids, max_batch_size=8)
    b = m8.forward_scheduled(ids, max_batch_size=2)
    for i, (x, y) in enumerate(zip(a, b)):
        np.testing.assert_allclose(x, y, rtol=1e-4, atol=1e-4, err_msg=f"chunking changed seq {i}")


def test_scheduled_zero_length_sequences(m8):
    ids = seqs([12, 9], seed=5)
    ids = [ids[0], np.zeros(0, np.int32), ids[1]]
    got = m8.forward_scheduled(ids)
    assert got[1].shape == (0, 33)
    want = serial(m8, [ids[0], ids[2]])
    np.testing.assert_allclose(got[0], want[0], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(got[2], want[1], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("parts", [1, 2])
def test_scheduled_w8a8_matches_packed(dev, parts):
    """Per-token W8A8 rows are independent of their batch, so the scheduled
    groups (several packed forwards, double-buffered) reproduce one packed
    forward of all sequences."""
    w = syn.make_weights(syn.ESM2_650M.with_layers(2), seed=20261201 + 4, int8=True, keep_f32_linears=False)
    m = eg.Model(dev, w, int8=True, act_mode=eg.ACT_PER_TOKEN)
    m.set_parts(parts)
    lengths = [60, 250, 61, 130, 2, 97, 200, 120, 75, 249]
    batch = syn.batch_from_lengths(lengths, seed=6)
    ids = [batch.ids[batch.cu[i]:batch.cu[i + 1]] for i in range(len(lengths))]
    packed = m.forward_packed(batch.ids, batch.cu)
    got = m.forward_scheduled(ids, max_batch_size=4)
    m.free()
    assert len(eg.plan_batches(lengths, max_batch_size=4)) >= 3
    for i, g in enumerate(got):
        np.testing.assert_allclose(g, packed[batch.cu[i]:batch.cu[i + 1]], rtol=1e-4, atol=1e-4,
                                   err_msg=f"seq {i}")
