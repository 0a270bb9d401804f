"""The GPU forward composition against HuggingFace ESM-2, and the hidden
states of esm_gfx950_forward_hidden_states.

tests/golden/hf_esm2_8m.npz is transformers' EsmForMaskedLM on the config-1
synthetic weights (tests/golden/make_hf_fixture.py), an implementation of
embed -> N x TransformerBlock -> final LN -> lm head independent of the
reference and of this repository. The reference's acceptance bars for it
(tests/python/test_against_hf.py:86-90) are every hidden state
allclose(rtol=1e-3, atol=8e-2) and logits max-abs < 1.5e-2. The config-1
fp32 forward on the device is also held at 2e-5: the oracle sits within
4.2e-6 of HuggingFace and the device within 1e-5 of the oracle.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import esm_gfx950 as eg
from esm_gfx950 import synthetic as syn

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hf_esm2_8m.npz")
REF_HIDDEN_RTOL, REF_HIDDEN_ATOL, REF_LOGITS_MAX = 1e-3, 8e-2, 1.5e-2
TIGHT = 2e-5


@pytest.fixture(scope="module")
def fx():
    return dict(np.load(FIXTURE, allow_pickle=False))


@pytest.fixture(scope="module")
def w8m():
    return syn.make_weights(syn.ESM2_8M, seed=20261201 + 1, int8=False)


def _batch(fx, key):
    cu = fx[key + "_cu"]
    return syn.PackedBatch(fx[key + "_ids"], cu, np.diff(cu).astype(np.int32))


def corr(a, b):
    return float(np.corrcoef(a.ravel().astype(np.float64), b.ravel().astype(np.float64))[0, 1])


def test_gpu_logits_match_hf(dev, fx, w8m):
    """The 16 config-1 sequences in one packed forward against HuggingFace
    run one sequence at a time."""
    b = _batch(fx, "seq")
    m = eg.Model(dev, w8m, int8=False)
    try:
        got = m.forward_packed(b.ids, b.cu)
    finally:
        m.free()
    d = float(np.max(np.abs(got - fx["seq_logits"])))
    print(f"config-1 logits vs HF: max |diff| = {d:.3e}")
    assert d < REF_LOGITS_MAX
    assert d < TIGHT, d


def test_gpu_hidden_states_match_hf(dev, fx, w8m):
    """Every hidden state of the masked batch (token dropout in play)."""
    b = _batch(fx, "mask")
    m = eg.Model(dev, w8m, int8=False)
    try:
        logits, hs = m.forward_hidden_states(b.ids, b.cu)
    finally:
        m.free()
    want = fx["mask_hidden"]
    assert hs.shape == want.shape
    worst = 0.0
    for i in range(want.shape[0]):
        np.testing.assert_allclose(hs[i], want[i], rtol=REF_HIDDEN_RTOL, atol=REF_HIDDEN_ATOL)
        np.testing.assert_allclose(hs[i], want[i], rtol=TIGHT, atol=TIGHT, err_msg=f"hidden_state_{i}")
        worst = max(worst, float(np.max(np.abs(hs[i] - want[i]))))
    d = float(np.max(np.abs(logits - fx["mask_logits"])))
    print(f"mask batch vs HF: hidden max |diff| = {worst:.3e}, logits {d:.3e}")
    assert d < TIGHT


def test_hidden_states_match_oracle_fp32(dev, oracle, w8m):
    """forward_hidden_states on config 1 against the oracle's hidden states
    (1e-5), split over two concurrent sequence groups as well as one."""
    b = syn.config1_batch()
    want_l, want_h = oracle.forward_packed(w8m, b, int8=False, per_token=False, hidden=True)
    m = eg.Model(dev, w8m, int8=False)
    try:
        for parts in (1, 2):
            m.set_parts(parts)
            logits, hs = m.forward_hidden_states(b.ids, b.cu)
            np.testing.assert_allclose(hs, want_h, rtol=1e-5, atol=1e-5)
            np.testing.assert_allclose(logits, want_l, rtol=1e-5, atol=1e-5)
    finally:
        m.free()


@pytest.mark.parametrize("numerics", ["per_token", "per_tensor", "x86"])
def test_hidden_states_leave_logits_unchanged(dev, numerics):
    """Capturing hidden states keeps every layer's residual whole (no split-K
    partial sums across layers, the x86 path's pending residual added): the
    logits stay bit-identical to forward_packed's."""
    cfg = syn.ESM2_650M.with_layers(2)
    w = syn.make_weights(cfg, seed=20261201 + 4, int8=True, keep_f32_linears=False)
    b = syn.batch_from_lengths([40, 129, 7, 61], seed=3)
    mode = eg.ACT_PER_TOKEN if numerics == "per_token" else eg.ACT_PER_TENSOR
    m = eg.Model(dev, w, int8=True, act_mode=mode)
    try:
        if numerics == "x86":
            m.set_numerics(eg.NUMERICS_X86_AVX512)
        ref = m.forward_packed(b.ids, b.cu)
        logits, hs = m.forward_hidden_states(b.ids, b.cu)
    finally:
        m.free()
    assert np.array_equal(logits, ref)
    assert hs.shape == (cfg.num_layers + 1, b.total_tokens, cfg.hidden_size)
    assert np.all(np.isfinite(hs))


def test_w8a8_hidden_states_vs_oracle(dev, oracle):
    """Per-token W8A8 hidden states against the oracle's same-mode forward with
    the 24-bit FFN intermediate: correlation >= 0.9999 at every state."""
    cfg = syn.ESM2_650M.with_layers(2)
    w = syn.make_weights(cfg, seed=20261201 + 4, int8=True, keep_f32_linears=False)
    b = syn.batch_from_lengths([130, 61, 250, 2, 97, 200], seed=7)
    m = eg.Model(dev, w, int8=True, act_mode=eg.ACT_PER_TOKEN)
    try:
        _, hs = m.forward_hidden_states(b.ids, b.cu)
    finally:
        m.free()
    _, want = oracle.forward_packed(w, b, int8=True, per_token=True, ffn_bits=24, hidden=True)
    for i in range(want.shape[0]):
        assert corr(hs[i], want[i]) >= 0.9999, i


def test_gpu_pad_masks(dev, oracle, fx, w8m):
    """BatchView's packed_masks on the device (esm_gfx950_forward_packed_masked,
    forward_hidden_states with masks): the post-embed state against HF's
    padded batch (1e-6), the logits against the oracle's masked forward
    (config-1 bar 1e-5), and all-ones masks bit-identical to no masks."""
    cu = fx["pad_cu"]
    b = syn.PackedBatch(fx["pad_ids"], cu, np.diff(cu).astype(np.int32))
    masks = fx["pad_masks"]
    want_l = oracle.forward_packed(w8m, b, int8=False, per_token=False, masks=masks)
    m = eg.Model(dev, w8m, int8=False)
    try:
        logits, hs = m.forward_hidden_states(b.ids, b.cu, masks=masks)
        got = m.forward_packed_masked(b.ids, masks, b.cu)
        plain = m.forward_packed(b.ids, b.cu)
        ones = m.forward_packed_masked(b.ids, np.ones_like(masks), b.cu)
    finally:
        m.free()
    assert np.all(hs[0][masks == 0] == 0)
    np.testing.assert_allclose(hs[0], fx["pad_hidden0"], rtol=1e-6, atol=1e-6)
    assert np.array_equal(logits, got)
    np.testing.assert_allclose(got, want_l, rtol=1e-5, atol=1e-5)
    assert np.array_equal(ones, plain)
    assert not np.array_equal(got, plain)


def test_gpu_pad_masks_w8a8(dev, oracle):
    """Pads in the per-token W8A8 forward against the oracle's same-mode
    masked forward (correlation >= 0.9999), over two sequence groups."""
    cfg = syn.ESM2_650M.with_layers(2)
    w = syn.make_weights(cfg, seed=20261201 + 4, int8=True, keep_f32_linears=False)
    b = syn.batch_from_lengths([130, 61, 250, 97], seed=9)
    masks = np.ones_like(b.ids)
    masks[b.cu[1] - 20:b.cu[1]] = 0
    masks[b.cu[2] + 5:b.cu[2] + 9] = 0
    m = eg.Model(dev, w, int8=True, act_mode=eg.ACT_PER_TOKEN)
    try:
        m.set_parts(2)
        got = m.forward_packed_masked(b.ids, masks, b.cu)
    finally:
        m.free()
    want = oracle.forward_packed(w, b, int8=True, per_token=True, ffn_bits=24, masks=masks)
    assert corr(got, want) >= 0.9999
