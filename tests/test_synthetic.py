"""Synthetic model and batch generator (CPU): weight quantisation matches the
reference's Quantize bit for bit; SmoothQuant folding preserves the fp32
function; batches follow the benchmark configs."""
import numpy as np
import pytest

from conftest import rng

from esm_gfx950 import synthetic as syn


def test_quantize_weight_matches_oracle_and_reference(oracle, ref):
    r = rng(0)
    W = (r.standard_normal((97, 320)) * r.uniform(0.001, 3, size=(97, 1))).astype(np.float32)
    W[5] = 0.0
    W[6, :] = 0.0
    W[6, 3] = -2.0
    q, s = syn.quantize_weight(W)
    oq, os_ = oracle.quantize_weight(W)
    rq, rs = ref.quantize(W)
    assert np.array_equal(q, oq) and np.array_equal(s, os_)
    assert np.array_equal(q, rq) and np.array_equal(s, rs)


def test_smoothquant_folding_preserves_function():
    """Each site computes the same fp32 function after folding (reference
    tests/cpp/test_smoothquant.cpp:76-125 identity, at 1e-4)."""
    cfg = syn.EsmConfig("tiny", 1, 64, 4, 128)
    plain = syn.make_weights(cfg, seed=3, int8=False)
    folded = syn.make_weights(cfg, seed=3, int8=True, keep_f32_linears=True)
    r = rng(1)
    x = r.standard_normal((9, 64)).astype(np.float32)
    xn = (x - x.mean(1, keepdims=True)) / np.sqrt(x.var(1, keepdims=True) + 1e-5)

    def ln(w, name):
        return xn * w.f32[f"layers.0.{name}.weight"] + w.f32[f"layers.0.{name}.bias"]

    def lin(w, name, a, bias=True):
        y = a @ w.f32[f"layers.0.{name}.weight"].T
        return y + w.f32[f"layers.0.{name}.bias"] if bias else y

    # site 1: attn_ln -> q, k (v's outputs are rescaled again by site 2)
    for n in ("q", "k"):
        np.testing.assert_allclose(lin(plain, n, ln(plain, "attn_ln")), lin(folded, n, ln(folded, "attn_ln")),
                                   rtol=1e-4, atol=1e-5)
    # site 2: v -> out_proj
    np.testing.assert_allclose(lin(plain, "out", lin(plain, "v", ln(plain, "attn_ln"))),
                               lin(folded, "out", lin(folded, "v", ln(folded, "attn_ln"))), rtol=1e-4, atol=1e-5)
    # site 3: ffn_ln -> fc1
    np.testing.assert_allclose(lin(plain, "fc1", ln(plain, "ffn_ln")), lin(folded, "fc1", ln(folded, "ffn_ln")),
                               rtol=1e-4, atol=1e-5)
    # the factors were not all 1, and fc2 is never migrated
    assert not np.allclose(plain.f32["layers.0.q.weight"], folded.f32["layers.0.q.weight"])
    assert np.array_equal(plain.f32["layers.0.fc2.weight"], folded.f32["layers.0.fc2.weight"])


def test_batches():
    b = syn.config4_varlen_batch()
    assert len(b.cu) == 257 and b.cu[0] == 0 and b.cu[-1] == b.ids.size
    assert b.lengths.min() >= 60 and b.lengths.max() <= 250
    assert abs(b.total_tokens - 30809) < 1500
    for i in range(256):
        s = b.ids[b.cu[i]:b.cu[i + 1]]
        assert s[0] == syn.CLS and s[-1] == syn.EOS
        assert s[1:-1].min() >= 4 and s[1:-1].max() <= 23
    u = syn.config4_uniform_batch()
    assert u.total_tokens == 2048 and u.residues == 2032
    c1 = syn.config1_batch()
    assert len(c1.cu) == 17 and c1.lengths.min() >= 22 and c1.lengths.max() <= 202
    c5 = syn.config5_batch()
    assert len(c5.cu) == 65 and c5.lengths.min() >= 50 and c5.lengths.max() <= 1024
    # determinism
    assert np.array_equal(syn.config4_varlen_batch().ids, b.ids)


def test_weights_deterministic():
    cfg = syn.EsmConfig("tiny", 1, 32, 2, 64)
    a = syn.make_weights(cfg, seed=1, int8=True)
    b = syn.make_weights(cfg, seed=1, int8=True)
    for k in a.f32:
        assert np.array_equal(a.f32[k], b.f32[k])
    for k in a.i8:
        assert np.array_equal(a.i8[k][0], b.i8[k][0])
