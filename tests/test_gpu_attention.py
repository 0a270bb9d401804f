"""Packed varlen attention on gfx950 against AttentionVarlenRef's restatement.

Bars: fp32 path within 1e-4 * (1 + |ref|) (the reference's own SIMD-vs-Ref
tolerance, tests/cpp/test_attention_varlen.cpp:370-375) and in practice
~1e-6; split-fp16 MFMA path (fp32 inputs, hi+lo fp16 operands, three MFMAs
per product) within rtol = atol = 1e-5 of the fp32 oracle on the same fp32
inputs; single-fp16 MFMA path (bf16 Q/K, fp16 V and P, fp32 softmax) on
bf16-rounded inputs within rtol = atol = 1e-3 of the fp32 kernel on the same
values.
"""
import numpy as np
import pytest

from conftest import cu_from_lengths, rng

pytestmark = pytest.mark.gpu

import esm_gfx950 as eg
from esm_gfx950 import synthetic as syn


def bf16_round(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def bf16_bits(x):
    return (np.ascontiguousarray(bf16_round(x), np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _qkv(r, T, H, dh, scale_q=True):
    q = r.standard_normal((T, H, dh)).astype(np.float32)
    k = r.standard_normal((T, H, dh)).astype(np.float32)
    v = r.standard_normal((T, H, dh)).astype(np.float32)
    if scale_q:
        q *= np.float32(1.0 / np.sqrt(dh))
    return q, k, v


@pytest.mark.parametrize("H,dh,lengths", [
    (2, 3, [5]), (4, 16, [32]), (4, 17, [9]), (4, 24, [16]), (4, 32, [17]), (4, 64, [33]),
    (4, 16, [17, 23]), (4, 64, [11, 31]), (20, 64, [256]), (20, 64, [128, 128]), (20, 24, [37, 100]),
    (20, 64, [1, 1]), (20, 16, [22, 202, 97, 0, 50]), (3, 128, [70, 5]),
])
def test_fp32_path(dev, oracle, H, dh, lengths):
    """Shapes of the reference's AttentionVarlenAvx512 sweep plus an empty sequence."""
    r = rng(sum(lengths) + H * dh)
    cu = cu_from_lengths(lengths)
    T = int(cu[-1])
    q, k, v = _qkv(r, T, H, dh, scale_q=False)
    out = dev.empty((T, H * dh), np.float32)
    dev.attention_varlen(dev.array(q), dev.array(k), dev.array(v), cu, H, dh, out, eg.ATTN_FP32)
    want = oracle.attention_varlen(q, k, v, cu, H, dh)
    got = out.numpy()
    assert np.all(np.abs(got - want) <= 1e-4 * (1 + np.abs(want)))
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def _mfma_vs_oracle(dev, oracle, lengths, H, seed, scale_q=True, check_seqs=None):
    r = rng(seed)
    cu = cu_from_lengths(lengths)
    T = int(cu[-1])
    q, k, v = _qkv(r, T, H, 64, scale_q=scale_q)
    qb, kb, vb = bf16_round(q), bf16_round(k), bf16_round(v)
    out = dev.empty((T, H * 64), np.float32)
    dev.attention_varlen_bf16(dev.array(bf16_bits(q)), dev.array(bf16_bits(k)), dev.array(bf16_bits(v)), cu, H, out)
    got = out.numpy()
    seqs = range(len(lengths)) if check_seqs is None else check_seqs
    for b in seqs:
        s0, s1 = int(cu[b]), int(cu[b + 1])
        if s1 == s0:
            continue
        sub = np.array([0, s1 - s0], np.int32)
        want = oracle.attention_varlen(qb[s0:s1], kb[s0:s1], vb[s0:s1], sub, H, 64)
        np.testing.assert_allclose(got[s0:s1], want, rtol=1e-3, atol=1e-3, err_msg=f"seq {b} L={s1 - s0}")
    return got, cu


@pytest.mark.parametrize("lengths", [[1], [7, 1, 16], [33, 129, 64], [250, 60, 128, 127], [1024], [300, 0, 5]])
def test_mfma_ragged(dev, oracle, lengths):
    _mfma_vs_oracle(dev, oracle, lengths, H=20, seed=sum(lengths))


def test_mfma_config2_full(dev, oracle):
    """Config 2: 256 sequences, L ~ clip(round(N(120,30)), 60, 250), H=20, dh=64.
    The whole batch runs on the GPU; 24 sequences are checked against the oracle."""
    lengths = syn.varlen_lengths(256, 20261201 + 2)
    r = rng(0)
    _mfma_vs_oracle(dev, oracle, list(lengths), H=20, seed=2,
                    check_seqs=sorted(r.choice(256, 24, replace=False).tolist() + [int(np.argmax(lengths))]))


def test_mfma_unscaled_q_stress(dev, oracle):
    """Q not pre-scaled (8x larger logits): peaked softmax rows."""
    _mfma_vs_oracle(dev, oracle, [200, 90, 64], H=8, seed=11, scale_q=False)


def _x3_vs_oracle(dev, oracle, lengths, H, seed, scale_q=True, check_seqs=None, tol=1e-5):
    r = rng(seed)
    cu = cu_from_lengths(lengths)
    T = int(cu[-1])
    q, k, v = _qkv(r, T, H, 64, scale_q=scale_q)
    out = dev.empty((T, H * 64), np.float32)
    dev.attention_varlen(dev.array(q), dev.array(k), dev.array(v), cu, H, 64, out, eg.ATTN_F16X3_MFMA)
    got = out.numpy()
    assert np.all(np.isfinite(got))
    seqs = range(len(lengths)) if check_seqs is None else check_seqs
    for b in seqs:
        s0, s1 = int(cu[b]), int(cu[b + 1])
        if s1 == s0:
            continue
        sub = np.array([0, s1 - s0], np.int32)
        want = oracle.attention_varlen(q[s0:s1], k[s0:s1], v[s0:s1], sub, H, 64)
        np.testing.assert_allclose(got[s0:s1], want, rtol=tol, atol=tol, err_msg=f"seq {b} L={s1 - s0}")


@pytest.mark.parametrize("lengths", [[1], [7, 1, 16], [33, 129, 64], [250, 60, 128, 127], [1024], [300, 0, 5]])
def test_x3_ragged(dev, oracle, lengths):
    _x3_vs_oracle(dev, oracle, lengths, H=20, seed=100 + sum(lengths))


def test_x3_config2_full(dev, oracle):
    """Config 2 on fp32 inputs: the whole batch on the GPU, 24 sequences plus
    the longest checked against the fp32 oracle at 1e-5."""
    lengths = syn.varlen_lengths(256, 20261201 + 2)
    r = rng(1)
    _x3_vs_oracle(dev, oracle, list(lengths), H=20, seed=3,
                  check_seqs=sorted(r.choice(256, 24, replace=False).tolist() + [int(np.argmax(lengths))]))


def test_x3_unscaled_q_stress(dev, oracle):
    """Q not pre-scaled (8x larger logits, peaked rows): the fp32 oracle's own
    rounding grows with |q.k|, so the bar here is the reference's SIMD-vs-Ref
    tolerance, 1e-4 * (1 + |ref|) (tests/cpp/test_attention_varlen.cpp:370-375)."""
    _x3_vs_oracle(dev, oracle, [200, 90, 64], H=8, seed=12, scale_q=False, tol=1e-4)


def test_x3_long_sequence_variant_is_bit_identical(dev):
    """Batches whose longest sequence passes 256 tokens run the split-fp16
    kernel's long-sequence variant (another V^T swizzle, rescales skipped
    when no running maximum moved): the same bits as the other variant, so
    sequences give identical rows packed beside a long one or on their own."""
    H = 20
    r = rng(77)
    short = [200, 77, 129, 1]
    lengths = short + [300]
    cu = cu_from_lengths(lengths)
    T = int(cu[-1])
    q, k, v = _qkv(r, T, H, 64)
    packed = dev.empty((T, H * 64), np.float32)
    dev.attention_varlen(dev.array(q), dev.array(k), dev.array(v), cu, H, 64, packed, eg.ATTN_F16X3_MFMA)
    Ts = int(cu[len(short)])
    alone = dev.empty((Ts, H * 64), np.float32)
    dev.attention_varlen(dev.array(q[:Ts]), dev.array(k[:Ts]), dev.array(v[:Ts]), cu_from_lengths(short), H, 64,
                         alone, eg.ATTN_F16X3_MFMA)
    assert np.array_equal(packed.numpy()[:Ts].view(np.uint32), alone.numpy().view(np.uint32))


def test_fp32_mfma_input_equivalence(dev, oracle):
    """The fp32-input MFMA entry (device bf16/fp16 cast) matches the bf16 entry."""
    r = rng(12)
    lengths = [130, 77]
    cu = cu_from_lengths(lengths)
    T = int(cu[-1])
    q, k, v = _qkv(r, T, 20, 64)
    out = dev.empty((T, 1280), np.float32)
    dev.attention_varlen(dev.array(q), dev.array(k), dev.array(v), cu, 20, 64, out, eg.ATTN_BF16_MFMA)
    want = oracle.attention_varlen(q, k, v, cu, 20, 64)
    np.testing.assert_allclose(out.numpy(), want, rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("precision", [eg.ATTN_FP32, eg.ATTN_BF16_MFMA, eg.ATTN_F16X3_MFMA])
def test_isolation(dev, precision):
    """A poisoned second sequence leaves the first bit-identical
    (reference tests/cpp/test_attention_varlen.cpp:185-225)."""
    H, dh, L1, L2 = 2 if precision == eg.ATTN_FP32 else 20, 4 if precision == eg.ATTN_FP32 else 64, 5, 3
    r = rng(13)
    q, k, v = _qkv(r, L1, H, dh)
    solo = dev.empty((L1, H * dh), np.float32)
    dev.attention_varlen(dev.array(q), dev.array(k), dev.array(v), np.array([0, L1], np.int32), H, dh, solo, precision)
    T = L1 + L2
    qp = np.concatenate([q, np.full((L2, H, dh), 50.0, np.float32)])
    kp = np.concatenate([k, np.full((L2, H, dh), 1000.0, np.float32)])
    vp = np.concatenate([v, np.full((L2, H, dh), 999.0, np.float32)])
    packed = dev.empty((T, H * dh), np.float32)
    dev.attention_varlen(dev.array(qp), dev.array(kp), dev.array(vp), np.array([0, L1, T], np.int32), H, dh, packed,
                         precision)
    assert np.array_equal(packed.numpy()[:L1], solo.numpy())


@pytest.mark.parametrize("precision", [eg.ATTN_FP32, eg.ATTN_BF16_MFMA, eg.ATTN_F16X3_MFMA])
def test_single_token_is_v(dev, precision):
    """L = 1: softmax is 1, out = V (reference tests/cpp/test_kernels.cpp:355-365)."""
    H, dh = 20, 64
    r = rng(14)
    q, k, v = _qkv(r, 3, H, dh)
    v16 = v.astype(np.float16).astype(np.float32)  # exact in fp16 for the MFMA path
    out = dev.empty((3, H * dh), np.float32)
    dev.attention_varlen(dev.array(q), dev.array(k), dev.array(v16), np.array([0, 1, 2, 3], np.int32), H, dh, out,
                         precision)
    np.testing.assert_array_equal(out.numpy(), v16.reshape(3, H * dh))


def test_cu_seqlens_validation(dev):
    H, dh = 2, 4
    x = dev.empty((4, H * dh), np.float32)
    with pytest.raises(eg.Gfx950Error, match="cu_seqlens\\[0\\] must be 0"):
        dev.attention_varlen(x, x, x, np.array([1, 4], np.int32), H, dh, x)
    with pytest.raises(eg.Gfx950Error, match="non-decreasing"):
        dev.attention_varlen(x, x, x, np.array([0, 3, 2], np.int32), H, dh, x)
