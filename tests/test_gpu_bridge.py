"""The reference-side bridge's facade arms on the GPU against the
reference's own compiled kernels (oracle/_ref/libesmref.so): what a
`case Isa::Gfx950:` arm in src/kernels/dispatch.cpp returns for the same
arguments as the reference's CPU arm.

Bars: LinearInt8 bit-exact against LinearVnni (same dynamic per-tensor
activation scale, same dequant expression, src/kernels/gemm_int8.cpp:
510-555); FP32 ops within rtol = atol = 1e-5 of the *Ref kernels; the
elementwise ops exact; AttentionVarlen within 1e-5 (split-fp16 MFMA at
head_dim 64, scalar fp32 otherwise) of AttentionVarlenRef."""
import os

import numpy as np
import pytest

from bridge_lib import BRIDGE_LIB, Bridge
from conftest import cu_from_lengths, rng

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not os.path.exists(BRIDGE_LIB),
                                 reason="bridge not built (needs the reference headers at build time)")]


@pytest.fixture(scope="module")
def bridge():
    return Bridge()


@pytest.mark.parametrize("M,N,K", [(64, 1280, 1280), (130, 5120, 1280), (37, 1280, 5120), (5, 48, 32)])
def test_linear_int8_equals_linear_vnni(bridge, ref, oracle, M, N, K):
    if ref.host_isa() not in ("avx512vnni", "amx"):
        pytest.skip(f"host ISA {ref.host_isa()} has no VNNI")
    r = rng(900 + M + N + K)
    A = r.normal(0, 1, size=(M, K)).astype(np.float32)
    Wf = r.normal(0, 0.02, size=(N, K)).astype(np.float32)
    q, s = ref.quantize(Wf)  # the reference's own Quantize (pack.cpp:149-177)
    bias = r.normal(0, 0.02, size=N).astype(np.float32)
    got = bridge.linear_int8(A, q, s, bias)
    assert np.array_equal(got, ref.linear_vnni(A, q, s, bias))
    aq, sc = oracle.quant_act_tensor(A)
    want = oracle.dequant(oracle.gemm_i8_i32(aq, q), np.full(M, sc, np.float32), s, bias)
    assert np.array_equal(got, want)


def test_linear_f32(bridge, ref):
    r = rng(31)
    A = r.normal(0, 1, size=(70, 320)).astype(np.float32)
    W = r.normal(0, 0.05, size=(96, 320)).astype(np.float32)
    b = r.normal(0, 0.05, size=96).astype(np.float32)
    np.testing.assert_allclose(bridge.linear(A, W, b), ref.linear_ref(A, W, b), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(bridge.linear(A, W, None), ref.linear_ref(A, W, None), rtol=1e-5, atol=1e-5)


def test_layernorm_gelu_residual_scale(bridge, ref):
    r = rng(32)
    x = r.normal(0.3, 2, size=(33, 1280)).astype(np.float32)
    g = (1 + r.normal(0, 0.02, 1280)).astype(np.float32)
    b = r.normal(0, 0.02, 1280).astype(np.float32)
    np.testing.assert_allclose(bridge.layernorm(x, g, b), ref.layernorm_ref(x, g, b), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(bridge.gelu(x), ref.gelu_ref(x), rtol=1e-5, atol=1e-5)
    y = r.normal(size=x.shape).astype(np.float32)
    assert np.array_equal(bridge.residual_add(y, x), y + x)
    assert np.array_equal(bridge.scale(x, 0.125), x * np.float32(0.125))


@pytest.mark.parametrize("H,dh", [(20, 64), (4, 16)])
def test_rope_and_attention_varlen(bridge, ref, H, dh):
    r = rng(33 + dh)
    lengths = [130, 1, 61, 250]
    cu = cu_from_lengths(lengths)
    T = int(cu[-1])
    cos, sin = ref.rope_tables(max(lengths), dh)
    x = r.normal(size=(T, H, dh)).astype(np.float32)
    np.testing.assert_allclose(bridge.rope_varlen(x, cos, sin, cu, H, dh), ref.rope_varlen_ref(x, cos, sin, cu, H, dh),
                               rtol=1e-6, atol=1e-6)
    q = (r.normal(size=(T, H, dh)) / np.sqrt(dh)).astype(np.float32)
    k = r.normal(size=(T, H, dh)).astype(np.float32)
    v = r.normal(size=(T, H, dh)).astype(np.float32)
    got = bridge.attention_varlen(q, k, v, cu, H, dh)
    np.testing.assert_allclose(got, ref.attention_varlen_ref(q, k, v, cu, H, dh), rtol=1e-5, atol=1e-5)
