"""FP32 facade ops on gfx950 against the oracle: LayerNorm, GELU, residual,
Q-scale, RoPE (tables + varlen apply) and FP32 Linear.

Bars follow the reference's own SIMD-vs-Ref tests: LN / GELU 1e-5
(tests/cpp/test_kernels.cpp:148-180,203-221), RoPE 1e-6 (:340-353), FP32
GEMM 1e-4 * (1 + |ref|) (tests/cpp/test_gemm_shapes.cpp:75); residual and
scale are exact.
"""
import numpy as np
import pytest

from conftest import cu_from_lengths, rng

pytestmark = pytest.mark.gpu

import esm_gfx950 as eg


@pytest.mark.parametrize("d", [4, 17, 47, 320, 480, 640, 1280, 2560, 5120])
def test_layernorm(dev, oracle, d):
    rows = 37
    r = rng(d)
    x = (0.5 * np.sin(np.arange(rows * d) * 0.013) + 0.2 * np.cos(np.arange(rows * d) * 0.007)).astype(np.float32)
    x = (x.reshape(rows, d) + r.standard_normal((rows, d)).astype(np.float32)).astype(np.float32)
    g = (1 + 0.1 * np.sin(np.arange(d) * 0.31)).astype(np.float32)
    b = (0.05 * np.cos(np.arange(d) * 0.17)).astype(np.float32)
    out = dev.empty((rows, d), np.float32)
    dev.layernorm(dev.array(x), dev.array(g), dev.array(b), 1e-5, out, rows, d)
    np.testing.assert_allclose(out.numpy(), oracle.layernorm(x, g, b, 1e-5), rtol=0, atol=1e-5)


def test_gelu(dev, oracle):
    n = 8195
    x = (-5 + 10 * np.arange(n) / (n - 1)).astype(np.float32)
    x = np.concatenate([x, np.array([0, 10, -10, 1, -1, 2], np.float32)])
    out = dev.empty(x.shape, np.float32)
    dev.gelu(dev.array(x), out, x.size)
    got = out.numpy()
    np.testing.assert_allclose(got, oracle.gelu(x), rtol=0, atol=1e-5)
    # known values (reference tests/cpp/test_kernels.cpp:189-201)
    np.testing.assert_allclose(got[-3:], [0.8413447, -0.1586553, 1.9544997], atol=1e-5)


def test_residual_and_scale(dev):
    r = rng(3)
    for n in (1, 15, 16, 17, 1000, 39_000):
        y = r.standard_normal(n).astype(np.float32)
        x = r.standard_normal(n).astype(np.float32)
        dy = dev.array(y)
        dev.residual_add(dy, dev.array(x), n)
        assert np.array_equal(dy.numpy(), y + x)
        dev.scale(dy, n, 0.125)
        assert np.array_equal(dy.numpy(), (y + x) * np.float32(0.125))


@pytest.mark.parametrize("H,dh,lengths", [
    (5, 16, [100]), (5, 16, [100] * 8), (20, 24, [128] * 4), (20, 32, [256, 37]), (20, 64, [256] * 8),
    (20, 64, [1, 1, 1]),
])
def test_rope_varlen(dev, oracle, H, dh, lengths):
    cu = cu_from_lengths(lengths)
    T = int(cu[-1])
    L = max(lengths)
    c, s = eg.rope_build_tables(L, dh)
    oc, os_ = oracle.rope_tables(L, dh)
    assert np.array_equal(c, oc) and np.array_equal(s, os_)
    x = (0.3 * np.sin(np.arange(T * H * dh) * 0.019)).astype(np.float32).reshape(T, H, dh)
    dx = dev.array(x)
    dev.rope_apply_varlen(dx, dev.array(c), dev.array(s), cu, H, dh)
    np.testing.assert_allclose(dx.numpy(), oracle.rope_varlen(x, c, s, cu, H, dh), rtol=0, atol=1e-6)


def test_rope_restarts_per_sequence(dev):
    """Positions restart at every cu_seqlens boundary
    (reference tests/cpp/test_attention_varlen.cpp:138-183)."""
    H, dh = 1, 4
    r = rng(31)
    src = r.uniform(-1, 1, size=(5, H, dh)).astype(np.float32)
    c, s = eg.rope_build_tables(3, dh)
    dc, ds = dev.array(c), dev.array(s)
    packed = dev.array(src)
    dev.rope_apply_varlen(packed, dc, ds, np.array([0, 3, 5], np.int32), H, dh)
    a = dev.array(src[:3])
    dev.rope_apply_varlen(a, dc, ds, np.array([0, 3], np.int32), H, dh)
    b = dev.array(src[3:])
    dev.rope_apply_varlen(b, dc, ds, np.array([0, 2], np.int32), H, dh)
    got = packed.numpy()
    assert np.array_equal(got[:3], a.numpy()) and np.array_equal(got[3:], b.numpy())


@pytest.mark.parametrize("M,N,K", [(2, 4, 3), (1, 2, 2), (33, 65, 17), (1792, 960, 320), (300, 1280, 1280),
                                   (200, 33, 1280), (64, 320, 1280)])
def test_linear_f32(dev, oracle, M, N, K):
    r = rng(M * 7 + N + K)
    A = r.uniform(-1, 1, size=(M, K)).astype(np.float32)
    W = r.uniform(-1, 1, size=(N, K)).astype(np.float32)
    b = r.uniform(-1, 1, size=N).astype(np.float32)
    out = dev.empty((M, N), np.float32)
    dev.linear_f32(dev.array(A), dev.array(W), dev.array(b), out, M, N, K)
    want = oracle.linear_f32(A, W, b)
    got = out.numpy()
    assert np.all(np.abs(got - want) <= 1e-4 * (1 + np.abs(want)))


def test_linear_f32_known_answer(dev):
    """Reference tests/cpp/test_kernels.cpp:88-111."""
    A = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    W = np.array([[1, 0, -1], [0, 1, 0], [1, 1, 1], [2, -1, 0]], np.float32)
    b = np.array([10, 20, 30, 40], np.float32)
    out = dev.empty((2, 4), np.float32)
    dev.linear_f32(dev.array(A), dev.array(W), dev.array(b), out, 2, 4, 3)
    assert np.array_equal(out.numpy(), np.array([[8, 22, 36, 40], [8, 25, 45, 43]], np.float32))
