"""esm_gfx950_linear_i8_noalloc (the allocation-free LinearInt8) against
esm_gfx950_linear_i8, through the C ABI: identical results, bit for bit, on
two calls in a row, the second smaller (the static scratch keeps the first
call's contents), in both activation modes; oversized calls rejected."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import esm_gfx950 as eg
from conftest import rng


def _case(dev, M, N, K, seed):
    r = rng(seed)
    A = (r.standard_normal((M, K)) * r.uniform(0.2, 3.0, size=(M, 1))).astype(np.float32)
    Wf = (0.02 * r.standard_normal((N, K))).astype(np.float32)
    from esm_gfx950 import synthetic as syn
    q, s = syn.quantize_weight(Wf)
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    return dev.array(A), dev.weight_i8(q, s), dev.array(bias)


@pytest.mark.parametrize("mode", [eg.ACT_PER_TOKEN, eg.ACT_PER_TENSOR])
def test_linear_i8_noalloc_equals_linear_i8(dev, mode):
    for M, N, K, seed in ((3001, 5120, 1280, 1), (77, 100, 330, 2)):
        A, W, bias = _case(dev, M, N, K, seed)
        want, got = dev.empty((M, N), np.float32), dev.empty((M, N), np.float32)
        dev.linear_i8(A, W, bias, want, M, N, K, mode)
        dev.linear_i8_noalloc(A, W, bias, got, M, N, K, mode)
        w, g = want.numpy(), got.numpy()
        assert np.all(np.isfinite(g))
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (M, N, K, mode)
        for a in (A, bias, want, got):
            a.free()
        W.free()


def _noalloc_bytes(M, K):
    """Scratch the call needs (esm_gfx950_linear_i8_noalloc's layout)."""
    up = lambda v: (v + 255) // 256 * 256
    return up(M * ((K + 15) // 16 * 16)) + up(4 * M) + 256


def test_linear_i8_noalloc_rejects_oversized_calls(dev):
    """A call whose activations exceed the 64 MiB scratch fails with
    OUT_OF_RANGE before launching anything. Every buffer is sized for the
    whole call, so memory safety never depends on the rejection."""
    M, N, K = 40000, 16, 2560
    assert _noalloc_bytes(M, K) > (64 << 20) + (32 << 20)
    A = dev.array(np.zeros((M, K), np.float32))
    _, W, bias = _case(dev, 8, N, K, 3)
    out = dev.empty((M, N), np.float32)
    with pytest.raises(eg.Gfx950Error, match="exceed its 64 MiB static scratch"):
        dev.linear_i8_noalloc(A, W, bias, out, M, N, K, eg.ACT_PER_TOKEN)
    # The largest call that fits, then a small one: both equal linear_i8.
    M2 = 26000
    assert _noalloc_bytes(M2, K) <= 64 << 20
    for m in (M2, 8):
        want, got = dev.empty((m, N), np.float32), dev.empty((m, N), np.float32)
        x = dev.array(rng(m).standard_normal((m, K)).astype(np.float32))
        dev.linear_i8(x, W, bias, want, m, N, K, eg.ACT_PER_TOKEN)
        dev.linear_i8_noalloc(x, W, bias, got, m, N, K, eg.ACT_PER_TOKEN)
        assert np.array_equal(got.numpy(), want.numpy()), m
        for a in (want, got, x):
            a.free()
    for a in (A, out, bias):
        a.free()
    W.free()
