"""W8A8 INT8 GEMM on gfx950 against the CPU oracle.

Bar: int32 accumulators bit-exact (closed form sum_k a*w); dequant epilogue
bit-exact (same fmaf expression); GELU epilogue within 1e-5 (device erff vs
host erff).
"""
import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu

import esm_gfx950 as eg


@pytest.fixture(params=[0, 64, 128, 256, 320], ids=["rows-auto", "rows-64", "rows-128", "rows-256", "rows-320"])
def tile_rows(request):
    """INT8 GEMM tile height (0: the per-launch choice); reset afterwards."""
    eg.set_gemm_tile_rows(request.param)
    yield request.param
    eg.set_gemm_tile_rows(0)


def _pad(a, ld):
    out = np.zeros((a.shape[0], ld), a.dtype)
    out[:, :a.shape[1]] = a
    return out


def _i8(r, shape):
    return r.integers(-127, 128, size=shape, dtype=np.int8)


@pytest.mark.parametrize("M,N,K", [
    (1, 16, 16), (37, 64, 64), (5, 9, 17), (130, 260, 48), (300, 1280, 1280), (257, 3840, 1280),
    (129, 1280, 5120), (64, 5120, 1280), (31, 2560, 10240),
    (300, 200, 512), (513, 640, 768), (260, 384, 384), (777, 1000, 2560),
])
def test_int32_bit_exact(dev, oracle, tile_rows, M, N, K):
    r = rng(1000 + M + N + K)
    A = _i8(r, (M, K))
    W = _i8(r, (N, K))
    lda = (K + 15) // 16 * 16
    w = dev.weight_i8(W, np.ones(N, np.float32))
    dA = dev.array(_pad(A, lda))
    dC = dev.empty((M, N), np.int32)
    dev.gemm_i8_i32(dA, lda, w, M, dC)
    got = dC.numpy()
    want = oracle.gemm_i8_i32(A, W)
    assert np.array_equal(got, want)
    w.free()


def test_int32_extremes(dev, oracle):
    # All +-127 / -127 operands: the largest |acc| a K=5120 product can form.
    M, N, K = 64, 128, 5120
    A = np.full((M, K), 127, np.int8)
    A[1::2] = -127
    W = np.full((N, K), -127, np.int8)
    W[::3] = 127
    w = dev.weight_i8(W, np.ones(N, np.float32))
    dA = dev.array(A)
    dC = dev.empty((M, N), np.int32)
    dev.gemm_i8_i32(dA, K, w, M, dC)
    assert np.array_equal(dC.numpy(), oracle.gemm_i8_i32(A, W))
    w.free()


def _exact_i32(A, Wt):
    """int32 closed form sum_k a*w of every element through a float64 BLAS
    product (Wt: W^T as float64): |a*w| <= 127^2 and K <= 2^20, so every
    partial sum is an integer below 2^53 and the float64 result is exact."""
    return (A.astype(np.float64) @ Wt).astype(np.int32)


@pytest.fixture(scope="module")
def config3():
    """Config 3 operands and the exact int32 product of every element."""
    M, N, K = 30700, 5120, 1280
    r = rng(3)
    A = _i8(r, (M, K))
    W = _i8(r, (N, K))
    a_scale = r.uniform(0.005, 0.05, size=M).astype(np.float32)
    w_scale = r.uniform(0.005, 0.05, size=N).astype(np.float32)
    bias = (r.standard_normal(N) * 0.02).astype(np.float32)
    Wt = W.astype(np.float64).T
    acc = np.concatenate([_exact_i32(A[r0:r0 + 4096], Wt) for r0 in range(0, M, 4096)])
    rows = np.unique(np.concatenate([r.choice(M, 16, replace=False), [0, M - 1, 30591, 30592]]))
    return A, W, a_scale, w_scale, bias, acc, rows


def test_config3_full_size(dev, oracle, tile_rows, config3):
    """Config 3 shape [30700 x 1280] x [5120 x 1280]^T over the WHOLE output:
    int32 bit-exact against the exact float64 product on every element,
    dequant+bias bit-exact (the same fmaf on both sides) and
    dequant+bias+GELU within 1e-5, every element; the oracle's own int32
    GEMM cross-checks the float64 product on a row sample."""
    A, W, a_scale, w_scale, bias, want, rows = config3
    M, K = A.shape
    N = W.shape[0]
    assert np.array_equal(oracle.gemm_i8_i32(A[rows], W), want[rows])
    w = dev.weight_i8(W, w_scale)
    dA = dev.array(A)
    dC = dev.empty((M, N), np.int32)
    dev.gemm_i8_i32(dA, K, w, M, dC)
    acc = dC.numpy()
    dC.free()
    bad = np.argwhere(acc != want)
    assert bad.size == 0, f"{len(bad)} int32 mismatches, first at (row, col) {bad[:4].tolist()}"
    del acc

    ds = dev.array(a_scale)
    db = dev.array(bias)
    dY = dev.empty((M, N), np.float32)
    step = 4096
    dev.linear_i8_q(dA, K, ds, w, db, dY, M, gelu=False)
    y = dY.numpy()
    for r0 in range(0, M, step):
        ref = oracle.dequant(want[r0:r0 + step], a_scale[r0:r0 + step], w_scale, bias, gelu=False)
        assert np.array_equal(y[r0:r0 + step], ref), r0
    dev.linear_i8_q(dA, K, ds, w, db, dY, M, gelu=True)
    y = dY.numpy()
    for r0 in range(0, M, step):
        ref = oracle.dequant(want[r0:r0 + step], a_scale[r0:r0 + step], w_scale, bias, gelu=True)
        np.testing.assert_allclose(y[r0:r0 + step], ref, rtol=1e-5, atol=1e-5)
    for t in (dY, ds, db, dA):
        t.free()
    w.free()


@pytest.mark.parametrize("mode", [eg.ACT_PER_TENSOR, eg.ACT_PER_TOKEN])
@pytest.mark.parametrize("M,N,K", [(18, 1280, 1280), (96, 320, 320), (257, 5120, 1280), (64, 1280, 5120), (7, 33, 17)])
def test_linear_int8_facade(dev, oracle, tile_rows, mode, M, N, K):
    """esm_gfx950_linear_i8 == oracle quant -> int32 GEMM -> dequant, bit-exact."""
    r = rng(77 + M + N + K + mode)
    A = r.uniform(-1, 1, size=(M, K)).astype(np.float32)
    Wf = r.uniform(-1, 1, size=(N, K)).astype(np.float32)
    q, s = oracle.quantize_weight(Wf)
    bias = r.uniform(-1, 1, size=N).astype(np.float32)
    w = dev.weight_i8(q, s)
    dA, db, dC = dev.array(A), dev.array(bias), dev.empty((M, N), np.float32)
    dev.linear_i8(dA, w, db, dC, M, N, K, mode)
    got = dC.numpy()
    if mode == eg.ACT_PER_TENSOR:
        aq, sc = oracle.quant_act_tensor(A)
        scales = np.full(M, sc, np.float32)
    else:
        aq, scales = oracle.quant_act_rows(A)
    want = oracle.dequant(oracle.gemm_i8_i32(aq, q), scales, s, bias)
    assert np.array_equal(got, want)
    w.free()


def test_tile_rows_rejects_other_heights():
    with pytest.raises(eg.Gfx950Error):
        eg.set_gemm_tile_rows(300)


def test_linear_int8_zero_sizes(dev):
    """M, N or K <= 0 zeroes C (reference gemm_int8.cpp:513-520)."""
    w = dev.weight_i8(np.ones((4, 16), np.int8), np.ones(4, np.float32))
    dC = dev.array(np.full((3, 4), 5.0, np.float32))
    dA = dev.array(np.ones((3, 16), np.float32))
    dev.linear_i8(dA, w, None, dC, 3, 4, 0, eg.ACT_PER_TENSOR)
    assert np.all(dC.numpy() == 0.0)
    w.free()


@pytest.mark.parametrize("M,K,ldq", [(333, 1280, 1280), (70, 5120, 5136), (41, 260, 272), (9, 5121, 5136)])
@pytest.mark.parametrize("mode", [eg.ACT_PER_TENSOR, eg.ACT_PER_TOKEN])
def test_quantize_act(dev, oracle, mode, M, K, ldq):
    r = rng(5 + mode + K)
    x = (r.standard_normal((M, K)) * r.uniform(0.1, 10, size=(M, 1))).astype(np.float32)
    x[7] = 0.0  # all-zero row: per-token scale 1
    # exact ties of x * (127 / absmax) land on both rounding directions
    x[3, :6] = [127.0, 0.5, -0.5, 1.5, -2.5, 126.5]
    dx, dq, ds = dev.array(x), dev.array(np.full((M, ldq), 99, np.int8)), dev.empty((M,), np.float32)
    dev.quantize_act(dx, M, K, mode, dq, ldq, ds)
    if mode == eg.ACT_PER_TENSOR:
        q, s = oracle.quant_act_tensor(x)
        s = np.full(M, s, np.float32)
    else:
        q, s = oracle.quant_act_rows(x)
    got = dq.numpy()
    assert np.array_equal(got[:, :K], q)
    assert np.all(got[:, K:] == 0)
    assert np.array_equal(ds.numpy(), s)


@pytest.mark.parametrize("M,K,ldq", [(333, 5120, 5120), (65, 1280, 1296), (40, 4000, 4000), (9, 10240, 10240),
                                     (17, 7000, 7008)])
def test_gelu_quantize_act(dev, oracle, M, K, ldq):
    """Fused GELU + per-token quantisation against GeluRef then the oracle's
    per-row quantisation. The device erf is Abramowitz & Stegun 7.1.26
    (|error| <= 1.5e-7), so a byte may differ by one where the exact product
    sits within 1e-3 of a rounding tie; scales agree to 2e-6 relative."""
    r = rng(11 + K)
    x = (r.standard_normal((M, K)) * r.uniform(0.1, 4, size=(M, 1))).astype(np.float32)
    x[3] = 0.0  # all-zero row: GELU is zero, scale 1
    x[5, :8] = [0.0, -0.0, 10.0, -10.0, 1.0, -1.0, 2.0, -30.0]
    dx, dq, ds = dev.array(x), dev.array(np.full((M, ldq), 99, np.int8)), dev.empty((M,), np.float32)
    dev.gelu_quantize_act(dx, M, K, dq, ldq, ds)
    got, s = dq.numpy(), ds.numpy()
    g = oracle.gelu(x)
    q_ref, s_ref = oracle.quant_act_rows(g)
    assert s[3] == 1.0 and np.all(got[3] == 0)
    np.testing.assert_allclose(s, s_ref, rtol=2e-6)
    d = got[:, :K].astype(np.int32) - q_ref
    assert np.abs(d).max() <= 1
    prod = g.astype(np.float64) / s_ref.astype(np.float64)[:, None]
    tie = np.abs(prod - np.floor(prod) - 0.5)
    assert np.all(tie[d != 0] < 1e-3)
    assert (d != 0).mean() < 1e-3
    assert np.all(got[:, K:] == 0)


def test_gelu_quantize_act_rejects_bad_shapes(dev):
    dx, dq, ds = dev.empty((2, 8), np.float32), dev.empty((2, 16), np.int8), dev.empty((2,), np.float32)
    with pytest.raises(eg.Gfx950Error):
        dev.gelu_quantize_act(dx, 2, 6, dq, 16, ds)  # K % 4 != 0
    with pytest.raises(eg.Gfx950Error):
        dev.gelu_quantize_act(dx, 2, 8, dq, 4, ds)  # ldq < K


def _planes_to_f32(hi, lo):
    """The 24-bit intermediate's two planes back in column order: stored
    position p = 64 g + 2 i + j holds column 64 g + 32 j + i; the low plane
    interleaves row pairs, byte (r & ~1) N + 4 (p // 2) + 2 (r & 1) + (p & 1)
    holding row r, position p."""
    M, N = hi.shape
    Mp = M + (M & 1)
    lo = lo.reshape(-1)[:Mp * N].reshape(Mp // 2, N // 2, 2, 2)  # [pair, p // 2, r & 1, p & 1]
    lo = lo.transpose(0, 2, 1, 3).reshape(Mp, N)[:M]            # [row, p]
    bits = (hi.astype(np.uint32) << 16) | (lo.astype(np.uint32) << 8)
    g = bits.reshape(M, N // 64, 32, 2)           # [.., i, j] at position 2 i + j
    cols = g.transpose(0, 1, 3, 2).reshape(M, N)  # column 32 j + i
    return cols.view(np.float32)


@pytest.mark.parametrize("M,N,K,ldq", [
    (8191, 5120, 256, 5120),    # rows < 8192, N <= 5120: two waves per row, odd row count
    (8193, 5120, 256, 5136),    # rows >= 8192: one wave per row; padded ldq
    (777, 10240, 256, 10240),   # N > 5120: four waves per row
    (333, 1280, 1280, 1296),    # narrow rows (N < 5120), the 650M K
    (65, 2560, 1280, 2560),
])
def test_linear_i8_gelu_quant_r24(dev, oracle, M, N, K, ldq):
    """The default forward's fc1 -> 24-bit intermediate -> GELU + per-token
    quantisation (esm_gfx950_linear_i8_gelu_quant_r24) against the oracle:
    the two planes bit-exact against or_round24 of the oracle's dequant
    (fma(acc, a_scale w_scale, bias), itself bit-exact), and the codes and
    scales against GeluRef + per-row quantisation of those 24-bit values,
    with test_gelu_quantize_act's allowance (the device GELU's erf is A&S
    7.1.26: a byte may differ by one next to a rounding tie). Row 7's
    activation scale is NaN: its values must stay NaN in the planes."""
    r = rng(2400 + M + N)
    A = _i8(r, (M, K))
    W = _i8(r, (N, K))
    a_s = r.uniform(0.005, 0.05, size=M).astype(np.float32)
    w_s = r.uniform(0.005, 0.05, size=N).astype(np.float32)
    bias = (r.standard_normal(N) * 0.02).astype(np.float32)
    nan_row = 7
    a_s_dev = a_s.copy()
    a_s_dev[nan_row] = np.nan
    w = dev.weight_i8(W, w_s)
    dA, da, db = dev.array(A), dev.array(a_s_dev), dev.array(bias)
    dh, dl = dev.empty((M, N), np.uint16), dev.empty((M + (M & 1), N), np.uint8)
    dq, ds = dev.array(np.full((M, ldq), 99, np.int8)), dev.empty((M,), np.float32)
    dev.linear_i8_gelu_quant_r24(dA, K, da, w, db, M, dh, dl, dq, ldq, ds)
    inter = _planes_to_f32(dh.numpy(), dl.numpy())
    got, s = dq.numpy(), ds.numpy()
    w.free()

    acc = _exact_i32(A, W.T.astype(np.float64))
    want = oracle.round24(oracle.dequant(acc, a_s, w_s, bias))
    assert np.all(np.isnan(inter[nan_row]))
    ok = np.arange(M) != nan_row
    bad = np.argwhere((inter.view(np.uint32) != want.view(np.uint32)) & ok[:, None])
    if bad.size:
        g32, w32 = inter.view(np.uint32), want.view(np.uint32)
        detail = [(int(r), int(c), hex(int(g32[r, c])), hex(int(w32[r, c]))) for r, c in bad[:6]]
        # where else does the wrong value occur in the expected array (same row or rows nearby)?
        r0, c0 = bad[0]
        hits = np.argwhere(w32[max(r0 - 8, 0):r0 + 8] == g32[r0, c0])
        raise AssertionError(f"{len(bad)} values differ; {detail}; rows {np.unique(bad[:, 0])[:16].tolist()}; "
                             f"cols {np.unique(bad[:, 1])[:40].tolist()}; got value found at {(hits + [max(r0 - 8, 0), 0])[:4].tolist()}")

    g = oracle.gelu(want[ok])
    q_ref, s_ref = oracle.quant_act_rows(g)
    np.testing.assert_allclose(s[ok], s_ref, rtol=2e-6)
    d = got[ok, :N].astype(np.int32) - q_ref
    assert np.abs(d).max() <= 1
    prod = g.astype(np.float64) / s_ref.astype(np.float64)[:, None]
    tie = np.abs(prod - np.floor(prod) - 0.5)
    assert np.all(tie[d != 0] < 1e-3)
    assert (d != 0).mean() < 1e-3
    assert np.all(got[:, N:] == 0)


def test_linear_i8_gelu_quant_r24_rejects_bad_shapes(dev):
    r = rng(5)
    w = dev.weight_i8(_i8(r, (96, 256)), np.ones(96, np.float32))  # N % 64 != 0
    dA, da = dev.array(_i8(r, (4, 256))), dev.array(np.ones(4, np.float32))
    dh, dl = dev.empty((4, 96), np.uint16), dev.empty((4, 96), np.uint8)
    dq, ds = dev.empty((4, 96), np.int8), dev.empty((4,), np.float32)
    with pytest.raises(eg.Gfx950Error):
        dev.linear_i8_gelu_quant_r24(dA, 256, da, w, None, 4, dh, dl, dq, 96, ds)
    w.free()
    w = dev.weight_i8(_i8(r, (64, 200)), np.ones(64, np.float32))  # K % 128 != 0
    with pytest.raises(eg.Gfx950Error):
        dev.linear_i8_gelu_quant_r24(dA, 208, da, w, None, 4, dh, dl, dq, 64, ds)
    w.free()
