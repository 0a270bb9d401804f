"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Three independent anchors per function:
  1. the reference's own known-answer tests (values copied from
     tests/cpp/test_kernels.cpp, test_act_quant.cpp, test_quant.cpp,
     test_attention_varlen.cpp), stored in tests/golden/kats.json;
  2. the reference itself, compiled from its sources into
     oracle/_ref/libesmref.so -- bitwise equality for every *Ref function,
     and for the VNNI/AMX int8 path with identity scales;
  3. closed forms / invariants computed independently in numpy (float64
     softmax attention, int64 matmul, rotation norms, LN moments).
"""
import json
import os

import numpy as np
import pytest

from conftest import ROOT, cu_from_lengths, rng

GOLDEN = os.path.join(ROOT, "tests", "golden")


@pytest.fixture(scope="module")
def kats():
    with open(os.path.join(GOLDEN, "kats.json")) as f:
        return json.load(f)


# ------------------------------------------------------------------ KATs
def test_kat_linear(oracle, kats):
    k = kats["linear_2x3_times_4x3_plus_bias"]
    got = oracle.linear_f32(np.array(k["A"], np.float32), np.array(k["W"], np.float32), np.array(k["bias"], np.float32))
    assert np.allclose(got.ravel(), k["expected"], atol=1e-5)
    k = kats["linear_no_bias"]
    got = oracle.linear_f32(np.array(k["A"], np.float32), np.array(k["W"], np.float32), None)
    assert np.allclose(got.ravel(), k["expected"], atol=1e-5)


def test_kat_layernorm(oracle, kats):
    for name in ("layernorm_unit", "layernorm_gamma_beta"):
        k = kats[name]
        x = np.array([k["x"]], np.float32)
        got = oracle.layernorm(x, np.array(k["gamma"], np.float32), np.array(k["beta"], np.float32), 1e-5)
        assert np.allclose(got.ravel(), k["expected"], atol=1e-5), name


def test_kat_gelu(oracle, kats):
    k = kats["gelu_known_values"]
    got = oracle.gelu(np.array(k["x"], np.float32))
    assert np.allclose(got, k["expected"], atol=1e-5)


def test_kat_rope(oracle, kats):
    k = kats["rope_dh4_pos1"]
    c, s = oracle.rope_tables(2, 4)
    assert np.allclose(c[0], 1.0) and np.allclose(s[0], 0.0)
    assert np.array_equal(c[:, :2], c[:, 2:]) and np.array_equal(s[:, :2], s[:, 2:])
    x = np.array(k["x"], np.float32).reshape(2, 1, 4)
    got = oracle.rope_varlen(x, c, s, np.array([0, 2], np.int32), 1, 4)
    assert np.allclose(got.ravel()[4:], k["expected_pos1"], atol=1e-5)
    assert np.array_equal(got.ravel()[:4], x.ravel()[:4])  # position 0 is the identity


def test_kat_attention_single_token(oracle, kats):
    k = kats["attention_single_token"]
    q = np.array(k["q"], np.float32).reshape(1, 1, 2)
    kk = np.array(k["k"], np.float32).reshape(1, 1, 2)
    v = np.array(k["v"], np.float32).reshape(1, 1, 2)
    got = oracle.attention_varlen(q, kk, v, np.array([0, 1], np.int32), 1, 2)
    assert np.allclose(got.ravel(), k["expected"], atol=1e-5)


def test_kat_act_quant(oracle, kats):
    k = kats["act_quant_clamp"]
    # per-tensor scale 0.1 is what the reference test feeds; with absmax 1000
    # the dynamic scale is 1000/127, so check the clamp/zero-point semantics
    q, s = oracle.quant_act_tensor(np.array(k["x"], np.float32))
    assert q[0] == 127 and q[1] == -127 and q[2] == 0
    assert s == np.float32(1000.0) / np.float32(127.0)
    q0, s0 = oracle.quant_act_tensor(np.zeros(5, np.float32))
    assert s0 == 1.0 and np.all(q0 == 0)


def test_kat_quantize(oracle, kats):
    k = kats["quantize_intermediate"]
    q, s = oracle.quantize_weight(np.array([k["W"]], np.float32))
    assert abs(s[0] - 1.0 / 127.0) < 1e-9
    assert q[0, 0] == 127 and q[0, 1] == -127 and q[0, 4] == 0
    assert np.all(np.abs(q[0].astype(np.float32) - np.array(k["W"], np.float32) * 127.0) <= 1.0)
    qz, sz = oracle.quantize_weight(np.zeros((2, 5), np.float32))
    assert np.all(sz == 0) and np.all(qz == 0)


# --------------------------------------------------- committed golden vectors
def test_golden_vectors(oracle):
    """Vectors written by tests/golden/make_golden.py from the reference build."""
    g = np.load(os.path.join(GOLDEN, "ref_vectors.npz"), allow_pickle=False)
    assert np.array_equal(oracle.attention_varlen(g["attn_q"], g["attn_k"], g["attn_v"], g["attn_cu"], 4, 16),
                          g["attn_out"])
    assert np.array_equal(oracle.layernorm(g["ln_x"], g["ln_g"], g["ln_b"], 1e-5), g["ln_out"])
    assert np.array_equal(oracle.gelu(g["gelu_x"]), g["gelu_out"])
    c, s = oracle.rope_tables(12, 16)
    assert np.array_equal(c, g["rope_cos"]) and np.array_equal(s, g["rope_sin"])
    assert np.array_equal(oracle.rope_varlen(g["rope_x"], c, s, g["rope_cu"], 3, 16), g["rope_out"])
    q, sc = oracle.quantize_weight(g["quant_w"])
    assert np.array_equal(q, g["quant_q"]) and np.array_equal(sc, g["quant_s"])
    assert np.array_equal(oracle.linear_f32(g["lin_a"], g["lin_w"], g["lin_b"]), g["lin_out"])
    acc = oracle.gemm_i8_i32(g["i8_a"], g["i8_w"])
    assert np.array_equal(acc.astype(np.float32), g["i8_out"])
    aq, ascale = oracle.quant_act_tensor(g["actq_x"])
    assert np.array_equal(aq.astype(np.int32) + 128, g["actq_u8"].astype(np.int32)) and ascale == g["actq_scale"]
    got = oracle.dequant(oracle.gemm_i8_i32(aq.reshape(g["vnni_m"], -1), g["vnni_wq"]),
                         np.full(int(g["vnni_m"]), ascale, np.float32), g["vnni_ws"], g["vnni_b"])
    assert np.array_equal(got, g["vnni_out"])


# ------------------------------------------- live reference build (bitwise)
def test_vs_reference_build_ref_twins(oracle, ref):
    r = rng(0)
    A = r.uniform(-1, 1, (37, 320)).astype(np.float32)
    W = r.uniform(-1, 1, (50, 320)).astype(np.float32)
    b = r.uniform(-1, 1, 50).astype(np.float32)
    assert np.array_equal(oracle.linear_f32(A, W, b), ref.linear_ref(A, W, b))
    x = r.standard_normal((37, 1280)).astype(np.float32)
    g = r.standard_normal(1280).astype(np.float32)
    assert np.array_equal(oracle.layernorm(x, g, g), ref.layernorm_ref(x, g, g))
    assert np.array_equal(oracle.gelu(x), ref.gelu_ref(x))
    for L, dh in ((100, 16), (250, 64), (1024, 64)):
        c1, s1 = oracle.rope_tables(L, dh)
        c2, s2 = ref.rope_tables(L, dh)
        assert np.array_equal(c1, c2) and np.array_equal(s1, s2)
    cu = cu_from_lengths([40, 1, 59, 0, 33])
    T = int(cu[-1])
    q, k, v = (r.standard_normal((T, 5, 16)).astype(np.float32) for _ in range(3))
    c, s = oracle.rope_tables(59, 16)
    assert np.array_equal(oracle.rope_varlen(q, c, s, cu, 5, 16), ref.rope_varlen_ref(q, c, s, cu, 5, 16))
    assert np.array_equal(oracle.attention_varlen(q, k, v, cu, 5, 16), ref.attention_varlen_ref(q, k, v, cu, 5, 16))
    qw, sw = oracle.quantize_weight(W)
    qr, sr = ref.quantize(W)
    assert np.array_equal(qw, qr) and np.array_equal(sw, sr)
    assert np.array_equal(oracle.linear_int8_w8a16(A, qw, sw, b), ref.linear_int8_ref(A, qw, sw, b))


@pytest.mark.parametrize("M,N,K", [(32, 64, 64), (64, 1280, 1280), (50, 96, 320), (96, 1280, 5120)])
def test_vs_reference_build_int8(oracle, ref, M, N, K):
    """int32 closed form == the reference VNNI/AMX path with identity scales:
    A integer-valued with max|A| = 127 gives act_scale = 1 exactly, so
    C = fma(float(acc), 1, 0) = float(acc), exact for |acc| < 2^24."""
    if ref.host_isa() not in ("avx512vnni", "amx"):
        pytest.skip("host lacks VNNI")
    r = rng(M + N + K)
    A = r.integers(-127, 128, (M, K)).astype(np.int8)
    A[0, 0] = 127
    W = r.integers(-127, 128, (N, K)).astype(np.int8)
    acc = oracle.gemm_i8_i32(A, W)
    ones = np.ones(N, np.float32)
    zeros = np.zeros(N, np.float32)
    assert np.array_equal(ref.linear_int8(A.astype(np.float32), W, ones, zeros), acc.astype(np.float32))
    assert np.array_equal(ref.linear_vnni(A.astype(np.float32), W, ones, zeros), acc.astype(np.float32))


def test_vs_reference_build_w8a8_dequant(oracle, ref):
    """Oracle quant -> int32 -> dequant == reference LinearVnni bit for bit
    (same per-tensor scale, same fma epilogue)."""
    if ref.host_isa() not in ("avx512vnni", "amx"):
        pytest.skip("host lacks VNNI")
    r = rng(9)
    M, N, K = 64, 1280, 1280
    A = r.uniform(-3, 3, (M, K)).astype(np.float32)
    q, s = oracle.quantize_weight(r.uniform(-0.1, 0.1, (N, K)).astype(np.float32))
    b = r.uniform(-1, 1, N).astype(np.float32)
    aq, sc = oracle.quant_act_tensor(A)
    want = oracle.dequant(oracle.gemm_i8_i32(aq, q), np.full(M, sc, np.float32), s, b)
    assert np.array_equal(ref.linear_vnni(A, q, s, b), want)
    u8, sc2 = ref.quant_act_prefix(A)
    assert sc2 == sc and np.array_equal(u8.astype(np.int32) - 128, aq.astype(np.int32))


@pytest.mark.parametrize("fc1_fp16", [False, True])
def test_vs_reference_build_forward_fp32(oracle, ref, fc1_fp16):
    """Restated fp32 forward == the reference's kernels forced to the Ref ISA
    (with and without the first-block fp16 rounding of the fc1 input)."""
    from esm_gfx950 import synthetic as syn
    from pyoracle import RefModel
    cfg = syn.EsmConfig("tiny", 2, 64, 4, 128)
    w = syn.make_weights(cfg, seed=5)
    batch = syn.batch_from_lengths([9, 30, 2, 17], seed=5)
    os.environ["ESM_FORCE_ISA"] = "ref"
    try:
        m = RefModel(ref, w, int8=False, fc1_fp16=fc1_fp16)
        want = m.forward_packed(batch)
        m.free()
    finally:
        del os.environ["ESM_FORCE_ISA"]
    got = oracle.forward_packed(w, batch, int8=False, per_token=False, fc1_fp16=fc1_fp16)
    assert np.array_equal(got, want)
    if fc1_fp16:
        assert not np.array_equal(got, oracle.forward_packed(w, batch, int8=False, per_token=False))


def test_closed_form_round_fp16(oracle):
    """RoundToFp16Inplace == numpy's IEEE round-to-nearest-even float16 cast:
    normals, ties, subnormals, overflow to inf, NaN."""
    r = rng(11)
    x = np.concatenate([r.normal(0, 1, 4000), r.normal(0, 3e4, 500), r.normal(0, 1e-5, 500),
                        [1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 65504.0, 65520.0, 7e4, -7e4, 2.0 ** -25, 0.0, -0.0]])
    x = x.astype(np.float32)
    with np.errstate(over="ignore"):  # the overflow to inf is one of the cases
        want = x.astype(np.float16).astype(np.float32)
    got = oracle.round_fp16(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------- independent closed forms
def test_closed_form_int8_gemm(oracle):
    r = rng(1)
    A = r.integers(-127, 128, (23, 77)).astype(np.int8)
    W = r.integers(-127, 128, (41, 77)).astype(np.int8)
    assert np.array_equal(oracle.gemm_i8_i32(A, W), A.astype(np.int64) @ W.astype(np.int64).T)


def test_closed_form_attention(oracle):
    """float64 softmax(q k^T) v per sequence and head; q = 0 gives mean(v)."""
    r = rng(2)
    lengths = [13, 1, 40]
    cu = cu_from_lengths(lengths)
    T, H, dh = int(cu[-1]), 3, 8
    q, k, v = (r.standard_normal((T, H, dh)).astype(np.float32) for _ in range(3))
    got = oracle.attention_varlen(q, k, v, cu, H, dh).reshape(T, H, dh)
    for b in range(len(lengths)):
        sl = slice(cu[b], cu[b + 1])
        for h in range(H):
            s = q[sl, h].astype(np.float64) @ k[sl, h].astype(np.float64).T
            p = np.exp(s - s.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            np.testing.assert_allclose(got[sl, h], p @ v[sl, h], rtol=1e-5, atol=1e-5)
    z = oracle.attention_varlen(np.zeros_like(q), k, v, cu, H, dh).reshape(T, H, dh)
    np.testing.assert_allclose(z[cu[2]:cu[3]], np.broadcast_to(v[cu[2]:cu[3]].mean(0), (40, H, dh)), atol=1e-6)


def test_closed_form_rope(oracle):
    """Rotation keeps each (i, i + dh/2) pair's norm; positions restart per sequence."""
    r = rng(3)
    dh = 64
    cu = cu_from_lengths([50, 20])
    x = r.standard_normal((70, 2, dh)).astype(np.float32)
    c, s = oracle.rope_tables(50, dh)
    y = oracle.rope_varlen(x, c, s, cu, 2, dh)
    n_in = x[..., :32] ** 2 + x[..., 32:] ** 2
    n_out = y[..., :32] ** 2 + y[..., 32:] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5)
    assert np.array_equal(y[50], x[50])  # second sequence position 0: identity
    ang = np.arange(50)[:, None] * (10000.0 ** (-np.arange(32) * 2 / dh))[None, :]
    np.testing.assert_allclose(c[:, :32], np.cos(ang), atol=2e-6)


def test_closed_form_layernorm_and_gelu(oracle):
    r = rng(4)
    x = (r.standard_normal((16, 1280)) * 3 + 1).astype(np.float32)
    y = oracle.layernorm(x, np.ones(1280, np.float32), np.zeros(1280, np.float32), 1e-5)
    np.testing.assert_allclose(y.mean(1), 0, atol=1e-5)
    np.testing.assert_allclose(y.std(1), 1, atol=1e-4)
    from math import erf, sqrt
    xs = np.linspace(-6, 6, 97).astype(np.float32)
    want = np.array([float(t) * 0.5 * (1 + erf(float(t) / sqrt(2))) for t in xs])
    np.testing.assert_allclose(oracle.gelu(xs), want, atol=1e-6)


def test_closed_form_quant_round_trip(oracle):
    r = rng(6)
    x = r.uniform(-1, 1, (8, 256)).astype(np.float32)
    q, s = oracle.quant_act_rows(x)
    assert np.all(np.abs(q.astype(np.float32) * s[:, None] - x) <= s[:, None] * 0.51)
    assert np.all(np.abs(q).max(1) == 127)
