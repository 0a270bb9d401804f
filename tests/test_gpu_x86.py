"""The reference's x86 AVX-512 CPU path on gfx950, bit for bit.

Every x86 op against the oracle's lane-by-lane restatement (oracle/oracle_x86.c,
itself bit-equal to the reference's compiled AVX-512 kernels: tests/test_x86_oracle.py):
LayerNormAvx512, GeluAvx512, LinearAvx512, RopeApplyVarlenAvx512,
AttentionVarlenAvx512 (its std::exp tail keys included), and the device
restatement of glibc's expf against glibc itself on every float.

The forward in ESM_GFX950_NUMERICS_X86_AVX512 / _X86_AMX against the
reference's own CPU forward (oracle/_ref, ESM_FORCE_ISA=avx512vnni / amx)
and the oracle's: identical logits, every bit -- at 2 layers of the 650M and
3B shapes, on config 1's all-fp32 8M model, and at full 33-layer depth
against the committed fixture tests/golden/full_depth_650m.npz.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import esm_gfx950 as eg
from conftest import ROOT, cu_from_lengths, rng
from esm_gfx950 import synthetic as syn

FIXTURE = os.path.join(ROOT, "tests", "golden", "full_depth_650m.npz")


def assert_bits(got, want, what=""):
    got = np.ascontiguousarray(got, np.float32)
    want = np.ascontiguousarray(want, np.float32)
    assert got.shape == want.shape, what
    diff = got.view(np.uint32) != want.view(np.uint32)
    both_nan = np.isnan(got) & np.isnan(want)
    bad = diff & ~both_nan
    n = int(bad.sum())
    assert n == 0, f"{what}: {n} of {got.size} values differ, e.g. {got[bad][:4]} vs {want[bad][:4]}"


@pytest.mark.parametrize("d", [1280, 2560, 320, 480, 100, 37])
def test_layernorm_avx512(dev, oracle, d):
    r = rng(d)
    x = (r.standard_normal((257, d)) * r.uniform(0.05, 8.0, size=(257, 1)) + r.uniform(-3, 3, size=(257, 1))
         ).astype(np.float32)
    g = (1 + 0.02 * r.standard_normal(d)).astype(np.float32)
    b = (0.02 * r.standard_normal(d)).astype(np.float32)
    out = dev.empty(x.shape, np.float32)
    dev.layernorm_avx512(dev.array(x), dev.array(g), dev.array(b), 1e-5, out, x.shape[0], d)
    assert_bits(out.numpy(), oracle.x86_layernorm(x, g, b), f"layernorm d={d}")


def test_gelu_avx512(dev, oracle):
    r = rng(3)
    x = np.concatenate([r.standard_normal(1 << 20) * s for s in (0.3, 2.0, 6.0)] +
                       [np.linspace(-20, 20, 400001), [0.0, -0.0, 13.2, -13.3, 1e-30, -1e-30, 88.0]]).astype(np.float32)
    out = dev.empty(x.shape, np.float32)
    dev.gelu_avx512(dev.array(x), out, x.size)
    assert_bits(out.numpy(), oracle.x86_gelu(x), "gelu")


def test_expf_glibc_on_every_nonpositive_float(dev, oracle):
    """The device's glibc expf equals glibc's expf on every float <= 0 (the
    attention feeds it score - max <= 0; NaNs compare as NaN), in chunks of
    2^26, and on 2^22 random floats in (0, 89]."""
    chunk = 1 << 26
    xd, yd = dev.empty((chunk,), np.float32), dev.empty((chunk,), np.float32)
    checked = 0
    for start in range(0x80000000, 0x100000000, chunk):
        x = np.arange(start, start + chunk, dtype=np.uint32).view(np.float32)
        xd.upload(x)
        dev.expf_glibc(xd, yd, chunk)
        assert_bits(yd.numpy(), oracle.expf(x), f"expf chunk at 0x{start:08x}")
        checked += chunk
    x = rng(89).uniform(0, 89, size=1 << 22).astype(np.float32)
    x[:2] = [0.0, 88.72283]
    out = dev.empty(x.shape, np.float32)
    dev.expf_glibc(dev.array(x), out, x.size)
    assert_bits(out.numpy(), oracle.expf(x), "expf positive sample")
    print(f"expf_glibc: {checked + x.size} floats equal to glibc")
    xd.free()
    yd.free()


@pytest.mark.parametrize("M,N,K", [(37, 1283, 1280), (300, 33, 1280), (65, 48, 33), (16, 16, 1)])
def test_linear_f32_avx512(dev, oracle, M, N, K):
    r = rng(M * N + K)
    A = r.standard_normal((M, K)).astype(np.float32)
    W = (0.05 * r.standard_normal((N, K))).astype(np.float32)
    bias = r.standard_normal(N).astype(np.float32)
    out = dev.empty((M, N), np.float32)
    dev.linear_f32_avx512(dev.array(A), dev.array(W), dev.array(bias), out, M, N, K)
    assert_bits(out.numpy(), oracle.x86_linear_f32(A, W, bias), f"linear {M}x{N}x{K}")


@pytest.mark.parametrize("dh", [16, 32, 64])
def test_rope_and_attention_avx512(dev, oracle, dh):
    """Ragged lengths around the 16-key chunking (1, 15, 16, 17, ...) and a
    1024-token sequence; Q pre-scaled as the reference does."""
    lengths = [1, 15, 16, 17, 250, 33, 1024, 2, 64]
    cu = cu_from_lengths(lengths)
    T, H = int(cu[-1]), 3
    r = rng(dh)
    q = (r.standard_normal((T, H * dh)) * (1.0 / np.sqrt(dh))).astype(np.float32)
    k = r.standard_normal((T, H * dh)).astype(np.float32)
    v = r.standard_normal((T, H * dh)).astype(np.float32)
    cos, sin = eg.rope_build_tables(1024, dh)
    qd, kd, vd, od = dev.array(q), dev.array(k), dev.array(v), dev.empty((T, H * dh), np.float32)
    cd, sd = dev.array(cos), dev.array(sin)
    dev.rope_apply_varlen_avx512(qd, cd, sd, cu, H, dh)
    dev.rope_apply_varlen_avx512(kd, cd, sd, cu, H, dh)
    qr = oracle.x86_rope_varlen(q, cos, sin, cu, H, dh)
    kr = oracle.x86_rope_varlen(k, cos, sin, cu, H, dh)
    assert_bits(qd.numpy(), qr, "rope q")
    assert_bits(kd.numpy(), kr, "rope k")
    dev.attention_varlen_avx512(qd, kd, vd, cu, H, dh, od)
    assert_bits(od.numpy(), oracle.x86_attention_varlen(qr, kr, v, cu, H, dh), f"attention dh={dh}")


def test_attention_avx512_config2(dev, oracle):
    """Config 2's shape: 256 sequences, lengths clip(N(120, 30), 60, 250), 20
    heads of 64."""
    lengths = syn.varlen_lengths(256, seed=20261201 + 2)
    cu = cu_from_lengths(lengths)
    T, H, dh = int(cu[-1]), 20, 64
    r = rng(2)
    q = (r.standard_normal((T, H * dh)) / 8).astype(np.float32)
    k = r.standard_normal((T, H * dh)).astype(np.float32)
    v = r.standard_normal((T, H * dh)).astype(np.float32)
    out = dev.empty((T, H * dh), np.float32)
    dev.attention_varlen_avx512(dev.array(q), dev.array(k), dev.array(v), cu, H, dh, out)
    assert_bits(out.numpy(), oracle.x86_attention_varlen(q, k, v, cu, H, dh), "attention config 2")


def test_attention_avx512_zero_weights_against_nonfinite_v(dev, oracle):
    """The reference skips a zero weight (attention.cpp:392), so a key whose
    weight is exactly 0 adds nothing even when its V row holds an Inf or a
    NaN, while the queries that give it a weight carry the Inf / NaN. Every
    Q row is constant: 1 for half the queries, 1e-4 for the others; the
    marked keys (inside whole 16-key chunks) are -88 / 64 in every dim, so
    for the first half their score lies 88.0-88.3 below the maximum, where
    the reference's chunk exponential returns exactly 0 (2^-127 built from a
    zero exponent field), and for the second half every weight is about
    1 / L. Lengths give 128-query items with both halves, with one half,
    and short ones."""
    lengths = [200, 70, 130, 40]
    cu = cu_from_lengths(lengths)
    T, H, dh = int(cu[-1]), 2, 64
    r = rng(77)
    small = r.random(T) < 0.5
    q = np.repeat(np.where(small, 1e-4, 1.0)[:, None], H * dh, axis=1).astype(np.float32)
    k = (r.standard_normal((T, H * dh)) * 0.01).astype(np.float32)
    v = r.standard_normal((T, H * dh)).astype(np.float32)
    marked = [int(cu[0]) + 5, int(cu[0]) + 150, int(cu[1]) + 3, int(cu[2]) + 17, int(cu[3]) + 31]
    for t in marked:
        k[t] = -88.0 / dh
    v[marked[0]] = np.inf
    v[marked[1], :dh] = np.nan
    v[marked[2], dh:] = -np.inf
    v[marked[3], 7] = np.inf
    v[marked[4], dh + 1] = np.nan
    out = dev.empty((T, H * dh), np.float32)
    dev.attention_varlen_avx512(dev.array(q), dev.array(k), dev.array(v), cu, H, dh, out)
    want = oracle.x86_attention_varlen(q, k, v, cu, H, dh)
    # The case is the intended one: the first half's outputs stay finite,
    # the second half's are not.
    assert np.isfinite(want[~small]).all() and not np.isfinite(want[small]).all()
    assert_bits(out.numpy(), want, "zero weights against non-finite V")


def _x86_model(dev, w, int8, numerics):
    m = eg.Model(dev, w, int8=int8, act_mode=eg.ACT_PER_TENSOR)
    m.set_numerics(numerics)
    return m


@pytest.mark.parametrize("numerics,isa", [(eg.NUMERICS_X86_AVX512, "avx512vnni"), (eg.NUMERICS_X86_AMX, "amx")])
def test_x86_forward_650m_two_layers(dev, oracle, numerics, isa):
    """T = 446 (a 30-row tail for LinearAmx). Against the oracle, and against
    the reference's compiled forward where oracle/_ref is present."""
    w = syn.make_weights(syn.ESM2_650M.with_layers(2), seed=20261201 + 4, int8=True, keep_f32_linears=False)
    b = syn.config4_varlen_batch().subset([4, 5, 6, 7])
    m = _x86_model(dev, w, True, numerics)
    m.set_parts(2)  # x86 numerics run as one group whatever the setting
    got = m.forward_packed(b.ids, b.cu)
    m.free()
    assert_bits(got, oracle.forward_packed(w, b, int8=True, per_token=False, x86=isa), f"oracle {isa}")
    from pyoracle import REF_LIB, RefLib, RefModel
    if os.path.exists(REF_LIB):
        ref = RefLib(threads=8)
        if isa == "avx512vnni" or ref.host_isa() == "amx":
            os.environ["ESM_FORCE_ISA"] = isa
            try:
                rm = RefModel(ref, w, int8=True)
                assert_bits(got, rm.forward_packed(b), f"reference {isa}")
                rm.free()
            finally:
                os.environ.pop("ESM_FORCE_ISA", None)


def test_x86_forward_3b_shapes(dev, oracle):
    """Config 5's shapes (d = 2560, 40 heads, K = 10240), one 520-token and
    one 90-token sequence, two layers; both x86 numerics."""
    w = syn.make_weights(syn.ESM2_3B.with_layers(2), seed=20261201 + 5, int8=True, keep_f32_linears=False)
    b = syn.batch_from_lengths([520, 90, 17], seed=5)
    for numerics, isa in ((eg.NUMERICS_X86_AVX512, "avx512vnni"), (eg.NUMERICS_X86_AMX, "amx")):
        m = _x86_model(dev, w, True, numerics)
        got = m.forward_packed(b.ids, b.cu)
        m.free()
        assert_bits(got, oracle.forward_packed(w, b, int8=True, per_token=False, x86=isa), f"3B {isa}")


def test_x86_forward_config1_fp32(dev, oracle):
    """Config 1 (8M, all fp32: LinearAvx512 everywhere, head_dim 16)."""
    w = syn.make_weights(syn.ESM2_8M, seed=20261201 + 1, int8=False)
    b = syn.config1_batch()
    m = _x86_model(dev, w, False, eg.NUMERICS_X86_AVX512)
    got = m.forward_packed(b.ids, b.cu)
    m.free()
    assert_bits(got, oracle.forward_packed(w, b, int8=False, per_token=False, x86=True), "config 1 x86")


@pytest.fixture(scope="module")
def full_depth():
    if not os.path.exists(FIXTURE):
        pytest.skip("tests/golden/full_depth_650m.npz missing")
    with np.load(FIXTURE) as z:
        data = {k: z[k] for k in z.files}
    w = syn.make_weights(syn.ESM2_650M, seed=20261201 + 4, int8=True, keep_f32_linears=False)
    return data, w


@pytest.mark.parametrize("numerics,key", [(eg.NUMERICS_X86_AVX512, "ref_avx512vnni"), (eg.NUMERICS_X86_AMX, "ref_amx")])
def test_x86_forward_full_depth_equals_reference(dev, full_depth, numerics, key):
    """All 33 layers of the 650M model: the GPU's logits equal the
    reference's own CPU forward (committed fixture) bit for bit."""
    data, w = full_depth
    if key not in data:
        pytest.skip(f"fixture has no {key}")
    m = _x86_model(dev, w, True, numerics)
    got = m.forward_packed(data["ids"], data["cu"])
    m.free()
    assert_bits(got, data[key], f"33 layers vs {key}")
