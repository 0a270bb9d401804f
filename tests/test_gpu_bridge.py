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


# ----------------------------------------------------------- forward level
import esm_gfx950 as eg  # noqa: E402
from esm_gfx950 import synthetic as syn  # noqa: E402


@pytest.fixture(scope="module")
def w650_two():
    return syn.make_weights(syn.ESM2_650M.with_layers(2), seed=20261201 + 4, int8=True, keep_f32_linears=False)


def test_forward_packed_through_batchview(bridge, dev, w650_two):
    """ForwardPacked(model, BatchView) -- the forward-level hand-off that
    ForwardPackedInto makes (model.cpp:1093-1255) -- against the library's
    packed forward: the per-sequence split of model.cpp:1240-1252 of the
    same logits, bit for bit; with hidden states the layout of
    ForwardPackedInto's hidden_packed_out, and with masks the masked forward."""
    b = syn.batch_from_lengths([130, 61, 250, 2, 97], seed=21)
    cfg = w650_two.cfg
    m = eg.Model(dev, w650_two, int8=True, act_mode=eg.ACT_PER_TOKEN)
    try:
        want = m.forward_packed(b.ids, b.cu)
        per_seq, _ = bridge.forward_packed(m, b.ids, b.cu)
        assert len(per_seq) == len(b.lengths)
        for s in range(len(b.lengths)):
            assert np.array_equal(per_seq[s], want[b.cu[s]:b.cu[s + 1]])
        want_l, want_h = m.forward_hidden_states(b.ids, b.cu)
        per_seq, hidden = bridge.forward_packed(m, b.ids, b.cu, layers=cfg.num_layers, hidden_size=cfg.hidden_size)
        assert np.array_equal(np.concatenate(per_seq), want_l)
        assert np.array_equal(hidden, want_h)
        masks = np.ones_like(b.ids)
        masks[b.cu[1] - 9:b.cu[1]] = 0
        want = m.forward_packed_masked(b.ids, masks, b.cu)
        per_seq, _ = bridge.forward_packed(m, b.ids, b.cu, masks=masks)
        assert np.array_equal(np.concatenate(per_seq), want)
    finally:
        m.free()


@pytest.mark.parametrize("case,msg", [
    ("batch0", "batch_size must be >= 1"),
    ("cu_size", "must equal batch_size + 1"),
    ("cu0", "cu_seqlens[0] must be 0"),
    ("decreasing", "non-decreasing"),
    ("back", "must equal packed_ids.size()"),
])
def test_forward_packed_batchview_errors(bridge, dev, w650_two, case, msg):
    """BatchView's own validation (src/batch.cpp:8-46) rejects the batch
    before the device is touched, with the reference's messages."""
    ids = np.full(10, 5, np.int32)
    cu = {"batch0": [0], "cu_size": [0, 5, 10], "cu0": [1, 10], "decreasing": [0, 6, 4, 10],
          "back": [0, 9]}[case]
    nb = {"batch0": 0, "cu_size": 1, "cu0": 1, "decreasing": 3, "back": 1}[case]
    m = eg.Model(dev, w650_two, int8=True, act_mode=eg.ACT_PER_TOKEN)
    try:
        c = np.array(cu, np.int32)
        logits = np.zeros((10, 33), np.float32)
        rc = bridge.lib.esm_gfx950_bridge_forward_packed(m.handle, ids.ctypes.data, None, c.ctypes.data, len(c), nb,
                                                         10, logits.ctypes.data, None)
        assert rc == -1
        assert msg in bridge.error()
    finally:
        m.free()


def test_forward_scheduled_through_bridge(bridge, dev, w650_two):
    """ForwardScheduled through the bridge: without masks the library's
    pipelined scheduled forward, with masks the PlanBatches groups as masked
    packed forwards. Per-token scales make every row depend on its own
    sequence only, so each output, in input order, equals that sequence's
    rows of one packed forward of the whole batch, bit for bit."""
    lengths = [40, 250, 33, 120, 61, 200, 7, 90]
    b = syn.batch_from_lengths(lengths, seed=23)
    seqs = [b.ids[b.cu[i]:b.cu[i + 1]] for i in range(len(lengths))]
    m = eg.Model(dev, w650_two, int8=True, act_mode=eg.ACT_PER_TOKEN)
    try:
        whole = m.forward_packed(b.ids, b.cu)
        out = bridge.forward_scheduled(m, seqs)
        for i in range(len(lengths)):
            assert np.array_equal(out[i], whole[b.cu[i]:b.cu[i + 1]])
        masks = [np.ones_like(s) for s in seqs]
        masks[1][-30:] = 0
        masks[5][100:110] = 0
        whole_m = m.forward_packed_masked(b.ids, np.concatenate(masks), b.cu)
        out = bridge.forward_scheduled(m, seqs, masks=masks)
        for i in range(len(lengths)):
            assert np.array_equal(out[i], whole_m[b.cu[i]:b.cu[i + 1]])
    finally:
        m.free()


def test_weight_cache_sees_in_place_rewrite(bridge):
    """A QuantizedTensor whose int8 values are rewritten in place (same
    storage, same scales) gets a new device copy: the second LinearInt8 call
    uses the new values."""
    r = rng(77)
    M, N, K = 64, 256, 512
    A = r.normal(0, 1, size=(M, K)).astype(np.float32)
    q = r.integers(-127, 128, size=(N, K), dtype=np.int8)
    s = r.uniform(0.005, 0.05, size=N).astype(np.float32)
    qt = bridge.lib.esm_gfx950_bridge_qt_create(q.ctypes.data, s.ctypes.data, N, K)
    try:
        out1 = np.zeros((M, N), np.float32)
        assert bridge.lib.esm_gfx950_bridge_linear_int8_qt(A.ctypes.data, qt, None, out1.ctypes.data, M) == 1
        import ctypes as C
        view = np.ctypeslib.as_array(C.cast(bridge.lib.esm_gfx950_bridge_qt_data(qt), C.POINTER(C.c_int8)),
                                     shape=(N, K))
        view[:] = -view  # in place: same pointer, same scales
        out2 = np.zeros((M, N), np.float32)
        assert bridge.lib.esm_gfx950_bridge_linear_int8_qt(A.ctypes.data, qt, None, out2.ctypes.data, M) == 1
        fresh = bridge.linear_int8(A, -q, s, None)
        assert np.array_equal(out2, fresh)
        assert np.array_equal(out2, -out1)
    finally:
        bridge.lib.esm_gfx950_bridge_qt_free(qt)
