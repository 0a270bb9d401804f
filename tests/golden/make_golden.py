"""Writes tests/golden/ref_vectors.npz: small input/output vectors produced by
the reference's own kernels, compiled from its sources into
oracle/_ref/libesmref.so (make -C oracle ref).

The *Ref functions are called directly (attention, LayerNorm, GELU, RoPE
tables and apply, fp32 Linear, weight Quantize); the INT8 vectors come from
the reference's VNNI path (LinearVnni and QuantizeActPrefixAvx512), which
needs an AVX-512 VNNI host. The fixtures let the oracle be checked on hosts
without the reference build. Run from the repository root:

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

from pyoracle import RefLib  # noqa: E402


def main():
    ref = RefLib(threads=1)
    if ref.host_isa() not in ("avx512vnni", "amx"):
        raise SystemExit("needs an AVX-512 VNNI host for the int8 vectors")
    r = np.random.default_rng(20261201)
    g = {}
    cu = np.array([0, 5, 14], np.int32)
    q, k, v = (r.standard_normal((14, 4, 16)).astype(np.float32) for _ in range(3))
    g.update(attn_q=q, attn_k=k, attn_v=v, attn_cu=cu, attn_out=ref.attention_varlen_ref(q, k, v, cu, 4, 16))
    x = (r.standard_normal((3, 47)) * 2 + 0.5).astype(np.float32)
    lg, lb = r.standard_normal(47).astype(np.float32), r.standard_normal(47).astype(np.float32)
    g.update(ln_x=x, ln_g=lg, ln_b=lb, ln_out=ref.layernorm_ref(x, lg, lb))
    gx = np.linspace(-5, 5, 101).astype(np.float32)
    g.update(gelu_x=gx, gelu_out=ref.gelu_ref(gx))
    c, s = ref.rope_tables(12, 16)
    rcu = np.array([0, 7, 7, 12], np.int32)
    rx = r.standard_normal((12, 3, 16)).astype(np.float32)
    g.update(rope_cos=c, rope_sin=s, rope_cu=rcu, rope_x=rx, rope_out=ref.rope_varlen_ref(rx, c, s, rcu, 3, 16))
    W = r.uniform(-1, 1, (7, 13)).astype(np.float32)
    W[3] = 0.0
    qw, sw = ref.quantize(W)
    g.update(quant_w=W, quant_q=qw, quant_s=sw)
    A = r.uniform(-1, 1, (5, 9)).astype(np.float32)
    LW = r.uniform(-1, 1, (6, 9)).astype(np.float32)
    LB = r.uniform(-1, 1, 6).astype(np.float32)
    g.update(lin_a=A, lin_w=LW, lin_b=LB, lin_out=ref.linear_ref(A, LW, LB))
    ia = r.integers(-127, 128, (32, 128)).astype(np.int8)
    ia[0, 0] = 127
    iw = r.integers(-127, 128, (64, 128)).astype(np.int8)
    g.update(i8_a=ia, i8_w=iw,
             i8_out=ref.linear_vnni(ia.astype(np.float32), iw, np.ones(64, np.float32), np.zeros(64, np.float32)))
    ax = r.uniform(-3, 3, (32 * 64,)).astype(np.float32)
    u8, sc = ref.quant_act_prefix(ax)
    g.update(actq_x=ax, actq_u8=u8, actq_scale=np.float32(sc))
    vq, vs = ref.quantize(r.uniform(-0.1, 0.1, (48, 64)).astype(np.float32))
    vb = r.uniform(-1, 1, 48).astype(np.float32)
    g.update(vnni_m=np.int32(32), vnni_wq=vq, vnni_ws=vs, vnni_b=vb,
             vnni_out=ref.linear_vnni(ax.reshape(32, 64), vq, vs, vb))
    out = os.path.join(ROOT, "tests", "golden", "ref_vectors.npz")
    np.savez_compressed(out, **g)
    print(out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main()
