"""Writes tests/golden/full_depth_650m.npz: 33-layer ESM-2-650M W8A8 logits
of one fixed config-4 batch through every reference CPU path and the oracle.

Run from the repository root after `make -C oracle` (needs oracle/_ref,
i.e. /root/reference at build time, and a host with AVX-512-VNNI; the AMX
leg needs AMX-INT8):

    python tests/golden/make_full_depth.py

Batch: sequences 4..7 of the config-4 varlen batch (synthetic.config4_varlen_batch),
446 tokens, so 446 % 32 = 30 rows take LinearAmx's separately quantised tail.
Weights: synthetic.make_weights(ESM2_650M, seed 20261201 + 4, int8=True).

Arrays (fp32 logits [T, 33] unless noted):
  ids, cu                 the batch (int32)
  ref_avx512vnni          the reference's kernels, ESM_FORCE_ISA=avx512vnni
  ref_amx                 the same, ESM_FORCE_ISA=amx (absent without AMX)
  ref_isa_ref             the same, ESM_FORCE_ISA=ref (the scalar *Ref kernels,
                          W8A16 LinearInt8Ref: several minutes)
  oracle_per_tensor       oracle.c's W8A8 forward (Ref-order kernels, per-tensor scales)
  oracle_per_token        oracle.c's W8A8 forward, per-token scales
  oracle_per_token_ffn24  the same with fc1's output rounded to 24 bits
                          (the GPU's default per-token FFN intermediate)
Arrays already in an existing file are kept; only missing ones are computed.
The reference's forward is oracle/ref_shim.cpp's ForwardPackedInto sequence
over the reference's compiled kernels (oracle/_ref/libesmref.so).
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "esm-cpp_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

OUT = os.path.join(HERE, "full_depth_650m.npz")
SEQS = [4, 5, 6, 7]


def batch():
    from esm_gfx950 import synthetic as syn
    return syn.config4_varlen_batch().subset(SEQS)


def weights():
    from esm_gfx950 import synthetic as syn
    return syn.make_weights(syn.ESM2_650M, seed=20261201 + 4, int8=True)


def main():
    from pyoracle import Oracle, RefLib, RefModel
    b = batch()
    w = weights()
    out = {"ids": b.ids, "cu": b.cu}
    if os.path.exists(OUT):
        with np.load(OUT, allow_pickle=False) as z:
            assert np.array_equal(z["ids"], b.ids) and np.array_equal(z["cu"], b.cu)
            out.update({k: z[k] for k in z.files})
    ref = RefLib(threads=os.cpu_count() or 8)
    isas = ["avx512vnni", "ref"] + (["amx"] if ref.host_isa() == "amx" else [])
    todo = [isa for isa in isas if f"ref_{'isa_ref' if isa == 'ref' else isa}" not in out]
    if todo:
        rm = RefModel(ref, w, int8=True)
        for isa in todo:
            os.environ["ESM_FORCE_ISA"] = isa
            t = time.time()
            out[f"ref_{'isa_ref' if isa == 'ref' else isa}"] = rm.forward_packed(b)
            print(f"reference {isa}: {time.time() - t:.1f}s", flush=True)
        os.environ.pop("ESM_FORCE_ISA", None)
        rm.free()
    o = Oracle()
    if "oracle_per_tensor" not in out:
        out["oracle_per_tensor"] = o.forward_packed(w, b, int8=True, per_token=False)
    if "oracle_per_token" not in out:
        out["oracle_per_token"] = o.forward_packed(w, b, int8=True, per_token=True)
    if "oracle_per_token_ffn24" not in out:
        out["oracle_per_token_ffn24"] = o.forward_packed(w, b, int8=True, per_token=True, ffn_bits=24)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: T={b.total_tokens}")


if __name__ == "__main__":
    main()
