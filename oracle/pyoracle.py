"""ctypes wrappers of the CPU checkers: lib/liboracle.so (the C restatement)
and _ref/libesmref.so (the reference's own kernels, built by the Makefile).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "lib", "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libesmref.so")

vp, i32, sz, f32 = C.c_void_p, C.c_int, C.c_size_t, C.c_float


def _p(a: Optional[np.ndarray]):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


class _OrModel(C.Structure):
    _fields_ = [("num_layers", i32), ("hidden", i32), ("heads", i32), ("head_dim", i32), ("ffn", i32),
                ("vocab", i32), ("eps", f32), ("mask_token_id", i32), ("weights_int8", i32),
                ("act_per_token", i32), ("embed", vp), ("ln1_w", C.POINTER(vp)), ("ln1_b", C.POINTER(vp)),
                ("ln2_w", C.POINTER(vp)), ("ln2_b", C.POINTER(vp)), ("w_f32", C.POINTER(vp)),
                ("w_i8", C.POINTER(vp)), ("w_scale", C.POINTER(vp)), ("bias", C.POINTER(vp)),
                ("final_ln_w", vp), ("final_ln_b", vp), ("lm_dense_w", vp), ("lm_dense_b", vp),
                ("lm_ln_w", vp), ("lm_ln_b", vp), ("lm_decoder_bias", vp), ("fc1_fp16", i32), ("x86", i32),
                ("ffn_round24", i32)]


LINEARS = ("q", "k", "v", "out", "fc1", "fc2")


def make_or_model(weights, int8: bool, per_token: bool, fc1_fp16: bool = False, x86: bool = False,
                  ffn_bits: int = 32):
    """Builds the or_model descriptor (and keeps its arrays alive)."""
    cfg = weights.cfg
    keep = []

    def p(a):
        a = np.ascontiguousarray(a)
        keep.append(a)
        return a.ctypes.data

    L = cfg.num_layers
    arr = lambda n: (vp * max(n, 1))()
    ln1w, ln1b, ln2w, ln2b = arr(L), arr(L), arr(L), arr(L)
    wf, wi, ws, bs = arr(6 * L), arr(6 * L), arr(6 * L), arr(6 * L)
    F = weights.f32
    for i in range(L):
        ln1w[i] = p(F[f"layers.{i}.attn_ln.weight"])
        ln1b[i] = p(F[f"layers.{i}.attn_ln.bias"])
        ln2w[i] = p(F[f"layers.{i}.ffn_ln.weight"])
        ln2b[i] = p(F[f"layers.{i}.ffn_ln.bias"])
        for j, n in enumerate(LINEARS):
            bs[i * 6 + j] = p(F[f"layers.{i}.{n}.bias"])
            if int8:
                q, s = weights.i8[f"layers.{i}.{n}"]
                wi[i * 6 + j] = p(q)
                ws[i * 6 + j] = p(s)
            else:
                wf[i * 6 + j] = p(F[f"layers.{i}.{n}.weight"])
    m = _OrModel()
    m.num_layers, m.hidden, m.heads, m.head_dim = L, cfg.hidden_size, cfg.num_heads, cfg.head_dim
    m.ffn, m.vocab, m.eps, m.mask_token_id = cfg.intermediate_size, cfg.vocab_size, cfg.layer_norm_eps, \
        cfg.mask_token_id
    m.weights_int8, m.act_per_token = int(int8), int(per_token)
    m.embed = p(F["embed"])
    m.ln1_w, m.ln1_b, m.ln2_w, m.ln2_b = ln1w, ln1b, ln2w, ln2b
    m.w_f32, m.w_i8, m.w_scale, m.bias = wf, wi, ws, bs
    m.final_ln_w, m.final_ln_b = p(F["final_ln.weight"]), p(F["final_ln.bias"])
    m.lm_dense_w, m.lm_dense_b = p(F["lm_head.dense.weight"]), p(F["lm_head.dense.bias"])
    m.lm_ln_w, m.lm_ln_b = p(F["lm_head.ln.weight"]), p(F["lm_head.ln.bias"])
    m.lm_decoder_bias = p(F["lm_head.decoder.bias"])
    m.fc1_fp16 = int(fc1_fp16)
    m.x86 = int(x86)  # 0 none, 1 avx512vnni, 2 amx
    if ffn_bits not in (24, 32):
        raise ValueError("ffn_bits must be 24 or 32")
    if ffn_bits == 24 and not (int8 and per_token and not x86):
        raise ValueError("the 24-bit FFN intermediate exists only in the per-token W8A8 forward")
    m.ffn_round24 = int(ffn_bits == 24)
    keep.extend([ln1w, ln1b, ln2w, ln2b, wf, wi, ws, bs])
    return m, keep


class Oracle:
    """The C restatement (liboracle.so)."""

    def __init__(self, path: str = ORACLE_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (make -C oracle)")
        lib = C.CDLL(path)
        sig = {
            "or_gemm_i8_i32": [vp, i32, vp, i32, i32, i32, i32, vp],
            "or_quant_act_tensor": [vp, sz, vp, vp],
            "or_quant_act_rows": [vp, i32, i32, vp, vp],
            "or_dequant": [vp, vp, vp, vp, i32, i32, i32, vp],
            "or_quantize_weight": [vp, i32, i32, vp, vp],
            "or_linear_int8_w8a16": [vp, vp, vp, vp, vp, i32, i32, i32],
            "or_linear_f32": [vp, vp, vp, vp, i32, i32, i32],
            "or_layernorm": [vp, vp, vp, f32, vp, i32, i32],
            "or_gelu": [vp, vp, sz],
            "or_round_fp16": [vp, sz],
            "or_rope_tables": [i32, i32, vp, vp],
            "or_rope_varlen": [vp, vp, vp, vp, i32, i32, i32],
            "or_attention_varlen": [vp, vp, vp, vp, i32, i32, i32, vp],
            "or_forward_packed": [C.POINTER(_OrModel), vp, vp, i32, i32, vp],
            "or_forward_packed_hidden": [C.POINTER(_OrModel), vp, vp, i32, i32, vp, vp],
            "or_forward_packed_masked": [C.POINTER(_OrModel), vp, vp, vp, i32, i32, vp, vp],
            "or_round24_array": [vp, vp, sz],
            "or_x86_gelu": [vp, vp, sz],
            "or_x86_layernorm": [vp, vp, vp, f32, vp, i32, i32],
            "or_x86_rope_varlen": [vp, vp, vp, vp, i32, i32, i32],
            "or_x86_attention_varlen": [vp, vp, vp, vp, i32, i32, i32, vp],
            "or_x86_linear_f32": [vp, vp, vp, vp, i32, i32, i32],
            "or_x86_quant_act": [vp, sz, vp, vp],
            "or_expf_array": [vp, vp, sz],
        }
        for name, args in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = i32 if name.startswith("or_forward_packed") else None
        self.lib = lib

    def gemm_i8_i32(self, A, W):
        A, W = _c(A, np.int8), _c(W, np.int8)
        M, K = A.shape
        N = W.shape[0]
        out = np.empty((M, N), np.int32)
        self.lib.or_gemm_i8_i32(_p(A), K, _p(W), K, M, N, K, _p(out))
        return out

    def quant_act_tensor(self, x):
        x = _c(x, np.float32)
        q = np.empty(x.shape, np.int8)
        s = C.c_float()
        self.lib.or_quant_act_tensor(_p(x), x.size, _p(q), C.byref(s))
        return q, float(s.value)

    def quant_act_rows(self, x):
        x = _c(x, np.float32)
        M, K = x.shape
        q = np.empty((M, K), np.int8)
        s = np.empty(M, np.float32)
        self.lib.or_quant_act_rows(_p(x), M, K, _p(q), _p(s))
        return q, s

    def dequant(self, acc, a_scale, w_scale, bias, gelu=False):
        acc = _c(acc, np.int32)
        M, N = acc.shape
        out = np.empty((M, N), np.float32)
        a_scale, w_scale = _c(a_scale, np.float32), _c(w_scale, np.float32)
        bias = None if bias is None else _c(bias, np.float32)
        self.lib.or_dequant(_p(acc), _p(a_scale), _p(w_scale), _p(bias), M, N, int(gelu), _p(out))
        return out

    def quantize_weight(self, W):
        W = _c(W, np.float32)
        N, K = W.shape
        q = np.empty((N, K), np.int8)
        s = np.empty(N, np.float32)
        self.lib.or_quantize_weight(_p(W), N, K, _p(q), _p(s))
        return q, s

    def linear_int8_w8a16(self, A, q, s, bias):
        A = _c(A, np.float32)
        M, K = A.shape
        N = q.shape[0]
        out = np.empty((M, N), np.float32)
        self.lib.or_linear_int8_w8a16(_p(A), _p(_c(q, np.int8)), _p(_c(s, np.float32)),
                                      _p(None if bias is None else _c(bias, np.float32)), _p(out), M, N, K)
        return out

    def linear_f32(self, A, W, bias):
        A, W = _c(A, np.float32), _c(W, np.float32)
        M, K = A.shape
        N = W.shape[0]
        out = np.empty((M, N), np.float32)
        self.lib.or_linear_f32(_p(A), _p(W), _p(None if bias is None else _c(bias, np.float32)), _p(out), M, N, K)
        return out

    def layernorm(self, x, g, b, eps=1e-5):
        x = _c(x, np.float32)
        rows, d = x.shape
        out = np.empty_like(x)
        self.lib.or_layernorm(_p(x), _p(_c(g, np.float32)), _p(_c(b, np.float32)), eps, _p(out), rows, d)
        return out

    def round_fp16(self, x):
        out = _c(x, np.float32).copy()
        self.lib.or_round_fp16(_p(out), out.size)
        return out

    def gelu(self, x):
        x = _c(x, np.float32)
        out = np.empty_like(x)
        self.lib.or_gelu(_p(x), _p(out), x.size)
        return out

    def rope_tables(self, L, dh):
        c = np.zeros((max(L, 1), dh), np.float32)
        s = np.zeros_like(c)
        self.lib.or_rope_tables(L, dh, _p(c), _p(s))
        return c[:L], s[:L]

    def rope_varlen(self, x, cos, sin, cu, H, dh):
        x = np.array(x, np.float32, copy=True, order="C")
        cu = _c(cu, np.int32)
        self.lib.or_rope_varlen(_p(x), _p(_c(cos, np.float32)), _p(_c(sin, np.float32)), _p(cu), len(cu) - 1, H, dh)
        return x

    def attention_varlen(self, q, k, v, cu, H, dh):
        q, k, v, cu = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32), _c(cu, np.int32)
        out = np.zeros((int(cu[-1]), H * dh), np.float32)
        self.lib.or_attention_varlen(_p(q), _p(k), _p(v), _p(cu), len(cu) - 1, H, dh, _p(out))
        return out

    # The reference's x86 AVX-512 kernels (oracle_x86.c).
    def x86_gelu(self, x):
        x = _c(x, np.float32)
        out = np.empty_like(x)
        self.lib.or_x86_gelu(_p(x), _p(out), x.size)
        return out

    def x86_layernorm(self, x, g, b, eps=1e-5):
        x = _c(x, np.float32)
        rows, d = x.shape
        out = np.empty_like(x)
        self.lib.or_x86_layernorm(_p(x), _p(_c(g, np.float32)), _p(_c(b, np.float32)), eps, _p(out), rows, d)
        return out

    def x86_rope_varlen(self, x, cos, sin, cu, H, dh):
        x = np.array(x, np.float32, copy=True, order="C")
        cu = _c(cu, np.int32)
        self.lib.or_x86_rope_varlen(_p(x), _p(_c(cos, np.float32)), _p(_c(sin, np.float32)), _p(cu), len(cu) - 1,
                                    H, dh)
        return x

    def x86_attention_varlen(self, q, k, v, cu, H, dh):
        q, k, v, cu = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32), _c(cu, np.int32)
        out = np.zeros((int(cu[-1]), H * dh), np.float32)
        self.lib.or_x86_attention_varlen(_p(q), _p(k), _p(v), _p(cu), len(cu) - 1, H, dh, _p(out))
        return out

    def x86_linear_f32(self, A, W, bias):
        A, W = _c(A, np.float32), _c(W, np.float32)
        M, K = A.shape
        N = W.shape[0]
        out = np.empty((M, N), np.float32)
        self.lib.or_x86_linear_f32(_p(A), _p(W), _p(None if bias is None else _c(bias, np.float32)), _p(out), M, N,
                                   K)
        return out

    def expf(self, x):
        """glibc expf of every element (the reference's std::exp)."""
        x = _c(x, np.float32)
        out = np.empty_like(x)
        self.lib.or_expf_array(_p(x), _p(out), x.size)
        return out

    def x86_quant_act(self, x):
        x = _c(x, np.float32)
        q = np.empty(x.shape, np.int8)
        s = C.c_float()
        self.lib.or_x86_quant_act(_p(x), x.size, _p(q), C.byref(s))
        return q, float(s.value)

    def round24(self, x):
        """or_round24 of every element (the 24-bit FFN intermediate)."""
        x = _c(x, np.float32)
        out = np.empty_like(x)
        self.lib.or_round24_array(_p(x), _p(out), x.size)
        return out

    def forward_packed(self, weights, batch, int8: bool, per_token: bool, fc1_fp16: bool = False,
                       x86=False, ffn_bits: int = 32, hidden: bool = False, masks=None):
        """Restated packed forward. x86=True (or "avx512vnni") runs the
        reference's x86 AVX-512 kernels, per-tensor scales and LinearVnni in
        W8A8; x86="amx" the same with LinearAmx's row split. ffn_bits=24
        rounds fc1's output to 24 bits (per-token W8A8, the GPU's default).
        hidden=True also returns the hidden states [N + 1, T, d]
        (ForwardWithHiddenStates' layout). masks: BatchView's packed_masks
        (int32 [T], 0 = pad) or None."""
        if x86 and int8 and per_token:
            raise ValueError("the x86 path quantises activations per tensor")
        m, keep = make_or_model(weights, int8, per_token, fc1_fp16, 2 if x86 == "amx" else int(bool(x86)),
                                ffn_bits)
        T = batch.total_tokens
        cfg = weights.cfg
        logits = np.empty((T, cfg.vocab_size), np.float32)
        hs = np.empty((cfg.num_layers + 1, T, cfg.hidden_size), np.float32) if hidden else None
        mk = None if masks is None else _c(masks, np.int32)
        if mk is not None and mk.shape != (T,):
            raise ValueError("masks must have one entry per token")
        rc = self.lib.or_forward_packed_masked(C.byref(m), _p(_c(batch.ids, np.int32)), _p(mk),
                                               _p(_c(batch.cu, np.int32)), len(batch.cu) - 1, T, _p(logits),
                                               _p(hs))
        if rc != 0:
            raise MemoryError("or_forward_packed")
        return (logits, hs) if hidden else logits


class RefLib:
    """The reference's own kernels (oracle/_ref/libesmref.so)."""

    def __init__(self, path: str = REF_LIB, threads: Optional[int] = None):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (make -C oracle ref)")
        if threads is not None:
            os.environ["ESM_NUM_THREADS"] = str(threads)
        lib = C.CDLL(path)
        sig = {
            "esmref_isa": (C.c_char_p, []),
            "esmref_host_isa": (C.c_char_p, []),
            "esmref_quantize": (None, [vp, i32, i32, vp, vp]),
            "esmref_linear_int8": (None, [vp, vp, vp, vp, vp, i32, i32, i32]),
            "esmref_linear_int8_ref": (None, [vp, vp, vp, vp, vp, i32, i32, i32]),
            "esmref_has_avx512_prefix": (i32, []),
            "esmref_quant_act_prefix": (None, [vp, sz, vp, vp]),
            "esmref_linear_vnni": (None, [vp, vp, vp, vp, vp, i32, i32, i32]),
            "esmref_linear": (None, [vp, vp, vp, vp, i32, i32, i32]),
            "esmref_linear_ref": (None, [vp, vp, vp, vp, i32, i32, i32]),
            "esmref_layernorm_ref": (None, [vp, vp, vp, f32, vp, i32, i32]),
            "esmref_layernorm": (None, [vp, vp, vp, f32, vp, i32, i32]),
            "esmref_gelu_ref": (None, [vp, vp, sz]),
            "esmref_gelu": (None, [vp, vp, sz]),
            "esmref_rope_tables": (None, [i32, i32, vp, vp]),
            "esmref_rope_varlen_ref": (None, [vp, vp, vp, vp, i32, i32, i32]),
            "esmref_rope_varlen": (None, [vp, vp, vp, vp, i32, i32, i32]),
            "esmref_attention_varlen_ref": (None, [vp, vp, vp, vp, i32, i32, i32, vp]),
            "esmref_attention_varlen": (None, [vp, vp, vp, vp, i32, i32, i32, vp]),
            "esmref_model_create": (vp, [C.POINTER(_OrModel)]),
            "esmref_model_free": (None, [vp]),
            "esmref_forward_packed": (i32, [vp, vp, vp, i32, i32, vp]),
            "esmref_forward_packed_observed": (i32, [vp, vp, vp, i32, i32, vp, vp]),
            "esmref_observer_new": (vp, []),
            "esmref_observer_free": (None, [vp]),
            "esmref_observer_clear": (None, [vp]),
            "esmref_observer_observe": (None, [vp, C.c_char_p, vp, sz]),
            "esmref_observer_percentile": (i32, [vp, C.c_char_p, f32, C.POINTER(f32)]),
            "esmref_observer_site_count": (i32, [vp]),
            "esmref_plan_batches": (i32, [vp, i32, f32, i32, vp, vp, C.POINTER(C.c_int)]),
            "esmref_gguf_save_model": (i32, [vp, C.c_char_p]),
            "esmref_gguf_tensor": (i32, [C.c_char_p, C.c_char_p, vp, sz, C.POINTER(C.c_uint32),
                                         C.POINTER(C.c_uint64), C.POINTER(C.c_uint32), C.POINTER(sz)]),
            "esmref_gguf_meta": (i32, [C.c_char_p, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int64),
                                       C.POINTER(C.c_double)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        self.lib = lib

    def isa(self) -> str:
        return self.lib.esmref_isa().decode()

    def observer(self) -> "RefObserver":
        return RefObserver(self)

    def gguf_tensor(self, path: str, name: str, cap: int = 1 << 30):
        """(type, dims, raw bytes) of one tensor through the reference's GGUF
        reader, None when absent; raises when the reader rejects the file."""
        buf = np.zeros(0, np.uint8)
        t, nd, nbytes = C.c_uint32(), C.c_uint32(), C.c_size_t()
        shape = (C.c_uint64 * 8)()
        rc = self.lib.esmref_gguf_tensor(os.fsencode(path), name.encode(), None, 0, C.byref(t), shape, C.byref(nd),
                                         C.byref(nbytes))
        if rc == 1:
            return None
        if rc != 0:
            raise ValueError(f"reference GGUF reader rejected {path}")
        buf = np.zeros(min(nbytes.value, cap), np.uint8)
        self.lib.esmref_gguf_tensor(os.fsencode(path), name.encode(), _p(buf), buf.size, C.byref(t), shape,
                                    C.byref(nd), C.byref(nbytes))
        return int(t.value), tuple(int(shape[i]) for i in range(nd.value)), buf.tobytes()

    def gguf_meta(self, path: str, key: str):
        """A metadata value through the reference's reader: int, float, bool,
        ("str", length), or None when absent."""
        kind, iv, fv = C.c_int(), C.c_int64(), C.c_double()
        if self.lib.esmref_gguf_meta(os.fsencode(path), key.encode(), C.byref(kind), C.byref(iv), C.byref(fv)) != 0:
            raise ValueError(f"reference GGUF reader rejected {path}")
        return {0: None, 1: iv.value, 2: fv.value, 3: bool(iv.value), 4: ("str", iv.value)}[kind.value]

    def plan_batches(self, lengths, max_batch_size: int = 256, imbalance_threshold: float = 1.2):
        """The reference's PlanBatches (src/sched/scheduler.cpp:54-75) as a list of groups."""
        lens = _c(lengths, np.int32)
        n = int(lens.shape[0])
        order = np.zeros(max(n, 1), np.int32)
        sizes = np.zeros(max(n, 1), np.int32)
        ng = C.c_int(0)
        self.lib.esmref_plan_batches(_p(lens), n, float(imbalance_threshold), int(max_batch_size), _p(order),
                                     _p(sizes), C.byref(ng))
        out, k = [], 0
        for g in range(ng.value):
            out.append([int(i) for i in order[k:k + sizes[g]]])
            k += int(sizes[g])
        return out

    def host_isa(self) -> str:
        return self.lib.esmref_host_isa().decode()

    def quantize(self, W):
        W = _c(W, np.float32)
        N, K = W.shape
        q = np.empty((N, K), np.int8)
        s = np.empty(N, np.float32)
        self.lib.esmref_quantize(_p(W), N, K, _p(q), _p(s))
        return q, s

    def _lin8(self, fn, A, q, s, bias):
        A = _c(A, np.float32)
        M, K = A.shape
        N = q.shape[0]
        out = np.empty((M, N), np.float32)
        fn(_p(A), _p(_c(q, np.int8)), _p(_c(s, np.float32)), _p(None if bias is None else _c(bias, np.float32)),
           _p(out), M, N, K)
        return out

    def linear_int8(self, A, q, s, bias):
        return self._lin8(self.lib.esmref_linear_int8, A, q, s, bias)

    def linear_int8_ref(self, A, q, s, bias):
        return self._lin8(self.lib.esmref_linear_int8_ref, A, q, s, bias)

    def linear_vnni(self, A, q, s, bias):
        return self._lin8(self.lib.esmref_linear_vnni, A, q, s, bias)

    def quant_act_prefix(self, A):
        A = _c(A, np.float32)
        q = np.empty(A.shape, np.uint8)
        s = C.c_float()
        self.lib.esmref_quant_act_prefix(_p(A), A.size, _p(q), C.byref(s))
        return q, float(s.value)

    def linear_ref(self, A, W, bias):
        A, W = _c(A, np.float32), _c(W, np.float32)
        M, K = A.shape
        N = W.shape[0]
        out = np.empty((M, N), np.float32)
        self.lib.esmref_linear_ref(_p(A), _p(W), _p(None if bias is None else _c(bias, np.float32)), _p(out), M, N, K)
        return out

    def layernorm_ref(self, x, g, b, eps=1e-5):
        x = _c(x, np.float32)
        out = np.empty_like(x)
        self.lib.esmref_layernorm_ref(_p(x), _p(_c(g, np.float32)), _p(_c(b, np.float32)), eps, _p(out), *x.shape)
        return out

    def gelu_ref(self, x):
        x = _c(x, np.float32)
        out = np.empty_like(x)
        self.lib.esmref_gelu_ref(_p(x), _p(out), x.size)
        return out

    def rope_tables(self, L, dh):
        c = np.zeros((max(L, 1), dh), np.float32)
        s = np.zeros_like(c)
        self.lib.esmref_rope_tables(L, dh, _p(c), _p(s))
        return c[:L], s[:L]

    def rope_varlen_ref(self, x, cos, sin, cu, H, dh):
        x = np.array(x, np.float32, copy=True, order="C")
        cu = _c(cu, np.int32)
        self.lib.esmref_rope_varlen_ref(_p(x), _p(_c(cos, np.float32)), _p(_c(sin, np.float32)), _p(cu),
                                        len(cu) - 1, H, dh)
        return x

    def rope_varlen(self, x, cos, sin, cu, H, dh):
        """The facade's RopeApplyVarlen (the current ISA's kernel)."""
        x = np.array(x, np.float32, copy=True, order="C")
        cu = _c(cu, np.int32)
        self.lib.esmref_rope_varlen(_p(x), _p(_c(cos, np.float32)), _p(_c(sin, np.float32)), _p(cu), len(cu) - 1,
                                    H, dh)
        return x

    def layernorm(self, x, g, b, eps=1e-5):
        """The facade's LayerNorm (the current ISA's kernel)."""
        x = _c(x, np.float32)
        out = np.empty_like(x)
        self.lib.esmref_layernorm(_p(x), _p(_c(g, np.float32)), _p(_c(b, np.float32)), eps, _p(out), *x.shape)
        return out

    def gelu(self, x):
        """The facade's Gelu (the current ISA's kernel)."""
        x = _c(x, np.float32)
        out = np.empty_like(x)
        self.lib.esmref_gelu(_p(x), _p(out), x.size)
        return out

    def linear(self, A, W, bias):
        """The facade's FP32 Linear (the current ISA's kernel)."""
        A, W = _c(A, np.float32), _c(W, np.float32)
        M, K = A.shape
        N = W.shape[0]
        out = np.empty((M, N), np.float32)
        self.lib.esmref_linear(_p(A), _p(W), _p(None if bias is None else _c(bias, np.float32)), _p(out), M, N, K)
        return out

    def attention_varlen_ref(self, q, k, v, cu, H, dh):
        q, k, v, cu = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32), _c(cu, np.int32)
        out = np.zeros((int(cu[-1]), H * dh), np.float32)
        self.lib.esmref_attention_varlen_ref(_p(q), _p(k), _p(v), _p(cu), len(cu) - 1, H, dh, _p(out))
        return out

    def attention_varlen(self, q, k, v, cu, H, dh):
        q, k, v, cu = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32), _c(cu, np.int32)
        out = np.zeros((int(cu[-1]), H * dh), np.float32)
        self.lib.esmref_attention_varlen(_p(q), _p(k), _p(v), _p(cu), len(cu) - 1, H, dh, _p(out))
        return out


class RefModel:
    """Reference CPU forward (reference kernels, restated ForwardPackedInto)."""

    def __init__(self, ref: RefLib, weights, int8: bool, fc1_fp16: bool = False):
        m, keep = make_or_model(weights, int8, per_token=False, fc1_fp16=fc1_fp16)
        self.ref, self.cfg = ref, weights.cfg
        self.handle = ref.lib.esmref_model_create(C.byref(m))

    def save_gguf(self, path: str):
        """Model::SaveToGguf's tensors and metadata through the reference's writer."""
        if self.ref.lib.esmref_gguf_save_model(self.handle, os.fsencode(path)) != 0:
            raise ValueError("reference GGUF writer failed")

    def forward_packed(self, batch, observer: Optional["RefObserver"] = None):
        """Logits [T, vocab]; with an observer, also feeds the reference's
        ActivationObserver at TransformerBlock's four sites."""
        T = batch.total_tokens
        logits = np.empty((T, self.cfg.vocab_size), np.float32)
        self.ref.lib.esmref_forward_packed_observed(self.handle, _p(_c(batch.ids, np.int32)),
                                                    _p(_c(batch.cu, np.int32)), len(batch.cu) - 1, T, _p(logits),
                                                    observer.handle if observer is not None else None)
        return logits

    def free(self):
        if self.handle:
            self.ref.lib.esmref_model_free(self.handle)
            self.handle = None


class RefObserver:
    """The reference's esm::ActivationObserver (oracle/_ref)."""

    def __init__(self, ref: RefLib):
        self.ref = ref
        self.handle = ref.lib.esmref_observer_new()
        self.keys = set()

    def observe(self, site: str, values):
        v = _c(np.asarray(values, np.float32).ravel(), np.float32)
        self.ref.lib.esmref_observer_observe(self.handle, site.encode(), _p(v), v.size)
        if v.size:
            self.keys.add(site)

    def percentile(self, pctile: float, sites=None):
        """{site: value} for the given sites (default: every site observed
        through observe()); sites the reference does not hold are left out."""
        out = {}
        v = C.c_float()
        for key in (self.keys if sites is None else sites):
            if self.ref.lib.esmref_observer_percentile(self.handle, key.encode(), float(pctile), C.byref(v)):
                out[key] = v.value
        return out

    def site_count(self) -> int:
        return int(self.ref.lib.esmref_observer_site_count(self.handle))

    def clear(self):
        self.ref.lib.esmref_observer_clear(self.handle)
        self.keys.clear()

    def free(self):
        if self.handle:
            self.ref.lib.esmref_observer_free(self.handle)
            self.handle = None
