"""ctypes binding of the gfx950 C ABI (include/esm_gfx950.h).

The binding holds no compute: every array operation is a call into
libesm_gfx950.so. Loading fails loudly when the library is missing; there
is no CPU fallback. Device memory comes from the library itself
(esm_gfx950_malloc), so the process carries a single HIP runtime.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libesm_gfx950.so")

OK = 0
# esm::StatusCode values (status codes of include/esm_gfx950.h)
INVALID_ARGUMENT, OUT_OF_RANGE, NOT_FOUND, IO_ERROR, SHAPE_MISMATCH, INTERNAL, HIP_ERROR = 1, 2, 3, 4, 5, 6, 7
ACT_PER_TENSOR = 0
ACT_PER_TOKEN = 1
ATTN_FP32 = 0
ATTN_BF16_MFMA = 1
ATTN_F16X3_MFMA = 2
ATTN_MODE_FP16 = 0
ATTN_MODE_BF16 = 1
ATTN_MODE_FP32 = 2
ATTN_MODE_F16X3 = 3
NUMERICS_DEFAULT = 0
NUMERICS_X86_AVX512 = 1
NUMERICS_X86_AMX = 2

# Every symbol the header declares (checked by the CPU test suite).
EXPORTED = [
    "esm_gfx950_init", "esm_gfx950_destroy", "esm_gfx950_last_error", "esm_gfx950_device_arch",
    "esm_gfx950_sync", "esm_gfx950_malloc", "esm_gfx950_free", "esm_gfx950_memcpy_h2d",
    "esm_gfx950_memcpy_d2h", "esm_gfx950_memcpy_d2d", "esm_gfx950_timer_start", "esm_gfx950_timer_stop",
    "esm_gfx950_kernel_timing", "esm_gfx950_kernel_timing_query", "esm_gfx950_weight_upload_i8",
    "esm_gfx950_weight_free", "esm_gfx950_gemm_i8_i32", "esm_gfx950_linear_i8_q", "esm_gfx950_quantize_act",
    "esm_gfx950_gelu_quantize_act", "esm_gfx950_set_gemm_tile_rows", "esm_gfx950_set_gemm_split_k", "esm_gfx950_model_set_lm_dense_split",
    "esm_gfx950_linear_i8", "esm_gfx950_linear_f32", "esm_gfx950_layernorm", "esm_gfx950_gelu",
    "esm_gfx950_residual_add", "esm_gfx950_scale", "esm_gfx950_rope_build_tables",
    "esm_gfx950_rope_apply_varlen", "esm_gfx950_attention_varlen", "esm_gfx950_attention_varlen_bf16",
    "esm_gfx950_model_create", "esm_gfx950_model_free", "esm_gfx950_model_set_act_mode",
    "esm_gfx950_forward_packed", "esm_gfx950_batch_upload", "esm_gfx950_forward_device",
    "esm_gfx950_model_arena_bytes", "esm_gfx950_model_set_parts", "esm_gfx950_model_staged_parts",
    "esm_gfx950_plan_batches",
    "esm_gfx950_forward_scheduled", "esm_gfx950_model_create_from_gguf",
    "esm_gfx950_model_set_first_block_fc1_fp16", "esm_gfx950_observer_create", "esm_gfx950_observer_free",
    "esm_gfx950_observer_clear", "esm_gfx950_observer_observe", "esm_gfx950_observer_site_count",
    "esm_gfx950_observer_site_name", "esm_gfx950_observer_percentile", "esm_gfx950_forward_with_observer",
    "esm_gfx950_attention_work_items", "esm_gfx950_layernorm_avx512", "esm_gfx950_gelu_avx512",
    "esm_gfx950_expf_glibc", "esm_gfx950_linear_f32_avx512", "esm_gfx950_rope_apply_varlen_avx512",
    "esm_gfx950_attention_varlen_avx512", "esm_gfx950_model_set_numerics", "esm_gfx950_linear_i8_noalloc",
    "esm_gfx950_model_set_ffn_intermediate_bits", "esm_gfx950_linear_i8_gelu_quant_r24",
    "esm_gfx950_forward_hidden_states", "esm_gfx950_forward_packed_masked", "esm_gfx950_batch_upload_masked",
    "esm_gfx950_model_get_config",
]


class Gfx950Error(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"esm_gfx950 error {code}: {msg}")
        self.code = code


_lib: Optional[C.CDLL] = None


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Loads libesm_gfx950.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} not built (run python esm-cpp_amd/build.py)")
    lib = C.CDLL(path)
    vp, i32, sz, f32 = C.c_void_p, C.c_int, C.c_size_t, C.c_float
    sig = {
        "esm_gfx950_init": (i32, [i32, C.POINTER(vp)]),
        "esm_gfx950_destroy": (i32, [vp]),
        "esm_gfx950_last_error": (C.c_char_p, [vp]),
        "esm_gfx950_device_arch": (C.c_char_p, [vp]),
        "esm_gfx950_sync": (i32, [vp]),
        "esm_gfx950_malloc": (i32, [vp, sz, C.POINTER(vp)]),
        "esm_gfx950_free": (i32, [vp, vp]),
        "esm_gfx950_memcpy_h2d": (i32, [vp, vp, vp, sz]),
        "esm_gfx950_memcpy_d2h": (i32, [vp, vp, vp, sz]),
        "esm_gfx950_memcpy_d2d": (i32, [vp, vp, vp, sz]),
        "esm_gfx950_timer_start": (i32, [vp]),
        "esm_gfx950_timer_stop": (i32, [vp, C.POINTER(f32)]),
        "esm_gfx950_kernel_timing": (i32, [vp, i32]),
        "esm_gfx950_kernel_timing_query": (i32, [vp, C.c_char_p, C.POINTER(i32), C.POINTER(C.c_double)]),
        "esm_gfx950_weight_upload_i8": (i32, [vp, vp, vp, i32, i32, C.POINTER(vp)]),
        "esm_gfx950_weight_free": (i32, [vp, vp]),
        "esm_gfx950_gemm_i8_i32": (i32, [vp, vp, i32, vp, i32, vp]),
        "esm_gfx950_linear_i8_q": (i32, [vp, vp, i32, vp, vp, vp, vp, i32, i32]),
        "esm_gfx950_quantize_act": (i32, [vp, vp, i32, i32, i32, vp, i32, vp]),
        "esm_gfx950_gelu_quantize_act": (i32, [vp, vp, i32, i32, vp, i32, vp]),
        "esm_gfx950_linear_i8_gelu_quant_r24": (i32, [vp, vp, i32, vp, vp, vp, i32, vp, vp, vp, i32, vp]),
        "esm_gfx950_forward_hidden_states": (i32, [vp, vp, vp, vp, vp, i32, i32, vp, vp]),
        "esm_gfx950_forward_packed_masked": (i32, [vp, vp, vp, vp, vp, i32, i32, vp, i32]),
        "esm_gfx950_batch_upload_masked": (i32, [vp, vp, vp, vp, vp, i32, i32]),
        "esm_gfx950_set_gemm_tile_rows": (i32, [i32]),
        "esm_gfx950_set_gemm_split_k": (i32, [i32]),
        "esm_gfx950_model_set_lm_dense_split": (i32, [vp, vp, i32]),
        "esm_gfx950_linear_i8": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32]),
        "esm_gfx950_linear_i8_noalloc": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32]),
        "esm_gfx950_linear_f32": (i32, [vp, vp, vp, vp, vp, i32, i32, i32]),
        "esm_gfx950_layernorm": (i32, [vp, vp, vp, vp, f32, vp, i32, i32]),
        "esm_gfx950_gelu": (i32, [vp, vp, vp, sz]),
        "esm_gfx950_residual_add": (i32, [vp, vp, vp, sz]),
        "esm_gfx950_scale": (i32, [vp, vp, sz, f32]),
        "esm_gfx950_rope_build_tables": (i32, [i32, i32, vp, vp]),
        "esm_gfx950_rope_apply_varlen": (i32, [vp, vp, vp, vp, vp, i32, i32, i32]),
        "esm_gfx950_attention_work_items": (i32, [vp, i32, i32, i32, C.POINTER(sz), C.POINTER(sz)]),
        "esm_gfx950_layernorm_avx512": (i32, [vp, vp, vp, vp, f32, vp, i32, i32]),
        "esm_gfx950_gelu_avx512": (i32, [vp, vp, vp, sz]),
        "esm_gfx950_expf_glibc": (i32, [vp, vp, vp, sz]),
        "esm_gfx950_linear_f32_avx512": (i32, [vp, vp, vp, vp, vp, i32, i32, i32]),
        "esm_gfx950_rope_apply_varlen_avx512": (i32, [vp, vp, vp, vp, vp, i32, i32, i32]),
        "esm_gfx950_attention_varlen_avx512": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, vp]),
        "esm_gfx950_model_set_numerics": (i32, [vp, vp, i32]),
        "esm_gfx950_attention_varlen": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, vp, i32]),
        "esm_gfx950_attention_varlen_bf16": (i32, [vp, vp, vp, vp, i32, vp, i32, i32, vp]),
        "esm_gfx950_model_create": (i32, [vp, vp, C.POINTER(vp)]),
        "esm_gfx950_model_free": (i32, [vp, vp]),
        "esm_gfx950_model_set_act_mode": (i32, [vp, vp, i32]),
        "esm_gfx950_forward_packed": (i32, [vp, vp, vp, vp, i32, i32, vp, i32]),
        "esm_gfx950_batch_upload": (i32, [vp, vp, vp, vp, i32, i32]),
        "esm_gfx950_forward_device": (i32, [vp, vp, vp]),
        "esm_gfx950_model_arena_bytes": (i32, [vp, C.POINTER(sz)]),
        "esm_gfx950_model_set_parts": (i32, [vp, vp, i32]),
        "esm_gfx950_model_staged_parts": (i32, [vp, C.POINTER(C.c_int)]),
        "esm_gfx950_plan_batches": (i32, [vp, i32, f32, i32, vp, vp, C.POINTER(C.c_int)]),
        "esm_gfx950_forward_scheduled": (i32, [vp, vp, vp, vp, i32, f32, i32, vp]),
        "esm_gfx950_model_create_from_gguf": (i32, [vp, C.c_char_p, i32, i32, C.POINTER(vp)]),
        "esm_gfx950_model_set_first_block_fc1_fp16": (i32, [vp, vp, i32]),
        "esm_gfx950_model_set_ffn_intermediate_bits": (i32, [vp, vp, i32]),
        "esm_gfx950_observer_create": (i32, [vp, C.POINTER(vp)]),
        "esm_gfx950_observer_free": (i32, [vp, vp]),
        "esm_gfx950_observer_clear": (i32, [vp]),
        "esm_gfx950_observer_observe": (i32, [vp, vp, C.c_char_p, vp, sz]),
        "esm_gfx950_observer_site_count": (i32, [vp, C.POINTER(sz)]),
        "esm_gfx950_observer_site_name": (i32, [vp, sz, C.POINTER(C.c_char_p)]),
        "esm_gfx950_observer_percentile": (i32, [vp, C.c_char_p, f32, C.POINTER(f32)]),
        "esm_gfx950_forward_with_observer": (i32, [vp, vp, vp, vp, i32, i32, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _ptr(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data)


def set_gemm_tile_rows(rows: int):
    """INT8 GEMM tile height for later launches: 64, 128, 256, 320 or 0 (automatic)."""
    rc = load_library().esm_gfx950_set_gemm_tile_rows(int(rows))
    if rc != OK:
        raise Gfx950Error(rc, f"set_gemm_tile_rows({rows})")


def set_gemm_split_k(splits: int):
    """K splits of the model's out-proj / fc2 GEMMs for later launches: 0
    automatic, 1 never, 2..4 forced."""
    rc = load_library().esm_gfx950_set_gemm_split_k(int(splits))
    if rc != OK:
        raise Gfx950Error(rc, f"set_gemm_split_k({splits})")


def rope_build_tables(seq_len: int, head_dim: int):
    """RopeBuildTables on the host (reference formula)."""
    lib = load_library()
    cos = np.zeros((max(seq_len, 1), head_dim), np.float32)
    sin = np.zeros_like(cos)
    rc = lib.esm_gfx950_rope_build_tables(seq_len, head_dim, _ptr(cos), _ptr(sin))
    if rc != OK:
        raise Gfx950Error(rc, "rope_build_tables")
    return cos[:seq_len], sin[:seq_len]


def attention_work_items(cu: np.ndarray, num_heads: int, mfma: bool = True):
    """(items, capacity): the attention work items a batch produces and the
    number the model's per-batch metadata reserves (host only)."""
    lib = load_library()
    cu = np.ascontiguousarray(cu, np.int32)
    items, cap = C.c_size_t(), C.c_size_t()
    rc = lib.esm_gfx950_attention_work_items(_ptr(cu), int(cu.size - 1), int(num_heads), int(mfma), C.byref(items),
                                             C.byref(cap))
    if rc:
        raise Gfx950Error(rc, "attention_work_items: invalid arguments")
    return int(items.value), int(cap.value)


def plan_batches(lengths, max_batch_size: int = 256, imbalance_threshold: float = 1.2):
    """PlanBatches on the host: list of groups of caller indices
    (reference src/sched/scheduler.cpp:54-75, defaults of scheduler.h:8-21)."""
    lib = load_library()
    lens = np.ascontiguousarray(lengths, np.int32)
    n = int(lens.shape[0])
    order = np.zeros(max(n, 1), np.int32)
    sizes = np.zeros(max(n, 1), np.int32)
    ng = C.c_int(0)
    rc = lib.esm_gfx950_plan_batches(_ptr(lens), n, float(imbalance_threshold), int(max_batch_size), _ptr(order),
                                     _ptr(sizes), C.byref(ng))
    if rc != OK:
        raise Gfx950Error(rc, "plan_batches")
    out, k = [], 0
    for g in range(ng.value):
        out.append([int(i) for i in order[k:k + sizes[g]]])
        k += int(sizes[g])
    return out


class DeviceArray:
    """A device allocation with a numpy dtype and shape."""

    def __init__(self, dev: "Device", shape, dtype):
        self.dev = dev
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        dev._check(dev.lib.esm_gfx950_malloc(dev.ctx, max(self.nbytes, 1), C.byref(p)))
        self.ptr = p

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            self.dev._check(self.dev.lib.esm_gfx950_memcpy_d2h(self.dev.ctx, _ptr(out), self.ptr, self.nbytes))
        return out

    def upload(self, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        if self.nbytes:
            self.dev._check(self.dev.lib.esm_gfx950_memcpy_h2d(self.dev.ctx, self.ptr, _ptr(a), self.nbytes))
        return self

    def free(self):
        if self.ptr:
            self.dev.lib.esm_gfx950_free(self.dev.ctx, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and self.dev.ctx:
                self.free()
        except Exception:
            pass


class Weight:
    def __init__(self, dev: "Device", packed: np.ndarray, scales: np.ndarray):
        packed = np.ascontiguousarray(packed, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        N, K = packed.shape
        h = C.c_void_p()
        dev._check(dev.lib.esm_gfx950_weight_upload_i8(dev.ctx, _ptr(packed), _ptr(scales), N, K, C.byref(h)))
        self.dev, self.handle, self.N, self.K = dev, h, N, K

    def free(self):
        if self.handle:
            self.dev.lib.esm_gfx950_weight_free(self.dev.ctx, self.handle)
            self.handle = None


class Device:
    """One gfx950 context (one HIP stream)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        ctx = C.c_void_p()
        rc = self.lib.esm_gfx950_init(device, C.byref(ctx))
        if rc != OK:
            raise Gfx950Error(rc, "esm_gfx950_init failed (no gfx950 device?)")
        self.ctx = ctx
        self.arch = self.lib.esm_gfx950_device_arch(ctx).decode()

    def _check(self, rc: int):
        if rc != OK:
            raise Gfx950Error(rc, self.lib.esm_gfx950_last_error(self.ctx).decode())

    def close(self):
        if self.ctx:
            self.lib.esm_gfx950_destroy(self.ctx)
            self.ctx = None

    # -------------------------------------------------------------- memory
    def empty(self, shape, dtype) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def array(self, a: np.ndarray, dtype=None) -> DeviceArray:
        a = np.ascontiguousarray(a, dtype=dtype)
        return DeviceArray(self, a.shape, a.dtype).upload(a)

    def sync(self):
        self._check(self.lib.esm_gfx950_sync(self.ctx))

    def timer_start(self):
        self._check(self.lib.esm_gfx950_timer_start(self.ctx))

    def timer_stop(self) -> float:
        ms = C.c_float()
        self._check(self.lib.esm_gfx950_timer_stop(self.ctx, C.byref(ms)))
        return float(ms.value)

    def kernel_timing(self, enable: bool = True):
        self._check(self.lib.esm_gfx950_kernel_timing(self.ctx, int(enable)))

    def kernel_timing_query(self, site: str):
        """(launches, total_ms) of the timed launches of `site` since enabling."""
        n, ms = C.c_int(), C.c_double()
        self._check(self.lib.esm_gfx950_kernel_timing_query(self.ctx, site.encode(), C.byref(n), C.byref(ms)))
        return int(n.value), float(ms.value)

    # ------------------------------------------------------------------ ops
    def weight_i8(self, packed: np.ndarray, scales: np.ndarray) -> Weight:
        return Weight(self, packed, scales)

    def gemm_i8_i32(self, A: DeviceArray, lda: int, W: Weight, M: int, C_out: DeviceArray):
        self._check(self.lib.esm_gfx950_gemm_i8_i32(self.ctx, A.ptr, lda, W.handle, M, C_out.ptr))

    def linear_i8_q(self, A: DeviceArray, lda: int, a_scale: DeviceArray, W: Weight, bias: Optional[DeviceArray],
                    C_out: DeviceArray, M: int, gelu: bool = False):
        self._check(self.lib.esm_gfx950_linear_i8_q(self.ctx, A.ptr, lda, a_scale.ptr, W.handle,
                                                    bias.ptr if bias is not None else None, C_out.ptr, M, int(gelu)))

    def quantize_act(self, x: DeviceArray, M: int, K: int, mode: int, q: DeviceArray, ldq: int, scales: DeviceArray):
        self._check(self.lib.esm_gfx950_quantize_act(self.ctx, x.ptr, M, K, mode, q.ptr, ldq, scales.ptr))

    def gelu_quantize_act(self, x: DeviceArray, M: int, K: int, q: DeviceArray, ldq: int, scales: DeviceArray):
        """GELU then per-token int8 quantisation, fused (fc2's input in the INT8 FFN)."""
        self._check(self.lib.esm_gfx950_gelu_quantize_act(self.ctx, x.ptr, M, K, q.ptr, ldq, scales.ptr))

    def linear_i8_gelu_quant_r24(self, A: DeviceArray, lda: int, a_scale: DeviceArray, W: Weight,
                                 bias: Optional[DeviceArray], M: int, inter_hi: DeviceArray, inter_lo: DeviceArray,
                                 q: DeviceArray, ldq: int, q_scale: DeviceArray):
        """fc1 with the 24-bit intermediate, then GELU + per-token quantisation
        (the default forward's FFN up path, esm_gfx950_linear_i8_gelu_quant_r24)."""
        self._check(self.lib.esm_gfx950_linear_i8_gelu_quant_r24(
            self.ctx, A.ptr, lda, a_scale.ptr, W.handle, bias.ptr if bias is not None else None, M, inter_hi.ptr,
            inter_lo.ptr, q.ptr, ldq, q_scale.ptr))

    def linear_i8(self, A: DeviceArray, W: Weight, bias: Optional[DeviceArray], C_out: DeviceArray, M: int, N: int,
                  K: int, mode: int):
        self._check(self.lib.esm_gfx950_linear_i8(self.ctx, A.ptr, W.handle, bias.ptr if bias is not None else None,
                                                  C_out.ptr, M, N, K, mode))

    def linear_i8_noalloc(self, A: DeviceArray, W: Weight, bias: Optional[DeviceArray], C_out: DeviceArray, M: int,
                          N: int, K: int, mode: int):
        """linear_i8 without any device allocation (static 64 MiB scratch)."""
        self._check(self.lib.esm_gfx950_linear_i8_noalloc(self.ctx, A.ptr, W.handle,
                                                          bias.ptr if bias is not None else None, C_out.ptr, M, N, K,
                                                          mode))

    def linear_f32(self, A, W, bias, C_out, M, N, K):
        self._check(self.lib.esm_gfx950_linear_f32(self.ctx, A.ptr, W.ptr, bias.ptr if bias is not None else None,
                                                   C_out.ptr, M, N, K))

    def layernorm(self, x, gamma, beta, eps, out, rows, d):
        self._check(self.lib.esm_gfx950_layernorm(self.ctx, x.ptr, gamma.ptr, beta.ptr, eps, out.ptr, rows, d))

    def gelu(self, x, out, n):
        self._check(self.lib.esm_gfx950_gelu(self.ctx, x.ptr, out.ptr, n))

    def residual_add(self, y, x, n):
        self._check(self.lib.esm_gfx950_residual_add(self.ctx, y.ptr, x.ptr, n))

    def scale(self, x, n, s):
        self._check(self.lib.esm_gfx950_scale(self.ctx, x.ptr, n, s))

    def rope_apply_varlen(self, x, cos, sin, cu: np.ndarray, H: int, dh: int):
        cu = np.ascontiguousarray(cu, np.int32)
        self._check(self.lib.esm_gfx950_rope_apply_varlen(self.ctx, x.ptr, cos.ptr, sin.ptr, _ptr(cu), len(cu) - 1,
                                                          H, dh))

    def attention_varlen(self, q, k, v, cu: np.ndarray, H: int, dh: int, out, precision: int = ATTN_FP32):
        cu = np.ascontiguousarray(cu, np.int32)
        self._check(self.lib.esm_gfx950_attention_varlen(self.ctx, q.ptr, k.ptr, v.ptr, _ptr(cu), len(cu) - 1, H, dh,
                                                         out.ptr, precision))

    # The reference's x86 AVX-512 kernels, bit for bit.
    def layernorm_avx512(self, x, gamma, beta, eps, out, rows, d):
        self._check(self.lib.esm_gfx950_layernorm_avx512(self.ctx, x.ptr, gamma.ptr, beta.ptr, eps, out.ptr, rows, d))

    def gelu_avx512(self, x, out, n):
        self._check(self.lib.esm_gfx950_gelu_avx512(self.ctx, x.ptr, out.ptr, n))

    def expf_glibc(self, x, out, n):
        self._check(self.lib.esm_gfx950_expf_glibc(self.ctx, x.ptr, out.ptr, n))

    def linear_f32_avx512(self, A, W, bias, C_out, M, N, K):
        self._check(self.lib.esm_gfx950_linear_f32_avx512(self.ctx, A.ptr, W.ptr,
                                                          bias.ptr if bias is not None else None, C_out.ptr, M, N, K))

    def rope_apply_varlen_avx512(self, x, cos, sin, cu: np.ndarray, H: int, dh: int):
        cu = np.ascontiguousarray(cu, np.int32)
        self._check(self.lib.esm_gfx950_rope_apply_varlen_avx512(self.ctx, x.ptr, cos.ptr, sin.ptr, _ptr(cu),
                                                                 len(cu) - 1, H, dh))

    def attention_varlen_avx512(self, q, k, v, cu: np.ndarray, H: int, dh: int, out):
        cu = np.ascontiguousarray(cu, np.int32)
        self._check(self.lib.esm_gfx950_attention_varlen_avx512(self.ctx, q.ptr, k.ptr, v.ptr, _ptr(cu), len(cu) - 1,
                                                                H, dh, out.ptr))

    def attention_varlen_bf16(self, q, k, v, cu: np.ndarray, H: int, out, v_is_fp16: bool = False):
        cu = np.ascontiguousarray(cu, np.int32)
        self._check(self.lib.esm_gfx950_attention_varlen_bf16(self.ctx, q.ptr, k.ptr, v.ptr, int(v_is_fp16),
                                                              _ptr(cu), len(cu) - 1, H, out.ptr))


# ------------------------------------------------------------------ model
class ActivationObserver:
    """esm::ActivationObserver on the device (reference include/esm_cpp/observer.h:13-47):
    per-site reservoirs of |values| kept by Algorithm R with the reference's
    generator; observe() takes device values."""

    RESERVOIR_SIZE = 65536

    def __init__(self, dev: Device):
        self.dev = dev
        h = C.c_void_p()
        dev._check(dev.lib.esm_gfx950_observer_create(dev.ctx, C.byref(h)))
        self.handle = h

    def observe(self, site: str, values: DeviceArray, n: Optional[int] = None):
        n = int(np.prod(values.shape, dtype=np.int64)) if n is None else int(n)
        self.dev._check(self.dev.lib.esm_gfx950_observer_observe(self.dev.ctx, self.handle, site.encode(),
                                                                 values.ptr, n))

    def sites(self):
        lib = self.dev.lib
        n = C.c_size_t()
        self.dev._check(lib.esm_gfx950_observer_site_count(self.handle, C.byref(n)))
        out = []
        for i in range(n.value):
            name = C.c_char_p()
            self.dev._check(lib.esm_gfx950_observer_site_name(self.handle, i, C.byref(name)))
            out.append(name.value.decode())
        return out

    def percentile(self, pctile: float):
        """{site: pctile-th percentile} (ActivationObserver::Percentile)."""
        out = {}
        v = C.c_float()
        for site in self.sites():
            self.dev._check(self.dev.lib.esm_gfx950_observer_percentile(self.handle, site.encode(), float(pctile),
                                                                        C.byref(v)))
            out[site] = v.value
        return out

    def clear(self):
        self.dev._check(self.dev.lib.esm_gfx950_observer_clear(self.handle))

    def free(self):
        if self.handle:
            self.dev.lib.esm_gfx950_observer_free(self.dev.ctx, self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class _ModelConfig(C.Structure):
    _fields_ = [("num_layers", C.c_int), ("hidden_size", C.c_int), ("num_heads", C.c_int), ("head_dim", C.c_int),
                ("intermediate_size", C.c_int), ("vocab_size", C.c_int), ("layer_norm_eps", C.c_float),
                ("mask_token_id", C.c_int), ("weights_int8", C.c_int), ("act_quant_mode", C.c_int),
                ("attention_mode", C.c_int)]


class _LinearDesc(C.Structure):
    _fields_ = [("w_f32", C.c_void_p), ("w_i8", C.c_void_p), ("w_scale", C.c_void_p), ("bias", C.c_void_p)]


class _LayerDesc(C.Structure):
    _fields_ = [("attn_ln_w", C.c_void_p), ("attn_ln_b", C.c_void_p), ("q", _LinearDesc), ("k", _LinearDesc),
                ("v", _LinearDesc), ("out", _LinearDesc), ("ffn_ln_w", C.c_void_p), ("ffn_ln_b", C.c_void_p),
                ("fc1", _LinearDesc), ("fc2", _LinearDesc)]


class _ModelDesc(C.Structure):
    _fields_ = [("cfg", _ModelConfig), ("embed", C.c_void_p), ("layers", C.POINTER(_LayerDesc)),
                ("final_ln_w", C.c_void_p), ("final_ln_b", C.c_void_p), ("lm_dense_w", C.c_void_p),
                ("lm_dense_b", C.c_void_p), ("lm_ln_w", C.c_void_p), ("lm_ln_b", C.c_void_p),
                ("lm_decoder_bias", C.c_void_p)]


class Model:
    """Device-resident packed ESM-2 encoder (esm_gfx950_model).

    `weights` is an esm_gfx950.synthetic.EsmWeights (fp32 tensors plus, for
    W8A8, the per-channel int8 packs).
    """

    def __init__(self, dev: Device, weights, int8: bool, act_mode: int = ACT_PER_TOKEN,
                 attention_mode: int = ATTN_MODE_F16X3):
        cfg = weights.cfg
        keep: List[np.ndarray] = []

        def p(a):
            a = np.ascontiguousarray(a)
            keep.append(a)
            return a.ctypes.data

        def lin(name, i):
            d = _LinearDesc()
            d.bias = p(weights.f32[f"layers.{i}.{name}.bias"].astype(np.float32))
            if int8:
                q, s = weights.i8[f"layers.{i}.{name}"]
                d.w_i8 = p(q)
                d.w_scale = p(s)
            else:
                d.w_f32 = p(weights.f32[f"layers.{i}.{name}.weight"].astype(np.float32))
            return d

        layers = (_LayerDesc * max(cfg.num_layers, 1))()
        for i in range(cfg.num_layers):
            L = layers[i]
            L.attn_ln_w = p(weights.f32[f"layers.{i}.attn_ln.weight"])
            L.attn_ln_b = p(weights.f32[f"layers.{i}.attn_ln.bias"])
            L.ffn_ln_w = p(weights.f32[f"layers.{i}.ffn_ln.weight"])
            L.ffn_ln_b = p(weights.f32[f"layers.{i}.ffn_ln.bias"])
            L.q, L.k, L.v, L.out = lin("q", i), lin("k", i), lin("v", i), lin("out", i)
            L.fc1, L.fc2 = lin("fc1", i), lin("fc2", i)
        desc = _ModelDesc()
        desc.cfg = _ModelConfig(cfg.num_layers, cfg.hidden_size, cfg.num_heads, cfg.head_dim, cfg.intermediate_size,
                                cfg.vocab_size, cfg.layer_norm_eps, cfg.mask_token_id, int(int8), act_mode,
                                int(attention_mode))
        f = weights.f32
        desc.embed = p(f["embed"])
        desc.layers = layers
        desc.final_ln_w, desc.final_ln_b = p(f["final_ln.weight"]), p(f["final_ln.bias"])
        desc.lm_dense_w, desc.lm_dense_b = p(f["lm_head.dense.weight"]), p(f["lm_head.dense.bias"])
        desc.lm_ln_w, desc.lm_ln_b = p(f["lm_head.ln.weight"]), p(f["lm_head.ln.bias"])
        desc.lm_decoder_bias = p(f["lm_head.decoder.bias"])
        h = C.c_void_p()
        dev._check(dev.lib.esm_gfx950_model_create(dev.ctx, C.byref(desc), C.byref(h)))
        self.dev, self.handle, self.cfg = dev, h, cfg

    @classmethod
    def from_gguf(cls, dev: Device, path: str, act_mode: int = ACT_PER_TOKEN,
                  attention_mode: int = ATTN_MODE_F16X3) -> "Model":
        """A model from an esm.cpp GGUF file (esm_gfx950_model_create_from_gguf)."""
        from . import gguf
        from .synthetic import EsmConfig
        h = C.c_void_p()
        dev._check(dev.lib.esm_gfx950_model_create_from_gguf(dev.ctx, os.fsencode(path), int(act_mode),
                                                             int(attention_mode), C.byref(h)))
        meta = gguf.read_metadata(path)
        cfg = EsmConfig(str(meta.get("general.name", "gguf")), int(meta["esm.block_count"]),
                        int(meta["esm.embedding_length"]), int(meta["esm.attention.head_count"]),
                        int(meta["esm.feed_forward_length"]))
        m = cls.__new__(cls)
        m.dev, m.handle, m.cfg = dev, h, cfg
        return m

    def set_first_block_fc1_fp16(self, enabled: bool):
        """Round layer 0's fc1 input to fp16 (esm_gfx950_model_set_first_block_fc1_fp16)."""
        self.dev._check(self.dev.lib.esm_gfx950_model_set_first_block_fc1_fp16(self.dev.ctx, self.handle,
                                                                             int(bool(enabled))))

    def set_ffn_intermediate_bits(self, bits: int):
        """24 (default) or 32: width of the per-token W8A8 fc1 output that the
        GELU + quantisation pass reads (esm_gfx950_model_set_ffn_intermediate_bits)."""
        self.dev._check(self.dev.lib.esm_gfx950_model_set_ffn_intermediate_bits(self.dev.ctx, self.handle, int(bits)))

    def set_numerics(self, numerics: int):
        """NUMERICS_X86_AVX512: forward bit-equal to the reference's x86 AVX-512
        VNNI CPU path (esm_gfx950_model_set_numerics); drops the staged batch."""
        self.dev._check(self.dev.lib.esm_gfx950_model_set_numerics(self.dev.ctx, self.handle, int(numerics)))

    def set_act_mode(self, mode: int):
        self.dev._check(self.dev.lib.esm_gfx950_model_set_act_mode(self.dev.ctx, self.handle, mode))

    def set_lm_dense_split(self, enabled: bool):
        """lm head dense on the split-fp16 GEMM (True) or fp32 MFMA (False)."""
        self.dev._check(self.dev.lib.esm_gfx950_model_set_lm_dense_split(self.dev.ctx, self.handle, int(enabled)))

    def set_parts(self, parts: int):
        """Concurrent sequence groups per batch (esm_gfx950_model_set_parts);
        0 chooses per batch (the default)."""
        self.dev._check(self.dev.lib.esm_gfx950_model_set_parts(self.dev.ctx, self.handle, int(parts)))

    def staged_parts(self) -> int:
        """Groups the last staged batch was split into (esm_gfx950_model_staged_parts)."""
        n = C.c_int(0)
        self.dev._check(self.dev.lib.esm_gfx950_model_staged_parts(self.handle, C.byref(n)))
        return int(n.value)

    def forward_packed(self, ids: np.ndarray, cu: np.ndarray, out: Optional[DeviceArray] = None):
        """Packed forward; returns host logits [T, vocab] or fills `out` on device."""
        ids = np.ascontiguousarray(ids, np.int32)
        cu = np.ascontiguousarray(cu, np.int32)
        T = int(ids.shape[0])
        if out is None:
            logits = np.empty((T, self.cfg.vocab_size), np.float32)
            self.dev._check(self.dev.lib.esm_gfx950_forward_packed(self.dev.ctx, self.handle, _ptr(ids), _ptr(cu),
                                                                   len(cu) - 1, T, _ptr(logits), 0))
            return logits
        self.dev._check(self.dev.lib.esm_gfx950_forward_packed(self.dev.ctx, self.handle, _ptr(ids), _ptr(cu),
                                                               len(cu) - 1, T, out.ptr, 1))
        return out

    def forward_hidden_states(self, ids: np.ndarray, cu: np.ndarray, masks: Optional[np.ndarray] = None):
        """Packed forward returning (logits [T, vocab], hidden [layers + 1, T, d]):
        post-embed, each layer's output, and the post-final-LN state last
        (reference Model::ForwardWithHiddenStates, esm_gfx950_forward_hidden_states).
        masks: int32 [T], 0 marks a pad (None: every token real)."""
        ids = np.ascontiguousarray(ids, np.int32)
        cu = np.ascontiguousarray(cu, np.int32)
        mk = None if masks is None else np.ascontiguousarray(masks, np.int32)
        T = int(ids.shape[0])
        if mk is not None and mk.shape != ids.shape:
            raise ValueError("masks must match ids")
        logits = np.empty((T, self.cfg.vocab_size), np.float32)
        hidden = np.empty((self.cfg.num_layers + 1, T, self.cfg.hidden_size), np.float32)
        self.dev._check(self.dev.lib.esm_gfx950_forward_hidden_states(
            self.dev.ctx, self.handle, _ptr(ids), _ptr(mk) if mk is not None else None, _ptr(cu), len(cu) - 1, T,
            _ptr(logits), _ptr(hidden)))
        return logits, hidden

    def forward_packed_masked(self, ids: np.ndarray, masks: Optional[np.ndarray], cu: np.ndarray):
        """Packed forward with BatchView's pad masks (int32 [T], 0 = pad; None:
        every token real); host logits [T, vocab] (esm_gfx950_forward_packed_masked)."""
        ids = np.ascontiguousarray(ids, np.int32)
        cu = np.ascontiguousarray(cu, np.int32)
        mk = None if masks is None else np.ascontiguousarray(masks, np.int32)
        if mk is not None and mk.shape != ids.shape:
            raise ValueError("masks must match ids")
        T = int(ids.shape[0])
        logits = np.empty((T, self.cfg.vocab_size), np.float32)
        self.dev._check(self.dev.lib.esm_gfx950_forward_packed_masked(
            self.dev.ctx, self.handle, _ptr(ids), _ptr(mk) if mk is not None else None, _ptr(cu), len(cu) - 1, T,
            _ptr(logits), 0))
        return logits

    def forward_packed_with_observer(self, ids: np.ndarray, cu: np.ndarray, observer: "ActivationObserver"):
        """Packed forward that also feeds `observer` at the reference's four
        per-layer sites (esm_gfx950_forward_with_observer); host logits [T, vocab]."""
        ids = np.ascontiguousarray(ids, np.int32)
        cu = np.ascontiguousarray(cu, np.int32)
        T = int(ids.shape[0])
        logits = np.empty((T, self.cfg.vocab_size), np.float32)
        self.dev._check(self.dev.lib.esm_gfx950_forward_with_observer(
            self.dev.ctx, self.handle, _ptr(ids), _ptr(cu), len(cu) - 1, T, _ptr(logits), observer.handle))
        return logits

    def forward_with_observer(self, ids: np.ndarray, observer: "ActivationObserver"):
        """One sequence (reference Model::ForwardWithObserver, src/model.cpp:1084-1091)."""
        ids = np.ascontiguousarray(ids, np.int32)
        return self.forward_packed_with_observer(ids, np.array([0, ids.shape[0]], np.int32), observer)

    def forward_scheduled(self, ids_list, max_batch_size: int = 256, imbalance_threshold: float = 1.2):
        """Scheduled forward over a list of id arrays (esm_gfx950_forward_scheduled);
        returns one host logits array [L_i, vocab] per input, in input order."""
        n = len(ids_list)
        if n == 0:
            return []
        ids = [np.ascontiguousarray(x, np.int32) for x in ids_list]
        lens = np.array([x.shape[0] for x in ids], np.int32)
        outs = [np.empty((int(L), self.cfg.vocab_size), np.float32) for L in lens]
        id_ptrs = (C.c_void_p * n)(*[x.ctypes.data for x in ids])
        out_ptrs = (C.c_void_p * n)(*[o.ctypes.data for o in outs])
        self.dev._check(self.dev.lib.esm_gfx950_forward_scheduled(
            self.dev.ctx, self.handle, C.cast(id_ptrs, C.c_void_p), _ptr(lens), n, float(imbalance_threshold),
            int(max_batch_size), C.cast(out_ptrs, C.c_void_p)))
        return outs

    def upload_batch(self, ids: np.ndarray, cu: np.ndarray):
        """Stages a packed batch in device memory (esm_gfx950_batch_upload)."""
        ids = np.ascontiguousarray(ids, np.int32)
        cu = np.ascontiguousarray(cu, np.int32)
        self.dev._check(self.dev.lib.esm_gfx950_batch_upload(self.dev.ctx, self.handle, _ptr(ids), _ptr(cu),
                                                             len(cu) - 1, int(ids.shape[0])))

    def forward_device(self, out: DeviceArray):
        """Forward on the staged batch; logits stay on the device."""
        self.dev._check(self.dev.lib.esm_gfx950_forward_device(self.dev.ctx, self.handle, out.ptr))

    def arena_bytes(self) -> int:
        n = C.c_size_t()
        self.dev._check(self.dev.lib.esm_gfx950_model_arena_bytes(self.handle, C.byref(n)))
        return int(n.value)

    def free(self):
        if self.handle:
            self.dev.lib.esm_gfx950_model_free(self.dev.ctx, self.handle)
            self.handle = None
