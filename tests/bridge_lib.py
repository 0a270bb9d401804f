"""ctypes view of esm-cpp_amd/lib/libesm_gfx950_bridge.so, the reference-side
bridge compiled against the reference's headers (esm-cpp_amd/bridge/)."""
import ctypes as C
import os

import numpy as np

from conftest import ROOT

BRIDGE_LIB = os.path.join(ROOT, "esm-cpp_amd", "lib", "libesm_gfx950_bridge.so")
vp, i32, sz, f32 = C.c_void_p, C.c_int, C.c_size_t, C.c_float
SIGNATURES = {
    "esm_gfx950_bridge_last_error": (C.c_char_p, []),
    "esm_gfx950_bridge_linear": (i32, [vp, vp, vp, vp, i32, i32, i32]),
    "esm_gfx950_bridge_linear_int8": (i32, [vp, vp, vp, vp, vp, i32, i32, i32]),
    "esm_gfx950_bridge_layernorm": (i32, [vp, vp, vp, f32, vp, i32, i32]),
    "esm_gfx950_bridge_gelu": (i32, [vp, vp, sz]),
    "esm_gfx950_bridge_residual_add": (i32, [vp, vp, sz]),
    "esm_gfx950_bridge_scale": (i32, [vp, sz, f32]),
    "esm_gfx950_bridge_rope_apply_varlen": (i32, [vp, vp, vp, vp, i32, i32, i32]),
    "esm_gfx950_bridge_attention_varlen": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "esm_gfx950_bridge_forward_packed": (i32, [vp, vp, vp, vp, i32, i32, i32, vp, vp]),
    "esm_gfx950_bridge_forward_scheduled": (i32, [vp, vp, vp, vp, i32, f32, i32, vp]),
    "esm_gfx950_bridge_qt_create": (vp, [vp, vp, i32, i32]),
    "esm_gfx950_bridge_qt_data": (vp, [vp]),
    "esm_gfx950_bridge_linear_int8_qt": (i32, [vp, vp, vp, vp, i32]),
    "esm_gfx950_bridge_qt_free": (None, [vp]),
}


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _c(a, dt):
    return np.ascontiguousarray(a, dt)


class Bridge:
    def __init__(self):
        lib = C.CDLL(BRIDGE_LIB)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        self.lib = lib

    def error(self) -> str:
        return self.lib.esm_gfx950_bridge_last_error().decode()

    def _check(self, ran):
        if ran != 1:
            raise RuntimeError(f"bridge arm fell back to the CPU: {self.error()}")

    def linear(self, A, W, bias):
        A, W = _c(A, np.float32), _c(W, np.float32)
        out = np.empty((A.shape[0], W.shape[0]), np.float32)
        self._check(self.lib.esm_gfx950_bridge_linear(_p(A), _p(W), _p(None if bias is None else _c(bias, np.float32)),
                                                      _p(out), A.shape[0], W.shape[0], A.shape[1]))
        return out

    def linear_int8(self, A, q, s, bias):
        A = _c(A, np.float32)
        out = np.empty((A.shape[0], q.shape[0]), np.float32)
        self._check(self.lib.esm_gfx950_bridge_linear_int8(
            _p(A), _p(_c(q, np.int8)), _p(_c(s, np.float32)), _p(None if bias is None else _c(bias, np.float32)),
            _p(out), A.shape[0], q.shape[0], A.shape[1]))
        return out

    def layernorm(self, x, g, b, eps=1e-5):
        x = _c(x, np.float32)
        out = np.empty_like(x)
        self._check(self.lib.esm_gfx950_bridge_layernorm(_p(x), _p(_c(g, np.float32)), _p(_c(b, np.float32)), eps,
                                                         _p(out), *x.shape))
        return out

    def gelu(self, x):
        x = _c(x, np.float32)
        out = np.empty_like(x)
        self._check(self.lib.esm_gfx950_bridge_gelu(_p(x), _p(out), x.size))
        return out

    def residual_add(self, y, x):
        y = np.array(y, np.float32, copy=True, order="C")
        self._check(self.lib.esm_gfx950_bridge_residual_add(_p(y), _p(_c(x, np.float32)), y.size))
        return y

    def scale(self, x, s):
        x = np.array(x, np.float32, copy=True, order="C")
        self._check(self.lib.esm_gfx950_bridge_scale(_p(x), x.size, s))
        return x

    def rope_varlen(self, x, cos, sin, cu, H, dh):
        x = np.array(x, np.float32, copy=True, order="C")
        cu = _c(cu, np.int32)
        self._check(self.lib.esm_gfx950_bridge_rope_apply_varlen(_p(x), _p(_c(cos, np.float32)),
                                                                 _p(_c(sin, np.float32)), _p(cu), len(cu) - 1, H, dh))
        return x

    def attention_varlen(self, q, k, v, cu, H, dh):
        q, k, v, cu = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32), _c(cu, np.int32)
        out = np.zeros((int(cu[-1]), H * dh), np.float32)
        self._check(self.lib.esm_gfx950_bridge_attention_varlen(_p(q), _p(k), _p(v), _p(cu), len(cu) - 1, H, dh,
                                                                _p(out)))
        return out

    def forward_packed(self, model, ids, cu, masks=None, layers=None, hidden_size=None, vocab=33):
        """ForwardPacked through a BatchView: (per-sequence logits list,
        hidden [layers + 1, T, d] or None). Raises ValueError with BatchView's
        message when it rejects the batch."""
        ids, cu = _c(ids, np.int32), _c(cu, np.int32)
        mk = None if masks is None else _c(masks, np.int32)
        T = ids.shape[0]
        logits = np.zeros((T, vocab), np.float32)
        hidden = None if layers is None else np.zeros((layers + 1, T, hidden_size), np.float32)
        rc = self.lib.esm_gfx950_bridge_forward_packed(model.handle, _p(ids), _p(mk), _p(cu), len(cu), len(cu) - 1,
                                                       T, _p(logits), _p(hidden))
        if rc == -1:
            raise ValueError(self.error())
        self._check(rc)
        return [logits[cu[b]:cu[b + 1]] for b in range(len(cu) - 1)], hidden

    def forward_scheduled(self, model, seqs, masks=None, threshold=1.2, max_batch=256, vocab=33):
        lengths = np.array([len(x) for x in seqs], np.int32)
        ids = _c(np.concatenate(seqs), np.int32)
        mk = None if masks is None else _c(np.concatenate(masks), np.int32)
        out = np.zeros((ids.shape[0], vocab), np.float32)
        self._check(self.lib.esm_gfx950_bridge_forward_scheduled(model.handle, _p(ids), _p(lengths), _p(mk),
                                                                 len(seqs), threshold, max_batch, _p(out)))
        offs = np.concatenate([[0], np.cumsum(lengths)])
        return [out[offs[i]:offs[i + 1]] for i in range(len(seqs))]
