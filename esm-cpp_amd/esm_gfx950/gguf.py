"""GGUF v3 files in esm.cpp's layout (reference src/io/gguf.cpp, tensor names
and metadata of Model::SaveToGguf, src/model.cpp:562-700).

write_model() writes synthetic or converted ESM-2 weights so that
esm_gfx950_model_create_from_gguf (and the reference's Model::LoadFromGguf)
can load them; read() parses a file into metadata and numpy arrays.

Layout: "GGUF", uint32 version 3, uint64 tensor count, uint64 metadata count,
metadata (key string, uint32 type, value), tensor infos (name string, uint32
n_dims, uint64 dims fastest-first, uint32 type, uint64 offset), zero padding
to general.alignment (32), tensor data, each tensor padded to the alignment.
Strings are a uint64 length plus bytes. Q8_ESM (type 100) is esm.cpp's
per-channel int8 blob: [N, K] int8 followed by [N] fp32 scales, dims [K, N].
"""
from __future__ import annotations

import struct
from typing import Dict, List, Tuple

import numpy as np

MAGIC = b"GGUF"
VERSION = 3
ALIGNMENT = 32
F32, F16, Q8_ESM = 0, 1, 100
# metadata value types
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_SCALAR = {_U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f", _BOOL: "<B",
           _U64: "<Q", _I64: "<q", _F64: "<d"}


def _s(b: str) -> bytes:
    e = b.encode()
    return struct.pack("<Q", len(e)) + e


def _meta(value) -> bytes:
    if isinstance(value, bool):
        return struct.pack("<I", _BOOL) + struct.pack("<B", int(value))
    if isinstance(value, int):
        return struct.pack("<I", _I64) + struct.pack("<q", value)
    if isinstance(value, float):
        return struct.pack("<I", _F64) + struct.pack("<d", value)
    if isinstance(value, str):
        return struct.pack("<I", _STR) + _s(value)
    if isinstance(value, (list, tuple)):
        if all(isinstance(v, str) for v in value):
            return struct.pack("<IIQ", _ARR, _STR, len(value)) + b"".join(_s(v) for v in value)
        if all(isinstance(v, int) and not isinstance(v, bool) for v in value):
            return struct.pack("<IIQ", _ARR, _I64, len(value)) + b"".join(struct.pack("<q", v) for v in value)
        return struct.pack("<IIQ", _ARR, _F64, len(value)) + b"".join(struct.pack("<d", float(v)) for v in value)
    raise TypeError(f"unsupported metadata value {value!r}")


def write(path: str, metadata: Dict[str, object], tensors: List[Tuple[str, int, Tuple[int, ...], bytes]]):
    """Writes a GGUF v3 file. tensors: (name, type, dims fastest-first, raw bytes)."""
    align = int(metadata.get("general.alignment", ALIGNMENT))
    head = bytearray(MAGIC + struct.pack("<IQQ", VERSION, len(tensors), len(metadata)))
    for k, v in metadata.items():
        head += _s(k) + _meta(v)
    offsets, cursor = [], 0
    for _, _, _, data in tensors:
        offsets.append(cursor)
        cursor += len(data) + (-len(data)) % align
    for (name, ttype, dims, _), off in zip(tensors, offsets):
        head += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", int(x)) for x in dims)
        head += struct.pack("<IQ", ttype, off)
    head += b"\0" * ((-len(head)) % align)
    with open(path, "wb") as f:
        f.write(head)
        for _, _, _, data in tensors:
            f.write(data)
            f.write(b"\0" * ((-len(data)) % align))


def _q8_blob(q: np.ndarray, scales: np.ndarray) -> bytes:
    return np.ascontiguousarray(q, np.int8).tobytes() + np.ascontiguousarray(scales, np.float32).tobytes()


def write_model(path: str, weights, int8: bool):
    """ESM-2 weights (esm_gfx950.synthetic.EsmWeights layout) in the names,
    dims and metadata Model::SaveToGguf writes (src/model.cpp:562-700)."""
    cfg = weights.cfg
    d, f, V, L = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.num_layers
    F = weights.f32
    meta = {
        "general.architecture": "esm",
        "general.alignment": ALIGNMENT,
        "general.file_type": 2 if int8 else 1,
        "esm.block_count": L,
        "esm.embedding_length": d,
        "esm.feed_forward_length": f,
        "esm.attention.head_count": cfg.num_heads,
        "esm.attention.head_count_kv": cfg.num_heads,
        "esm.attention.layer_norm_epsilon": float(np.float32(cfg.layer_norm_eps)),
        "esm.rope.dimension_count": cfg.head_dim,
        "esm.context_length": 1024,
        "esm.gguf_writer": "esm-gfx950",
        "esm.weights_quantized": bool(int8),
        "esm.first_block_fc1_fp16": False,
    }

    def f32(name, arr, dims):
        return (name, F32, dims, np.ascontiguousarray(arr, np.float32).tobytes())

    def lin(name, key, N, K):
        if int8:
            q, s = weights.i8[key]
            return (name, Q8_ESM, (K, N), _q8_blob(q, s))
        return f32(name, F[key + ".weight"], (K, N))

    t = [f32("token_embd.weight", F["embed"], (d, V))]
    for i in range(L):
        p, b = f"layers.{i}.", f"blk.{i}."
        t += [f32(b + "attn_norm.weight", F[p + "attn_ln.weight"], (d,)),
              f32(b + "attn_norm.bias", F[p + "attn_ln.bias"], (d,))]
        t += [lin(b + f"attn_{n}.weight", p + m, d, d) for n, m in (("q", "q"), ("k", "k"), ("v", "v"),
                                                                    ("output", "out"))]
        t += [f32(b + f"attn_{n}.bias", F[p + m + ".bias"], (d,)) for n, m in (("q", "q"), ("k", "k"), ("v", "v"),
                                                                              ("output", "out"))]
        t += [f32(b + "ffn_norm.weight", F[p + "ffn_ln.weight"], (d,)),
              f32(b + "ffn_norm.bias", F[p + "ffn_ln.bias"], (d,)),
              lin(b + "ffn_up.weight", p + "fc1", f, d), lin(b + "ffn_down.weight", p + "fc2", d, f),
              f32(b + "ffn_up.bias", F[p + "fc1.bias"], (f,)), f32(b + "ffn_down.bias", F[p + "fc2.bias"], (d,))]
    t += [f32("enc_norm.weight", F["final_ln.weight"], (d,)), f32("enc_norm.bias", F["final_ln.bias"], (d,)),
          f32("lm_head.weight", F["lm_head.dense.weight"], (d, d)), f32("lm_head.bias", F["lm_head.dense.bias"], (d,)),
          f32("lm_head_norm.weight", F["lm_head.ln.weight"], (d,)),
          f32("lm_head_norm.bias", F["lm_head.ln.bias"], (d,)),
          f32("output.bias", F["lm_head.decoder.bias"], (V,))]
    write(path, meta, t)


class _Reader:
    def __init__(self, buf: bytes):
        self.b, self.p = buf, 0

    def take(self, n: int) -> bytes:
        if self.p + n > len(self.b):
            raise ValueError("gguf: truncated read")
        out = self.b[self.p:self.p + n]
        self.p += n
        return out

    def unpack(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        return self.take(self.unpack("<Q")).decode()

    def scalar(self, t: int):
        if t == _STR:
            return self.string()
        if t not in _SCALAR:
            raise ValueError(f"gguf: unknown metadata type {t}")
        v = self.unpack(_SCALAR[t])
        return bool(v) if t == _BOOL else v

    def value(self):
        t = self.unpack("<I")
        if t != _ARR:
            return self.scalar(t)
        et, n = self.unpack("<I"), self.unpack("<Q")
        return [self.scalar(et) for _ in range(n)]


def read_metadata(path: str) -> Dict[str, object]:
    """Only the metadata of a GGUF file (reads the header, not the data)."""
    with open(path, "rb") as fh:
        head = fh.read(1 << 20)
        r = _Reader(head)
        if r.take(4) != MAGIC:
            raise ValueError(f"gguf: bad magic in {path}")
        version = r.unpack("<I")
        if version != VERSION:
            raise ValueError(f"gguf: version {version} not supported (need v3)")
        r.unpack("<Q")
        nm = r.unpack("<Q")
        meta = {}
        for _ in range(nm):
            k = r.string()
            meta[k] = r.value()
    return meta


def read(path: str):
    """(metadata dict, {name: (type, dims, numpy array or (int8 [N, K], fp32 [N]))})."""
    with open(path, "rb") as fh:
        buf = fh.read()
    r = _Reader(buf)
    if r.take(4) != MAGIC:
        raise ValueError(f"gguf: bad magic in {path}")
    version = r.unpack("<I")
    if version != VERSION:
        raise ValueError(f"gguf: version {version} not supported (need v3)")
    nt, nm = r.unpack("<Q"), r.unpack("<Q")
    meta = {}
    for _ in range(nm):
        k = r.string()
        meta[k] = r.value()
    infos = []
    for _ in range(nt):
        name = r.string()
        nd = r.unpack("<I")
        dims = tuple(r.unpack("<Q") for _ in range(nd))
        infos.append((name, r.unpack("<I"), dims, r.unpack("<Q")))
    align = int(meta.get("general.alignment", ALIGNMENT))
    data0 = (r.p + align - 1) // align * align
    out = {}
    for name, ttype, dims, off in infos:
        n = int(np.prod(dims)) if dims else 1
        start = data0 + off
        if ttype == F32:
            arr = np.frombuffer(buf, np.float32, n, start)
        elif ttype == F16:
            arr = np.frombuffer(buf, np.float16, n, start)
        elif ttype == Q8_ESM:
            K, N = dims
            arr = (np.frombuffer(buf, np.int8, N * K, start).reshape(N, K),
                   np.frombuffer(buf, np.float32, N, start + N * K))
        else:
            raise ValueError(f"gguf: unknown tensor type {ttype} for {name}")
        out[name] = (ttype, dims, arr)
    return meta, out
