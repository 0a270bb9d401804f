"""Synthetic ESM-2 models and packed batches for the benchmark configs.

Nothing here touches the GPU. Weights follow the recipe used for every
measurement in this repository:
  * Linear weights, biases and embeddings ~ N(0, 0.02);
  * LayerNorm gamma = 1 + N(0, 0.02), beta ~ N(0, 0.02);
  * the decoder is tied to the embedding (reference src/model.cpp:142-143);
  * W8A8 models get synthetic SmoothQuant factors s ~ logU(0.5, 2) per
    input channel and site, folded with the reference's three site rules
    (src/quant/smoothquant.cpp:100-185), then per-channel symmetric INT8
    quantisation with the reference's Quantize (src/quant/pack.cpp:149-177).
Every tensor has its own numpy PCG64 stream keyed by (seed, crc32(name)).

Token ids: cls = 0, residues uniform over ids 4..23 (the 20 standard amino
acids, reference src/tokenizer.cpp:12-17), eos = 2; no masks, no pads.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import zlib
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

CLS, PAD, EOS, MASK = 0, 1, 2, 32
RESIDUE_LO, RESIDUE_HI = 4, 23  # inclusive


@dataclass(frozen=True)
class EsmConfig:
    name: str
    num_layers: int
    hidden_size: int
    num_heads: int
    intermediate_size: int
    vocab_size: int = 33
    layer_norm_eps: float = 1e-5
    mask_token_id: int = MASK

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    def with_layers(self, n: int) -> "EsmConfig":
        return EsmConfig(f"{self.name}-L{n}", n, self.hidden_size, self.num_heads, self.intermediate_size,
                         self.vocab_size, self.layer_norm_eps, self.mask_token_id)


ESM2_8M = EsmConfig("esm2_t6_8M", 6, 320, 20, 1280)
ESM2_650M = EsmConfig("esm2_t33_650M", 33, 1280, 20, 5120)
ESM2_3B = EsmConfig("esm2_t36_3B", 36, 2560, 40, 10240)

LINEARS = ("q", "k", "v", "out", "fc1", "fc2")


def _rng(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def _normal(seed: int, name: str, shape, std: float = 0.02, mean: float = 0.0) -> np.ndarray:
    a = _rng(seed, name).standard_normal(size=shape, dtype=np.float32)
    a *= np.float32(std)
    if mean:
        a += np.float32(mean)
    return a


def quantize_weight(W: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Per-output-channel symmetric INT8 (reference Quantize, pack.cpp:149-177).

    scale[n] = max|W[n,:]| / 127 (0 for an all-zero row),
    q = clamp(nearbyint(W * (1 / scale)), -127, 127); all float32 arithmetic.
    """
    W = np.ascontiguousarray(W, np.float32)
    row_max = np.max(np.abs(W), axis=1).astype(np.float32)
    scale = (row_max / np.float32(127.0)).astype(np.float32)
    zero = row_max == 0
    safe = np.where(zero, np.float32(1.0), scale).astype(np.float32)
    inv = (np.float32(1.0) / safe).astype(np.float32)
    q = np.rint(W * inv[:, None])
    np.clip(q, -127, 127, out=q)
    q = q.astype(np.int8)
    q[zero] = 0
    scale[zero] = 0.0
    return q, scale


def _smooth_factors(seed: int, name: str, n: int) -> np.ndarray:
    u = _rng(seed, name).uniform(np.log(0.5), np.log(2.0), size=n)
    return np.exp(u).astype(np.float32)


@dataclass
class EsmWeights:
    cfg: EsmConfig
    f32: Dict[str, np.ndarray] = field(default_factory=dict)
    i8: Dict[str, Tuple[np.ndarray, np.ndarray]] = field(default_factory=dict)


def make_weights(cfg: EsmConfig, seed: int, int8: bool = False, smooth: bool = True,
                 keep_f32_linears: Optional[bool] = None) -> EsmWeights:
    """Random-init ESM-2 weights; int8=True adds SmoothQuant folding + INT8 packs.

    keep_f32_linears (default: not int8) keeps the fp32 linear weights after
    quantisation (needed only by fp32 references).
    """
    if keep_f32_linears is None:
        keep_f32_linears = not int8
    d, f, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    w = EsmWeights(cfg)
    F = w.f32
    F["embed"] = _normal(seed, "embed", (V, d))

    def layer(i):
        """Layer i's tensors (fp32 dict, int8 dict); every tensor draws from
        its own stream, so layers can be made in any order or concurrently."""
        p = f"layers.{i}."
        f32, i8 = {}, {}
        for ln in ("attn_ln", "ffn_ln"):
            f32[p + ln + ".weight"] = _normal(seed, p + ln + ".weight", (d,), mean=1.0)
            f32[p + ln + ".bias"] = _normal(seed, p + ln + ".bias", (d,))
        shapes = {"q": (d, d), "k": (d, d), "v": (d, d), "out": (d, d), "fc1": (f, d), "fc2": (d, f)}
        lin = {n: _normal(seed, p + n + ".weight", s) for n, s in shapes.items()}
        for n, s in shapes.items():
            f32[p + n + ".bias"] = _normal(seed, p + n + ".bias", (s[0],))
        if int8 and smooth:
            # Site 1: attn_ln -> {q,k,v}
            s1 = _smooth_factors(seed, p + "smooth.attn_ln", d)
            f32[p + "attn_ln.weight"] = f32[p + "attn_ln.weight"] / s1
            f32[p + "attn_ln.bias"] = f32[p + "attn_ln.bias"] / s1
            for n in ("q", "k", "v"):
                lin[n] = lin[n] * s1[None, :]
            # Site 2: v output channels -> out_proj input channels
            s2 = _smooth_factors(seed, p + "smooth.attn_out", d)
            f32[p + "v.bias"] = f32[p + "v.bias"] / s2
            lin["v"] = lin["v"] / s2[:, None]
            lin["out"] = lin["out"] * s2[None, :]
            # Site 3: ffn_ln -> fc1
            s3 = _smooth_factors(seed, p + "smooth.ffn_ln", d)
            f32[p + "ffn_ln.weight"] = f32[p + "ffn_ln.weight"] / s3
            f32[p + "ffn_ln.bias"] = f32[p + "ffn_ln.bias"] / s3
            lin["fc1"] = lin["fc1"] * s3[None, :]
        for n, W in lin.items():
            W = W.astype(np.float32, copy=False)
            if int8:
                i8[p + n] = quantize_weight(W)
            if keep_f32_linears:
                f32[p + n + ".weight"] = W
        return f32, i8

    # numpy's generators and array arithmetic release the GIL on large
    # arrays, so layers are made on a few threads (same values as in order).
    workers = max(1, min(8, os.cpu_count() or 1, cfg.num_layers))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        for f32, i8 in ex.map(layer, range(cfg.num_layers)):
            F.update(f32)
            w.i8.update(i8)
    F["final_ln.weight"] = _normal(seed, "final_ln.weight", (d,), mean=1.0)
    F["final_ln.bias"] = _normal(seed, "final_ln.bias", (d,))
    F["lm_head.dense.weight"] = _normal(seed, "lm_head.dense.weight", (d, d))
    F["lm_head.dense.bias"] = _normal(seed, "lm_head.dense.bias", (d,))
    F["lm_head.ln.weight"] = _normal(seed, "lm_head.ln.weight", (d,), mean=1.0)
    F["lm_head.ln.bias"] = _normal(seed, "lm_head.ln.bias", (d,))
    F["lm_head.decoder.bias"] = _normal(seed, "lm_head.decoder.bias", (V,))
    for k in list(F):
        F[k] = np.ascontiguousarray(F[k], np.float32)
    return w


# ------------------------------------------------------------------ batches
@dataclass
class PackedBatch:
    ids: np.ndarray      # int32 [T]
    cu: np.ndarray       # int32 [B + 1]
    lengths: np.ndarray  # int32 [B] tokens per sequence (cls + residues + eos)

    @property
    def total_tokens(self) -> int:
        return int(self.cu[-1])

    @property
    def residues(self) -> int:
        return int(np.sum(self.lengths - 2))

    def subset(self, idx) -> "PackedBatch":
        seqs = [self.ids[self.cu[i]:self.cu[i + 1]] for i in idx]
        return pack(seqs)


def pack(seqs: List[np.ndarray]) -> PackedBatch:
    lengths = np.array([len(s) for s in seqs], np.int32)
    cu = np.zeros(len(seqs) + 1, np.int32)
    cu[1:] = np.cumsum(lengths)
    ids = np.concatenate(seqs).astype(np.int32) if seqs else np.zeros(0, np.int32)
    return PackedBatch(ids, cu, lengths)


def batch_from_lengths(lengths, seed: int) -> PackedBatch:
    rng = np.random.default_rng([seed, zlib.crc32(b"residues")])
    seqs = []
    for L in lengths:
        res = rng.integers(RESIDUE_LO, RESIDUE_HI + 1, size=int(L) - 2, dtype=np.int32)
        seqs.append(np.concatenate([[CLS], res, [EOS]]).astype(np.int32))
    return pack(seqs)


def varlen_lengths(n: int, seed: int, mean: float = 120.0, sd: float = 30.0, lo: int = 60, hi: int = 250):
    """Token lengths clip(round(N(mean, sd)), lo, hi) (configs 2 and 4)."""
    rng = np.random.default_rng([seed, zlib.crc32(b"lengths")])
    return np.clip(np.rint(rng.normal(mean, sd, size=n)), lo, hi).astype(np.int32)


def loguniform_lengths(n: int, seed: int, lo: int = 50, hi: int = 1024):
    """Token lengths clip(round(exp(U(ln lo, ln hi))), lo, hi) (config 5)."""
    rng = np.random.default_rng([seed, zlib.crc32(b"lengths")])
    return np.clip(np.rint(np.exp(rng.uniform(np.log(lo), np.log(hi), size=n))), lo, hi).astype(np.int32)


def config1_batch(seed: int = 20261201 + 1) -> PackedBatch:
    """16 sequences, residues uniform in [20, 200] (config 1)."""
    rng = np.random.default_rng([seed, zlib.crc32(b"lengths")])
    res = rng.integers(20, 201, size=16)
    return batch_from_lengths(res + 2, seed)


def config4_varlen_batch(seed: int = 20261201 + 4) -> PackedBatch:
    return batch_from_lengths(varlen_lengths(256, seed), seed)


def config4_uniform_batch(seed: int = 20261201 + 4) -> PackedBatch:
    return batch_from_lengths(np.full(8, 256, np.int32), seed)


def config5_batch(seed: int = 20261201 + 5) -> PackedBatch:
    return batch_from_lengths(loguniform_lengths(64, seed), seed)
