// Packed variable-length bidirectional attention for gfx950.
//
// Replaces esm::kernels::AttentionVarlen (reference
// src/kernels/attention.cpp:99-144 AttentionVarlenRef and :770-811
// AttentionVarlenAvx512): per sequence b (rows [cu[b], cu[b+1])), per head
// h, out = softmax(q k^T) v with no mask inside the segment and no
// attention across segments. Q arrives pre-scaled (ESM scales Q before
// RoPE, reference src/model.cpp:975-988).
//
// MFMA path (head_dim 64): one workgroup per (sequence, head, 128-query
// tile); its four waves each own 32 queries. Keys are processed in chunks
// of 128 staged through LDS: K row-major (bf16 or fp16), V transposed to
// [dim][key] and converted to fp16. Each wave computes S^T = K Q^T with
// v_mfma_f32_16x16x32_{bf16,f16}, so every lane ends up holding probabilities for
// one query and four consecutive keys per 16-key block -- exactly the B
// operand layout of O^T = V^T P^T on v_mfma_f32_16x16x32_f16. Softmax is an
// online (running max / running sum) fp32 softmax in base 2; the
// probabilities are rounded to fp16 before both the PV product and the
// running sum, so the normalisation uses the same weights as the product.
//
// fp32 path (any head_dim <= 128): one wave per (sequence, head, 64-query
// tile), one lane per query; two passes over the keys (max, then
// exp/sum/weighted V with a double-precision sum), the reference's order.
#include <math.h>

#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace esm_gfx950 {
namespace {

constexpr int KC = 128;                 // keys per LDS chunk
constexpr int kKPitch = 64 * 2 + 16;    // bytes per key row of K (bf16)
constexpr int kVPitch = KC * 2 + 16;    // bytes per dim row of V^T (fp16)
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ uint16_t bf16_to_f16_bits(uint16_t b) {
  return f32_to_f16_bits(bf16_bits_to_f32(b));
}

// Q/K operand type of S^T = K Q^T: bf16 (v_mfma_f32_16x16x32_bf16) or fp16
// (v_mfma_f32_16x16x32_f16), same rate; fp16 carries three more mantissa
// bits for the O(1) values attention sees.
template <bool F16>
struct QKOps;
template <>
struct QKOps<false> {
  using vec = bf16x8;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct QKOps<true> {
  using vec = f16x8;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <bool QK_F16, bool V_BF16>
__global__ __launch_bounds__(256) void attn_mfma_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, int ld, const int* __restrict__ cu,
    const AttnWork* __restrict__ work, float* __restrict__ out, int ld_out,
    float* tensor_absmax) {
  __shared__ __attribute__((aligned(16))) uint8_t sK[KC * kKPitch];
  __shared__ __attribute__((aligned(16))) uint8_t sVt[64 * kVPitch];

  const AttnWork w = work[blockIdx.x];
  const int start = cu[w.seq];
  const int L = cu[w.seq + 1] - start;
  if (w.q0 >= L) return;  // padding item of the work list (uniform)
  const int hoff = w.head * 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int qbase = w.q0 + wave * 32;
  const bool active = qbase < L;  // wave-uniform

  using QK = QKOps<QK_F16>;
  using qvec = typename QK::vec;
  qvec qf[2][2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    int qi = qbase + qb * 16 + lr;
    qi = qi < L ? qi : L - 1;
    const uint16_t* qp = q + static_cast<size_t>(start + qi) * ld + hoff;
    qf[qb][0] = *reinterpret_cast<const qvec*>(qp + lg * 8);
    qf[qb][1] = *reinterpret_cast<const qvec*>(qp + 32 + lg * 8);
  }

  f32x4 o[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int db = 0; db < 4; ++db) o[qb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mrun[2] = {-INFINITY, -INFINITY};
  float lrun[2] = {0.f, 0.f};

  for (int kc0 = 0; kc0 < L; kc0 += KC) {
    const int nkeys = min(KC, L - kc0);
    __syncthreads();
    // K chunk: KC rows x 128 bytes; rows past the sequence are zero.
#pragma unroll
    for (int i = 0; i < KC * 8 / 256; ++i) {
      const int idx = threadIdx.x + 256 * i;
      const int key = idx >> 3, c = idx & 7;
      uint4 val = make_uint4(0u, 0u, 0u, 0u);
      if (key < nkeys)
        val = *reinterpret_cast<const uint4*>(k + static_cast<size_t>(start + kc0 + key) * ld + hoff + c * 8);
      *reinterpret_cast<uint4*>(sK + key * kKPitch + c * 16) = val;
    }
    // V chunk transposed: each thread takes a key pair and 8 dims and
    // writes 8 dwords (key pair packed) into V^T rows.
#pragma unroll
    for (int i = 0; i < KC * 4 / 256; ++i) {
      const int idx = threadIdx.x + 256 * i;
      const int kp = idx % (KC / 2), dg = idx / (KC / 2);
      const int key0 = 2 * kp;
      uint4 a = make_uint4(0u, 0u, 0u, 0u), b = a;
      const uint16_t* vp = v + static_cast<size_t>(start + kc0 + key0) * ld + hoff + dg * 8;
      if (key0 < nkeys) a = *reinterpret_cast<const uint4*>(vp);
      if (key0 + 1 < nkeys) b = *reinterpret_cast<const uint4*>(vp + ld);
      const uint16_t* ah = reinterpret_cast<const uint16_t*>(&a);
      const uint16_t* bh = reinterpret_cast<const uint16_t*>(&b);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t lo = ah[j], hi = bh[j];
        if constexpr (V_BF16) {
          lo = bf16_to_f16_bits(static_cast<uint16_t>(lo));
          hi = bf16_to_f16_bits(static_cast<uint16_t>(hi));
        }
        *reinterpret_cast<uint32_t*>(sVt + (dg * 8 + j) * kVPitch + key0 * 2) = lo | (hi << 16);
      }
    }
    __syncthreads();
    if (!active) continue;

    const int nkb = (nkeys + 15) >> 4;
    f32x4 s[8][2];
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) {
      if (kb < nkb) {
        const uint8_t* kp = sK + (kb * 16 + lr) * kKPitch + lg * 16;
        const qvec k0 = *reinterpret_cast<const qvec*>(kp);
        const qvec k1 = *reinterpret_cast<const qvec*>(kp + 64);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          f32x4 acc = QK::mma(k0, qf[qb][0], f32x4{0.f, 0.f, 0.f, 0.f});
          s[kb][qb] = QK::mma(k1, qf[qb][1], acc);
        }
      }
    }

    // Online softmax in base 2; lane holds keys kb*16 + 4*lg + i.
    f16x4 pv[8][2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      float cmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 8; ++kb) {
        if (kb < nkb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kb * 16 + lg * 4 + i;
            const float sv = key < nkeys ? s[kb][qb][i] * kLog2e : -INFINITY;
            s[kb][qb][i] = sv;
            cmax = fmaxf(cmax, sv);
          }
        }
      }
      cmax = fmaxf(cmax, __shfl_xor(cmax, 16, kWave));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 32, kWave));
      const float mnew = fmaxf(mrun[qb], cmax);
      const float alpha = exp2f(mrun[qb] - mnew);
      mrun[qb] = mnew;
      float psum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 8; ++kb) {
        if (kb < nkb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const _Float16 ph = static_cast<_Float16>(exp2f(s[kb][qb][i] - mnew));
            pv[kb][qb][i] = ph;
            psum += static_cast<float>(ph);
          }
        }
      }
      lrun[qb] = lrun[qb] * alpha + psum;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[qb][db] *= alpha;
    }

    // O^T += V^T P^T over key-block pairs.
#pragma unroll
    for (int kp = 0; kp < 4; ++kp) {
      if (2 * kp < nkb) {
        f16x8 pf[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const f16x4 a = pv[2 * kp][qb];
          const f16x4 b = (2 * kp + 1 < nkb) ? pv[2 * kp + 1][qb] : f16x4{0, 0, 0, 0};
          pf[qb] = f16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        }
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const uint8_t* vr = sVt + (db * 16 + lr) * kVPitch;
          const f16x4 va = *reinterpret_cast<const f16x4*>(vr + ((2 * kp) * 16 + lg * 4) * 2);
          const f16x4 vb = *reinterpret_cast<const f16x4*>(vr + ((2 * kp + 1) * 16 + lg * 4) * 2);
          const f16x8 vf = f16x8{va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
            o[qb][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[qb], o[qb][db], 0, 0, 0);
        }
      }
    }
  }

  if (!active) return;
  float amax = 0.f;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float lt = lrun[qb];
    lt += __shfl_xor(lt, 16, kWave);
    lt += __shfl_xor(lt, 32, kWave);
    const float inv = 1.0f / lt;
    const int qi = qbase + qb * 16 + lr;
    if (qi < L) {
      float* orow = out + static_cast<size_t>(start + qi) * ld_out + hoff + lg * 4;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const float4 r = make_float4(o[qb][db][0] * inv, o[qb][db][1] * inv,
                                     o[qb][db][2] * inv, o[qb][db][3] * inv);
        *reinterpret_cast<float4*>(orow + db * 16) = r;
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(r.x), fabsf(r.y)), fmaxf(fabsf(r.z), fabsf(r.w))));
      }
    }
  }
  if (tensor_absmax) {
    amax = wave_max(amax);
    if (lane == 0) atomic_max_nonneg(tensor_absmax, amax);
  }
}

// ---- Split-fp16 MFMA path (head_dim 64): fp32 accuracy on fp16 MFMA.
//
// Every operand is split into hi + lo fp16 parts (hi = fp16(x), lo =
// fp16(x - hi): 22 significant bits together), written by the QKV GEMM
// epilogue after RoPE (or by launch_pack_x3 for the op-level entry), and each
// product uses three MFMAs: hi*hi + lo*hi + hi*lo (the dropped lo*lo term is
// below 2^-22 relative). Q comes multiplied by a power of two (q_prescale) so
// the lo parts of the small pre-scaled Q stay normal fp16; the factor is
// divided back out in the exp2 argument. Q arrives as split words (low half
// hi, high half lo), K and V as separate hi and lo fp16 planes. Within each
// head the 64 positions hold dims in the order 0, 32, 1, 33, ..., 31, 63 (the
// epilogue's rotary pairs side by side); the dot products run over positions,
// and O is written back in natural dim order. S^T = K Q^T puts each lane's
// probabilities in the B-operand layout of O^T = V^T P^T. The running sum
// uses the fp32 probabilities, so the normalisation is that of the
// reference's fp32/double softmax (attention.cpp:118-139).
//
// K and V chunks go straight from global memory into LDS
// (global_load_lds_dwordx4, no registers): each of the four waves loads one
// plane (K hi, K lo, V hi, V lo) of the next 32-key chunk while the current
// one is computed, into the other of two 16 KB buffers. 32 KB of LDS and
// about 125 VGPRs per workgroup let four workgroups share a CU (64-key
// chunks: two, and 8% / 12% slower at configurations 4 / 5). Plane rows are 128
// bytes, their 16-byte chunks stored at chunk ^ swizzle(row): (row / 2) % 8
// for K, whose fragment reads take one chunk of 16 consecutive rows, and
// 2 ((row / 2) % 4) for V, whose transposing reads (below) take two chunks of
// 8 consecutive rows; both read patterns then touch distinct LDS banks.
constexpr int KCX = 32;  // keys per LDS chunk
static_assert(KCX % 32 == 0, "the PV loop takes 32-key pairs of 16-key blocks");
constexpr int kPlaneBytes = KCX * 128;     // one plane of a chunk
constexpr int kChunkBytes = 4 * kPlaneBytes;
static_assert(2 * kChunkBytes >= 4 * 8192, "each wave's 32 x 64 fp32 output tile fits in the chunk buffers");

__device__ __forceinline__ int swz_k(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int swz_v(int row) { return 2 * ((row >> 1) & 3); }

// One 16-byte-per-lane global -> LDS load: a wave-uniform global base plus a
// 32-bit lane offset, into the wave-uniform LDS byte address lds (M0).
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, uint32_t lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0v)
               : "memory", "m0");
#endif
}

__device__ __forceinline__ uint32_t lds_byte_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

// Low (sel_lo) or high (sel_hi) 16-bit halves of two words, packed: the hi
// or lo fp16 parts of two consecutive values.
constexpr uint32_t kSelLo = 0x05040100u, kSelHi = 0x07060302u;
__device__ __forceinline__ uint32_t halves(uint32_t first, uint32_t second, uint32_t sel) {
  return __builtin_amdgcn_perm(second, first, sel);
}

// ds_read_b64_tr_b16 of the 8 bytes at LDS address p (8-byte aligned).
// Within each group of 16 lanes, lane i receives element i % 4 of the 8-byte
// rows read by lanes i / 4, i / 4 + 4, i / 4 + 8 and i / 4 + 12 (layout
// checked on the device). So when lane s of a group reads key s / 4 of a
// 4-key quad at positions 4 (s % 4) .. + 4 of a row-major V tile, lane i gets
// position i of the quad's four keys: the PV operand, read from rows.
__device__ __forceinline__ f16x4 lds_read_tr16(const uint8_t* p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((__attribute__((address_space(3))) uint8_t*)p));
  return __builtin_bit_cast(f16x4, v);
}

__device__ __forceinline__ f32x4 mma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 8 split words -> f16x8 hi and lo parts.
__device__ __forceinline__ void unpack8(const uint4& a, const uint4& b, f16x8* hi, f16x8* lo) {
  const uint32_t h[4] = {halves(a.x, a.y, kSelLo), halves(a.z, a.w, kSelLo), halves(b.x, b.y, kSelLo),
                         halves(b.z, b.w, kSelLo)};
  const uint32_t l[4] = {halves(a.x, a.y, kSelHi), halves(a.z, a.w, kSelHi), halves(b.x, b.y, kSelHi),
                         halves(b.z, b.w, kSelHi)};
  *hi = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(h));
  *lo = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(l));
}

// a * b rounded on its own: the product is never fused into a later add.
__device__ __forceinline__ float mul_unfused(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

// Raw v_exp_f32: 2^x for results >= 2^-126 exactly as exp2f, 0 below (the
// library's exp2f adds a rescale for subnormal results; probabilities under
// 2^-126 of the row maximum do not change an fp32 softmax sum).
__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }

// Eight probabilities as split-fp16 operands: hi = fp16(p), lo = fp16(p - hi)
// (the split of split_f16_word, in split_pair's packed form).
__device__ __forceinline__ void split8(const float (&p)[8], f16x8* hi, f16x8* lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) split_pair(p[2 * j], p[2 * j + 1], &h[j], &l[j]);
  *hi = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(h));
  *lo = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(l));
}

// LONG: the variant for batches with sequences past 256 tokens, whose many
// key chunks per work item make the chunk loop's VALU work count: O and the
// running sum are rescaled only when some lane's running maximum moved (else
// alpha = exp2(0) = 1 exactly, so skipping it changes no bit). Short-sequence
// batches keep the unconditional rescale: there the leaner loop ran as fast
// in isolation, but beside the second sequence group's kernels the
// configuration-4 forward got 1% slower.
template <bool LONG>
__global__ __launch_bounds__(256, 4) void attn_x3_kernel(
    const uint32_t* __restrict__ q, int ldq, const uint16_t* __restrict__ kh, const uint16_t* __restrict__ kl,
    const uint16_t* __restrict__ vh, const uint16_t* __restrict__ vl, int ldp, float s2, const int* __restrict__ cu,
    const AttnWork* __restrict__ work, float* __restrict__ out, int ld_out, float* __restrict__ part_max) {
  // Two chunk buffers, each [K hi | K lo | V hi | V lo] planes of 64 rows x
  // 128 bytes.
  __shared__ __attribute__((aligned(1024))) uint8_t sbuf[2 * kChunkBytes];

  const AttnWork w = work[blockIdx.x];
  const int start = cu[w.seq];
  const int L = cu[w.seq + 1] - start;
  // part_max (optional): slot 4 * item + wave receives the largest |output|
  // the wave stores (0 for a wave or item with no queries).
  if (w.q0 >= L) {  // padding item of the work list (uniform)
    if (part_max && threadIdx.x < 4) part_max[blockIdx.x * 4 + threadIdx.x] = 0.0f;
    return;
  }
  const int hoff = w.head * 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int qbase = w.q0 + wave * 32;
  const bool active = qbase < L;  // wave-uniform

  // Chunk loads: wave p moves plane p (K hi, K lo, V hi, V lo) as eight 1 KB
  // blocks of 8 rows; lane j of block rg fills row 8 rg + j / 8 at slot j % 8
  // with that row's chunk slot ^ swizzle(row). Rows past the sequence repeat
  // its last key (their scores are masked to -inf, so their probabilities are
  // exactly 0).
  const uint16_t* const plane = wave == 0 ? kh : wave == 1 ? kl : wave == 2 ? vh : vl;
  const uint32_t ldpb = static_cast<uint32_t>(ldp) * 2u;  // plane row pitch in bytes
  const int drow = lane >> 3, dslot = lane & 7;
  const uint32_t lds0 = lds_byte_addr(sbuf) + static_cast<uint32_t>(wave * kPlaneBytes);
  auto load_chunk = [&](int kc, int buf) {
    const int nk = min(KCX, L - kc);
    const char* base = reinterpret_cast<const char*>(plane + static_cast<size_t>(start + kc) * ldp + hoff);
#pragma unroll
    for (int rg = 0; rg < KCX / 8; ++rg) {
      const int row = rg * 8 + drow;
      const int c = dslot ^ (wave < 2 ? swz_k(row) : swz_v(row));
      lds_dma16(base, static_cast<uint32_t>(min(row, nk - 1)) * ldpb + static_cast<uint32_t>(c * 16),
                lds0 + static_cast<uint32_t>(buf * kChunkBytes + rg * 1024));
    }
  };

  // Q fragments (B operand of S^T = K Q^T): lane (lr, lg) holds query lr of
  // block qb, positions [lg*8, lg*8+8) and [32+lg*8, 32+lg*8+8). The Q words
  // are loaded first and chunk 0 right behind them, so both round trips
  // overlap.
  uint4 qw[2][2][2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qi = min(qbase + qb * 16 + lr, L - 1);
    const uint32_t* qp = q + static_cast<size_t>(start + qi) * ldq + hoff;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      qw[qb][half][0] = *reinterpret_cast<const uint4*>(qp + half * 32 + lg * 8);
      qw[qb][half][1] = *reinterpret_cast<const uint4*>(qp + half * 32 + lg * 8 + 4);
    }
  }
  load_chunk(0, 0);
  f16x8 qh[2][2], ql[2][2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int half = 0; half < 2; ++half) unpack8(qw[qb][half][0], qw[qb][half][1], &qh[qb][half], &ql[qb][half]);

  f32x4 o[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int db = 0; db < 4; ++db) o[qb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mrun[2] = {-INFINITY, -INFINITY};
  float lrun[2] = {0.f, 0.f};

  // Fragment offsets inside a plane. K: row kb*16 + lr, chunks lg and 4 + lg
  // (kb*16 leaves the swizzle unchanged). V (transposing reads): row
  // (2kp)*16 + lg*4 + lr/4 (+16 for the pair's second block, same swizzle),
  // positions db*16 + 4 (lr % 4): chunk 2 db + (lr % 4) / 2, half lr % 2.
  const int koff0 = lr * 128 + ((lg ^ swz_k(lr)) << 4);
  const int koff1 = lr * 128 + (((4 + lg) ^ swz_k(lr)) << 4);
  const int vrow = lg * 4 + (lr >> 2);
  const int vsw = swz_v(vrow);
  const int vbase = vrow * 128 + ((lr & 1) << 3);
  const int vc = (lr & 3) >> 1;

  // One chunk of keys from buffer buf; FULLC: all KCX keys are valid (every
  // chunk but the last of a sequence whose length is not a multiple of KCX),
  // so no key needs masking.
  auto chunk = [&](int kc0, int nkeys, int buf, auto fullc_tag) {
    constexpr bool FULLC = decltype(fullc_tag)::value;
    // This wave's loads of the chunk have landed; the barrier publishes
    // everyone's and retires the previous chunk's reads of the other buffer,
    // which then receives the next chunk, in flight during this one.
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (kc0 + KCX < L) load_chunk(kc0 + KCX, buf ^ 1);
    if (!active) return;
    const uint8_t* sKh = sbuf + buf * kChunkBytes;
    const uint8_t* sKl = sKh + kPlaneBytes;
    const uint8_t* sVh = sKh + 2 * kPlaneBytes;
    const uint8_t* sVl = sKh + 3 * kPlaneBytes;

    const int nkb = FULLC ? KCX / 16 : (nkeys + 15) >> 4;
    f32x4 s[KCX / 16][2];
#pragma unroll
    for (int kb = 0; kb < KCX / 16; ++kb) {
      if (kb < nkb) {
        const f16x8 kh0 = *reinterpret_cast<const f16x8*>(sKh + kb * 2048 + koff0);
        const f16x8 kh1 = *reinterpret_cast<const f16x8*>(sKh + kb * 2048 + koff1);
        const f16x8 kl0 = *reinterpret_cast<const f16x8*>(sKl + kb * 2048 + koff0);
        const f16x8 kl1 = *reinterpret_cast<const f16x8*>(sKl + kb * 2048 + koff1);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          f32x4 acc = mma16(kh0, qh[qb][0], f32x4{0.f, 0.f, 0.f, 0.f});
          acc = mma16(kl0, qh[qb][0], acc);
          acc = mma16(kh0, ql[qb][0], acc);
          acc = mma16(kh1, qh[qb][1], acc);
          acc = mma16(kl1, qh[qb][1], acc);
          s[kb][qb] = mma16(kh1, ql[qb][1], acc);
        }
      }
    }

    // Online softmax in base 2; lane holds keys kb*16 + 4*lg + i. The
    // running max and the rescale of O happen first; the probabilities are
    // then formed, summed and split per key-block pair inside the PV loop, so
    // only one pair's fp16 fragments are live at a time.
    float mnew[2], al[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      float cmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < KCX / 16; ++kb) {
        if (kb < nkb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kb * 16 + lg * 4 + i;
            // The scaled score is rounded once (no fused multiply-add with
            // the exponent's subtraction, which the compiler would form only
            // in some instantiations): the row's largest probability is then
            // exp2(0) = 1 exactly, and every variant rounds alike.
            const float sv = (FULLC || key < nkeys) ? mul_unfused(s[kb][qb][i], s2) : -INFINITY;
            s[kb][qb][i] = sv;
            cmax = fmaxf(cmax, sv);
          }
        }
      }
      cmax = fmaxf(cmax, __shfl_xor(cmax, 16, kWave));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 32, kWave));
      mnew[qb] = fmaxf(mrun[qb], cmax);
      // The running sum takes its rescale in one fused step with the chunk's
      // first probabilities, lrun = fma(lrun, alpha, psum), in both variants,
      // so that skipping the rescale (alpha = 1: fma(lrun, 1, psum) is the
      // rounded sum) changes no bit.
      al[qb] = 1.0f;
      if (!LONG || __builtin_amdgcn_ballot_w64(mnew[qb] != mrun[qb]) != 0) {
        const float alpha = exp2_raw(mrun[qb] - mnew[qb]);
        al[qb] = alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[qb][db] *= alpha;
      }
      mrun[qb] = mnew[qb];
    }

    // O^T += V^T P^T over key-block pairs, three MFMAs per product.
#pragma unroll
    for (int kp = 0; kp < KCX / 32; ++kp) {
      if (2 * kp < nkb) {
        f16x8 pfh[2], pfl[2];
        const bool two = FULLC || 2 * kp + 1 < nkb;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          float pr[8];
          float psum = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int kb = 2 * kp + (j >> 2);
            pr[j] = (j < 4 || two) ? exp2_raw(s[kb][qb][j & 3] - mnew[qb]) : 0.f;
            psum += pr[j];
          }
          split8(pr, &pfh[qb], &pfl[qb]);
          lrun[qb] = kp == 0 ? __builtin_fmaf(lrun[qb], al[qb], psum) : lrun[qb] + psum;
        }
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          // Lane (lr, lg) gets position db*16 + lr of keys (2kp)*16 + lg*4
          // .. +4 (ca) and (2kp+1)*16 + lg*4 .. +4 (cb).
          const int ca = kp * 4096 + vbase + (((2 * db + vc) ^ vsw) << 4);
          const int cb = ca + 2048;
          const f16x4 vah = lds_read_tr16(sVh + ca);
          const f16x4 vbh = lds_read_tr16(sVh + cb);
          const f16x4 val = lds_read_tr16(sVl + ca);
          const f16x4 vbl = lds_read_tr16(sVl + cb);
          const f16x8 vfh = f16x8{vah[0], vah[1], vah[2], vah[3], vbh[0], vbh[1], vbh[2], vbh[3]};
          const f16x8 vfl = f16x8{val[0], val[1], val[2], val[3], vbl[0], vbl[1], vbl[2], vbl[3]};
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            f32x4 acc = mma16(vfh, pfh[qb], o[qb][db]);
            acc = mma16(vfl, pfh[qb], acc);
            o[qb][db] = mma16(vfh, pfl[qb], acc);
          }
        }
      }
    }
  };

  // Whole chunks, then the sequence's partial last chunk (if any).
  int kc0 = 0, buf = 0;
  for (; kc0 + KCX <= L; kc0 += KCX, buf ^= 1) chunk(kc0, KCX, buf, std::true_type{});
  if (kc0 < L) {
    chunk(kc0, L - kc0, buf, std::false_type{});
    buf ^= 1;
  }

  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // every wave is done with the chunks
  if (!active) {
    if (part_max && lane == 0) part_max[blockIdx.x * 4 + wave] = 0.0f;
    return;
  }
  // Output: rows of o[qb][db] are positions db*16 + 4 lg .. +4, i.e. dims i,
  // i + 32, i + 1, i + 33 for i = 8 db + 2 lg. Each wave puts its 32 x 64
  // tile in natural order into its own 8 KB of the chunk buffers (free after
  // the barrier above), 256-byte rows with 16-byte unit u at u ^ (row % 16),
  // then stores whole rows: 16 lanes x 16 bytes per query.
  uint8_t* stage = sbuf + wave * 8192;
  auto soff = [](int row, int dim) { return row * 256 + (((dim >> 2) ^ (row & 15)) << 4) + ((dim & 3) << 2); };
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float lt = lrun[qb];
    lt += __shfl_xor(lt, 16, kWave);
    lt += __shfl_xor(lt, 32, kWave);
    const float inv = 1.0f / lt;
    const int row = qb * 16 + lr;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int i = 8 * db + 2 * lg;
      *reinterpret_cast<float2*>(stage + soff(row, i)) = make_float2(o[qb][db][0] * inv, o[qb][db][2] * inv);
      *reinterpret_cast<float2*>(stage + soff(row, i + 32)) = make_float2(o[qb][db][1] * inv, o[qb][db][3] * inv);
    }
  }
  const int unit = lane & 15;
  float m = 0.0f;
#pragma unroll
  for (int r4 = 0; r4 < 8; ++r4) {
    const int row = r4 * 4 + (lane >> 4);
    const float4 val = *reinterpret_cast<const float4*>(stage + soff(row, unit * 4));
    const int qi = qbase + row;
    if (qi < L) {
      *reinterpret_cast<float4*>(out + static_cast<size_t>(start + qi) * ld_out + hoff + unit * 4) = val;
      if (part_max) m = fmaxf(m, fmaxf(fmaxf(fabsf(val.x), fabsf(val.y)), fmaxf(fabsf(val.z), fabsf(val.w))));
    }
  }
  if (part_max) {
    m = wave_max(m);
    if (lane == 0) part_max[blockIdx.x * 4 + wave] = m;
  }
}

// fp32 rows -> the split-fp16 kernel's operand layout (head_dim 64, positions
// 0, 32, 1, 33, ... within each head): planes == 0, split words (x * scale)
// at out_w[r * ld_out + c]; planes != 0, fp16 hi parts at out_h[r * ld_out +
// c] and lo parts d elements further.
__global__ void pack_x3_kernel(const float* __restrict__ x, int ld_x, int rows, int d, float scale, int planes,
                               uint32_t* __restrict__ out_w, uint16_t* __restrict__ out_h, int ld_out) {
  const size_t total = static_cast<size_t>(rows) * d;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t r = i / d;
    const int c = static_cast<int>(i % d);
    const int pos = c & 63, dim = (c & ~63) + (pos >> 1) + ((pos & 1) << 5);
    const uint32_t wv = split_f16_word(x[r * ld_x + dim] * scale);
    if (planes) {
      out_h[r * ld_out + c] = static_cast<uint16_t>(wv & 0xffffu);
      out_h[r * ld_out + d + c] = static_cast<uint16_t>(wv >> 16);
    } else {
      out_w[r * ld_out + c] = wv;
    }
  }
}

template <int DH_MAX>
__global__ __launch_bounds__(64) void attn_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, int ld, int dh, const int* __restrict__ cu,
    const AttnWork* __restrict__ work, float* __restrict__ out, int ld_out) {
  const AttnWork w = work[blockIdx.x];
  const int start = cu[w.seq];
  const int L = cu[w.seq + 1] - start;
  const int hoff = w.head * dh;
  const int qi = w.q0 + static_cast<int>(threadIdx.x);
  const bool valid = qi < L;
  const int qc = valid ? qi : L - 1;

  float qr[DH_MAX];
  const float* qp = q + static_cast<size_t>(start + qc) * ld + hoff;
#pragma unroll
  for (int d = 0; d < DH_MAX; ++d) qr[d] = d < dh ? qp[d] : 0.f;

  float mx = -INFINITY;
  for (int j = 0; j < L; ++j) {
    const float* kp = k + static_cast<size_t>(start + j) * ld + hoff;
    float dot = 0.f;
#pragma unroll
    for (int d = 0; d < DH_MAX; ++d)
      if (d < dh) dot += qr[d] * kp[d];
    mx = fmaxf(mx, dot);
  }
  double sum = 0.0;
  float acc[DH_MAX];
#pragma unroll
  for (int d = 0; d < DH_MAX; ++d) acc[d] = 0.f;
  for (int j = 0; j < L; ++j) {
    const float* kp = k + static_cast<size_t>(start + j) * ld + hoff;
    float dot = 0.f;
#pragma unroll
    for (int d = 0; d < DH_MAX; ++d)
      if (d < dh) dot += qr[d] * kp[d];
    const float e = expf(dot - mx);
    sum += e;
    const float* vp = v + static_cast<size_t>(start + j) * ld + hoff;
#pragma unroll
    for (int d = 0; d < DH_MAX; ++d)
      if (d < dh) acc[d] += e * vp[d];
  }
  if (!valid) return;
  const float inv = sum > 0.0 ? static_cast<float>(1.0 / sum) : 0.f;
  float* orow = out + static_cast<size_t>(start + qi) * ld_out + hoff;
#pragma unroll
  for (int d = 0; d < DH_MAX; ++d)
    if (d < dh) orow[d] = acc[d] * inv;
}

}  // namespace

hipError_t launch_attention_mfma(const uint16_t* q, const uint16_t* k,
                                 const uint16_t* v, int qk_is_fp16, int v_is_bf16,
                                 int ld, const int* cu_seqlens,
                                 const AttnWork* work, int num_work, float* out,
                                 int ld_out, float* tensor_absmax,
                                 hipStream_t s) {
  if (num_work <= 0) return hipSuccess;
  const dim3 grid(num_work), block(256);
#define ESM_ATTN_LAUNCH(QF, VB)                                                  \
  hipLaunchKernelGGL((attn_mfma_kernel<QF, VB>), grid, block, 0, s, q, k, v, ld, \
                     cu_seqlens, work, out, ld_out, tensor_absmax)
  if (qk_is_fp16) {
    if (v_is_bf16) ESM_ATTN_LAUNCH(true, true); else ESM_ATTN_LAUNCH(true, false);
  } else {
    if (v_is_bf16) ESM_ATTN_LAUNCH(false, true); else ESM_ATTN_LAUNCH(false, false);
  }
#undef ESM_ATTN_LAUNCH
  return hipGetLastError();
}

hipError_t launch_attention_x3(const uint32_t* q, int ldq, const uint16_t* kh, const uint16_t* kl, const uint16_t* vh,
                               const uint16_t* vl, int ldp, float q_prescale, const int* cu_seqlens,
                               const AttnWork* work, int num_work, float* out, int ld_out, int max_len,
                               hipStream_t s, float* part_max) {
  if (num_work <= 0) return hipSuccess;
  const float s2 = kLog2e / q_prescale;
  if (max_len > kAttnLongSeq)
    hipLaunchKernelGGL(attn_x3_kernel<true>, dim3(num_work), dim3(256), 0, s, q, ldq, kh, kl, vh, vl, ldp, s2,
                       cu_seqlens, work, out, ld_out, part_max);
  else
    hipLaunchKernelGGL(attn_x3_kernel<false>, dim3(num_work), dim3(256), 0, s, q, ldq, kh, kl, vh, vl, ldp, s2,
                       cu_seqlens, work, out, ld_out, part_max);
  return hipGetLastError();
}

hipError_t launch_pack_x3(const float* x, int ld_x, int rows, int d, float scale, uint32_t* words, uint16_t* planes,
                          int ld_out, hipStream_t s) {
  const size_t n = static_cast<size_t>(rows) * d;
  if (n == 0) return hipSuccess;
  if (d % 64 != 0 || (words == nullptr) == (planes == nullptr)) return hipErrorInvalidValue;
  size_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  hipLaunchKernelGGL(pack_x3_kernel, dim3(static_cast<unsigned>(g)), dim3(256), 0, s, x, ld_x, rows, d, scale,
                     planes ? 1 : 0, words, planes, ld_out);
  return hipGetLastError();
}

hipError_t launch_attention_f32(const float* q, const float* k, const float* v,
                                int ld, int head_dim, const int* cu_seqlens,
                                const AttnWork* work, int num_work, float* out,
                                int ld_out, hipStream_t s) {
  if (num_work <= 0) return hipSuccess;
  const dim3 grid(num_work), block(64);
  if (head_dim <= 16) {
    hipLaunchKernelGGL(attn_f32_kernel<16>, grid, block, 0, s, q, k, v, ld, head_dim, cu_seqlens, work, out, ld_out);
  } else if (head_dim <= 32) {
    hipLaunchKernelGGL(attn_f32_kernel<32>, grid, block, 0, s, q, k, v, ld, head_dim, cu_seqlens, work, out, ld_out);
  } else if (head_dim <= 64) {
    hipLaunchKernelGGL(attn_f32_kernel<64>, grid, block, 0, s, q, k, v, ld, head_dim, cu_seqlens, work, out, ld_out);
  } else if (head_dim <= 128) {
    hipLaunchKernelGGL(attn_f32_kernel<128>, grid, block, 0, s, q, k, v, ld, head_dim, cu_seqlens, work, out, ld_out);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace esm_gfx950
