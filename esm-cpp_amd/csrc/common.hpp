// Shared device helpers for the gfx950 (CDNA4) backend of the packed ESM-2
// encoder path: vector types for the MFMA builtins, bf16/fp16 conversions,
// wave-level reductions and the launch-error plumbing used by every kernel
// translation unit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace esm_gfx950 {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet). Matches the
// usual RNE definition used by torch and by the CPU oracle.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
    return static_cast<uint16_t>((u >> 16) | 0x40u);
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

// Butterfly reductions over a full 64-lane wave.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Split-fp16 word: fp16(x) in the low half, fp16(x - fp16(x)) in the high
// half. x - fp16(x) is exact in fp32, so hi + lo keeps 22 significant bits of
// x (lo is subnormal when |x| < 2^-3, i.e. absolute error <= 2^-25 there).
__device__ __forceinline__ uint32_t split_f16_word(float x) {
  // hi = fp16(x) into the low half (v_cvt_f16_f32), then lo = fp16(x - hi)
  // into the high half (v_fma_mixhi_f16 reads hi as fp16; x - hi is exact in
  // fp32, so its single rounding equals convert-subtract-convert). Written
  // out so that every caller rounds x itself, never a wider intermediate the
  // compiler could fuse into the conversion.
  uint32_t w;
  asm("v_cvt_f16_f32 %0, %1\n\tv_fma_mixhi_f16 %0, -%0, 1.0, %1 op_sel_hi:[1,0,0]" : "=&v"(w) : "v"(x));
  return w;
}

// Split-fp16 parts of two values as two words: hi = (fp16(p0), fp16(p1)) and
// lo = (fp16(p0 - hi0), fp16(p1 - hi1)), each the low / high half.
__device__ __forceinline__ void split_pair(float p0, float p1, uint32_t* hi, uint32_t* lo) {
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{p0, p1}, f16x2));
  uint32_t l;  // high half written by the second instruction
  asm("v_fma_mixlo_f16 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mixhi_f16 %0, -%1, 1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "=&v"(l)
      : "v"(h), "v"(p0), "v"(p1));
  *hi = h;
  *lo = l;
}

// Non-negative IEEE floats order like their bit patterns, so an unsigned
// atomic max on the bits is a float max (used for absmax reductions).
__device__ __forceinline__ void atomic_max_nonneg(float* addr, float v) {
  atomicMax(reinterpret_cast<unsigned int*>(addr), __float_as_uint(v));
}

// atomic_max_nonneg of the maximum of v over a block of WAVES waves: the
// waves' maxima meet in LDS and one lane issues the atomic. Atomics on one
// address serialise in L2, so a launch that sends one per block instead of
// one per wave (and has a bounded grid) spends correspondingly less time on
// them; the maximum itself does not depend on the order. Every thread of the
// block must call it.
template <int WAVES = 4>
__device__ __forceinline__ void block_atomic_max_nonneg(float* addr, float v) {
  __shared__ float s_wave_max[WAVES];
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) s_wave_max[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    float m = s_wave_max[0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) m = fmaxf(m, s_wave_max[w]);
    atomic_max_nonneg(addr, m);
  }
}

// Exact-erf GELU: x * 0.5 * (1 + erf(x / sqrt(2))). erff is the HIP
// device library's erf.
__device__ __forceinline__ float gelu_erf(float x) {
  return x * 0.5f * (1.0f + erff(x * 0.70710678118654752440f));
}

// Twice GELU, with erf from Abramowitz & Stegun, Handbook of Mathematical
// Functions, eq. 7.1.26 (|error of erf| <= 1.5e-7 for every x): erf(u) =
// 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-u^2), t = 1/(1 + p|u|).
// The reference's AVX-512 GELU uses the same approximation (reference
// src/kernels/gelu.cpp:69-94). erf is odd, so 2 gelu(x) = x (1 + erf(x/√2))
// = x + |x| erf(|x|/√2); the 1/√2 is folded into p and the exponent, and the
// final 1/2 is left to the caller (an exact power-of-two scaling). exp(-u^2)
// is the hardware base-2 exponential, which returns 0 (not NaN) for large |u|.
__device__ __forceinline__ float gelu2_as(float x) {
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f * 0.70710678118654752440f, ax, 1.0f));
  float poly = __builtin_fmaf(1.061405429f, t, -1.453152027f);
  poly = __builtin_fmaf(poly, t, 1.421413741f);
  poly = __builtin_fmaf(poly, t, -0.284496736f);
  poly = __builtin_fmaf(poly, t, 0.254829592f);
  poly *= t;
  const float e = __builtin_amdgcn_exp2f((x * x) * (-0.5f * 1.44269504088896340736f));
  const float erf_abs = __builtin_fmaf(-poly, e, 1.0f);
  return __builtin_fmaf(ax, erf_abs, x);
}

// Activation scale rule of the reference prefix (gemm_int8.cpp:434,476):
// absmax/127, or 1 when the input is all zero.
__device__ __forceinline__ float act_scale_from_absmax(float amax) {
  return amax > 0.0f ? amax / 127.0f : 1.0f;
}

// Symmetric int8 quantisation of one value with a precomputed reciprocal
// scale: clamp(rne(x * inv), -127, 127).
__device__ __forceinline__ int quant_i8(float x, float inv) {
  float r = __builtin_rintf(x * inv);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return static_cast<int>(r);
}

// Four values quantised exactly as quant_i8 does, packed little-endian into
// one word. For |r| <= 127, r + 1.5*2^23 lies in [2^23, 2^24), where the
// float spacing is 1, so the addition rounds r to the nearest integer with
// ties to even and the low byte of the sum's bits is that integer in two's
// complement (checked against rint + clamp for every float in [-200, 200]).
__device__ __forceinline__ uint32_t quant_pack4(float4 v, float inv) {
  constexpr float kMagic = 12582912.0f;
  const uint32_t a = __float_as_uint(__builtin_amdgcn_fmed3f(v.x * inv, -127.0f, 127.0f) + kMagic);
  const uint32_t b = __float_as_uint(__builtin_amdgcn_fmed3f(v.y * inv, -127.0f, 127.0f) + kMagic);
  const uint32_t c = __float_as_uint(__builtin_amdgcn_fmed3f(v.z * inv, -127.0f, 127.0f) + kMagic);
  const uint32_t d = __float_as_uint(__builtin_amdgcn_fmed3f(v.w * inv, -127.0f, 127.0f) + kMagic);
  // v_perm_b32 byte k of the result = byte sel[k] of {src0 (bytes 4-7), src1 (bytes 0-3)}.
  const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);  // a.b0, b.b0
  const uint32_t hi = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);  // c.b0, d.b0
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

}  // namespace esm_gfx950
