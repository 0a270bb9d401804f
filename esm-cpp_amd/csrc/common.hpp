// Shared device helpers for the gfx950 (CDNA4) backend of the packed ESM-2
// encoder path: vector types for the MFMA builtins, bf16/fp16 conversions,
// wave-level reductions and the launch-error plumbing used by every kernel
// translation unit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace esm_gfx950 {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

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

// Non-negative IEEE floats order like their bit patterns, so an unsigned
// atomic max on the bits is a float max (used for absmax reductions).
__device__ __forceinline__ void atomic_max_nonneg(float* addr, float v) {
  atomicMax(reinterpret_cast<unsigned int*>(addr), __float_as_uint(v));
}

// Exact-erf GELU: x * 0.5 * (1 + erf(x / sqrt(2))). erff is the HIP
// device library's erf.
__device__ __forceinline__ float gelu_erf(float x) {
  return x * 0.5f * (1.0f + erff(x * 0.70710678118654752440f));
}

// Symmetric int8 quantisation of one value with a precomputed reciprocal
// scale: clamp(rne(x * inv), -127, 127).
__device__ __forceinline__ int quant_i8(float x, float inv) {
  float r = __builtin_rintf(x * inv);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return static_cast<int>(r);
}

}  // namespace esm_gfx950
