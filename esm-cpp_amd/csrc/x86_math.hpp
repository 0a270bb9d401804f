// The reference's x86 AVX-512 exp and GELU (ExpAvx512, GeluAvx512), shared
// by the x86-exact kernels and the INT8 GEMM's x86 GELU epilogue. Every
// fused multiply-add of the reference build is written out; each body
// switches contraction off, so these round the same in every translation
// unit whatever its -ffp-contract setting.
#pragma once

#include <stdint.h>

#include <hip/hip_runtime.h>

namespace esm_gfx950 {

// _mm512_cvtps_epi32 of an integral float: out of range gives 0x80000000.
__device__ __forceinline__ int32_t cvt_i32_x86(float x) {
  return (x > -2147483648.0f && x < 2147483648.0f) ? static_cast<int32_t>(x) : INT32_MIN;
}

// ExpAvx512 / ExpAvx512Attn (reference src/kernels/gelu.cpp:40-68,
// src/kernels/attention.cpp:156-175): n = rne(x * log2e), r = x - n*ln2_hi
// - n*ln2_lo (both fused, as the reference build contracts them), 5-term
// Horner polynomial, times the float whose exponent bits are n + 127 (the
// shift wraps for n < -127, as the reference's does).
__device__ __forceinline__ float exp_x86(float x) {
#pragma clang fp contract(off)
  const float n = __builtin_rintf(x * 1.44269504088896340736f);
  const float r = __builtin_fmaf(-n, 1.42860677e-6f, __builtin_fmaf(-n, 6.93145752e-1f, x));
  float p = 1.0f / 120.0f;
  p = __builtin_fmaf(p, r, 1.0f / 24.0f);
  p = __builtin_fmaf(p, r, 1.0f / 6.0f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const uint32_t e = static_cast<uint32_t>(cvt_i32_x86(n) + 127) << 23;
  return p * __uint_as_float(e);
}

// GeluAvx512 / ErfAvx512 (reference src/kernels/gelu.cpp:74-148): erf from
// Abramowitz & Stegun 7.1.26 with exp_x86, sign restored by OR;
// gelu = (v * 0.5) * (1 + erf(v * (1/sqrt 2))).
__device__ __forceinline__ float gelu_x86(float v) {
#pragma clang fp contract(off)
  const float x = v * 0.70710678118654752440f;
  const uint32_t sign = __float_as_uint(x) & 0x80000000u;
  const float ax = __uint_as_float(__float_as_uint(x) & 0x7fffffffu);
  const float t = static_cast<float>(1.0 / static_cast<double>(__builtin_fmaf(0.3275911f, ax, 1.0f)));
  float poly = 1.061405429f;
  poly = __builtin_fmaf(poly, t, -1.453152027f);
  poly = __builtin_fmaf(poly, t, 1.421413741f);
  poly = __builtin_fmaf(poly, t, -0.284496736f);
  poly = __builtin_fmaf(poly, t, 0.254829592f);
  poly = poly * t;
  const float xx = x * x;
  const float e = exp_x86(0.0f - xx);
  const float erf = __uint_as_float(__float_as_uint(__builtin_fmaf(-poly, e, 1.0f)) | sign);
  const float h = v * 0.5f;
  return h * (1.0f + erf);
}

}  // namespace esm_gfx950
