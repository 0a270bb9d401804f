// Kernels that reproduce the reference's x86 AVX-512 CPU path bit for bit:
// the kernels its facade selects for Isa::Avx512 / Avx512Vnni / Amx
// (reference src/kernels/dispatch.cpp). Together with the INT8 GEMM's plain
// dequant epilogue (LinearVnni's FinalizeStore16 expression) and per-tensor
// activation scales they make the packed forward's logits equal, bit for
// bit, to the reference's ForwardPackedInto on an AVX-512-VNNI host.
//
// Bit-exactness needs the reference's operation order, lane by lane:
//   - _mm512_reduce_add_ps as GCC 11 defines it (avx512fintrin.h): lanes
//     8..15 added to 0..7, 4..7 to 0..3, then a [2,3,0,1] shuffle-add, then
//     lane 0 + lane 1 (red16 / red16_lanes below);
//   - every fused multiply-add the reference build executes, explicit here:
//     its _mm512_fmadd_ps / _mm512_fnmadd_ps, plus the products GCC contracts
//     (-ffp-contract=fast, its default) in ExpAvx512's range reduction and in
//     LayerNormAvx512's var * (1/d) + eps;
//   - this translation unit is compiled with -ffp-contract=off so the
//     compiler forms no others;
//   - IEEE division and square root, taken in double and rounded once to
//     float (correctly rounded: double carries more than 2 * 24 + 2 bits);
//   - std::exp on the attention's last L % 16 keys is glibc's expf, restated
//     from its published algorithm (expf_glibc below).
#include <math.h>

#include "common.hpp"
#include "kernels.hpp"
#include "x86_math.hpp"

namespace esm_gfx950 {
namespace {

// _mm512_reduce_add_ps (GCC 11) of 16 values held by one thread.
__device__ __forceinline__ float red16(const float (&v)[16]) {
  float t3[8], t6[4];
#pragma unroll
  for (int j = 0; j < 8; ++j) t3[j] = v[8 + j] + v[j];
#pragma unroll
  for (int j = 0; j < 4; ++j) t6[j] = t3[4 + j] + t3[j];
  const float a = t6[0] + t6[2];
  const float b = t6[1] + t6[3];
  return a + b;
}

// The same sum of v held by lanes 0..15 of each 16-lane group (every lane of
// the group gets the result). IEEE addition is commutative, so lane j and
// lane j ^ m forming a + b and b + a agree bit for bit.
__device__ __forceinline__ float red16_lanes(float v) {
  const float t3 = v + __shfl_xor(v, 8, 16);
  const float t6 = t3 + __shfl_xor(t3, 4, 16);
  const float t8 = t6 + __shfl_xor(t6, 2, 16);
  return t8 + __shfl_xor(t8, 1, 16);
}

// glibc's expf (the std::exp of the reference's x86 attention on its last
// L % 16 keys, src/kernels/attention.cpp:376-381), restated from its
// published algorithm (ARM optimized-routines, in glibc since 2.27; the
// x86_64 build runs its FMA variant): x * 32/ln2 = k + r with k rounded to
// nearest, exp(x) = 2^(k/32) * P(r) with P cubic, all in double, rounded
// once to float. T[i] = bits(2^(i/32)) - (i << 47). Equal to glibc 2.35's
// expf on every float in [-inf, 89] (checked exhaustively on the host).
__constant__ uint64_t kExp2Table[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

__device__ __forceinline__ float expf_glibc(float x) {
  const uint32_t ux = __float_as_uint(x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= (0x42b00000u >> 20)) {  // |x| >= 88, inf or nan
    if (ux == 0xff800000u) return 0.0f;
    if (abstop >= (0x7f800000u >> 20)) return x + x;
    if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
  constexpr double kShift = 0x1.8p+52;
  constexpr double kC0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const double xd = static_cast<double>(x);
  double kd = __builtin_fma(kInvLn2N, xd, kShift);
  const uint64_t ki = __double_as_longlong(kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  const uint64_t t = kExp2Table[ki % 32] + (ki << 47);
  const double s = __longlong_as_double(t);
  const double z = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  return static_cast<float>(y * s);
}

// ------------------------------------------------------------ LayerNorm
// LayerNormAvx512 (reference src/kernels/layernorm.cpp:59-149), one wave per
// row. Lane l accumulates the reference's lane l % 16 of accumulator l / 16
// over the row's 64-element blocks (the same elements, in the same order);
// leftover 16-element blocks go to accumulator 0 (lanes 0..15), the last
// d % 16 elements into a scalar sum. With resid, hidden += resid first
// (ResidualAddInplace, written back). absmax (optional): atomic max of
// |out| for the per-tensor activation scale, one atomic per block (the
// waves walk rows grid-stride, so a launch sends at most one per block of its
// bounded grid). round16: the output rounded to fp16 and back
// (RoundToFp16Inplace, reference src/model.cpp:912-930).
template <int NB>
__global__ __launch_bounds__(256) void layernorm_x86_kernel(float* __restrict__ x, const float* __restrict__ resid,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta, float eps,
                                                             float* __restrict__ out, int rows, int d,
                                                             float* __restrict__ absmax, int round16) {
  const int lane = threadIdx.x & 63;
  float m = 0.0f;
  for (int row = blockIdx.x * 4 + (threadIdx.x >> 6); row < rows; row += gridDim.x * 4) {
    float* xr = x + static_cast<size_t>(row) * d;
    const float* rr = resid ? resid + static_cast<size_t>(row) * d : nullptr;
    const int nfull = d >> 6;
    const int rem = d - (nfull << 6);
    const int rem16 = rem >> 4;
    const int tail = rem & 15;
    float xv[NB];
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      if (t < nfull) {
        float v = xr[(t << 6) + lane];
        if (rr) {
          v = v + rr[(t << 6) + lane];
          xr[(t << 6) + lane] = v;
        }
        xv[t] = v;
      }
    }
    float xrem = 0.0f;
    if (lane < rem) {
      xrem = xr[(nfull << 6) + lane];
      if (rr) {
        xrem = xrem + rr[(nfull << 6) + lane];
        xr[(nfull << 6) + lane] = xrem;
      }
    }
    const float inv_d = 1.0f / static_cast<float>(d);

    // Pass 1: mean.
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < NB; ++t)
      if (t < nfull) s = s + xv[t];
    for (int bb = 0; bb < rem16; ++bb) {
      const float v = __shfl(xrem, (bb << 4) + (lane & 15));
      if (lane < 16) s = s + v;
    }
    float tsum = 0.0f;
    for (int i = 0; i < tail; ++i) tsum += __shfl(xrem, (rem16 << 4) + i);
    float a = s + __shfl_down(s, 16);
    float v16 = a + __shfl_down(a, 32);
    const float mean = (__shfl(red16_lanes(v16), 0) + tsum) * inv_d;

    // Pass 2: variance.
    s = 0.0f;
#pragma unroll
    for (int t = 0; t < NB; ++t)
      if (t < nfull) {
        const float df = xv[t] - mean;
        s = __builtin_fmaf(df, df, s);
      }
    for (int bb = 0; bb < rem16; ++bb) {
      const float df = __shfl(xrem, (bb << 4) + (lane & 15)) - mean;
      if (lane < 16) s = __builtin_fmaf(df, df, s);
    }
    float vtail = 0.0f;
    for (int i = 0; i < tail; ++i) {
      const float df = __shfl(xrem, (rem16 << 4) + i) - mean;
      vtail = __builtin_fmaf(df, df, vtail);
    }
    a = s + __shfl_down(s, 16);
    v16 = a + __shfl_down(a, 32);
    const float ve = __builtin_fmaf(__shfl(red16_lanes(v16), 0) + vtail, inv_d, eps);
    const float sd = static_cast<float>(sqrt(static_cast<double>(ve)));
    const float inv_std = static_cast<float>(1.0 / static_cast<double>(sd));

    // Pass 3.
    float* yr = out + static_cast<size_t>(row) * d;
    auto emit = [&](int c, float xc) {
      float y = __builtin_fmaf((xc - mean) * inv_std, gamma[c], beta[c]);
      if (round16) y = static_cast<float>(static_cast<_Float16>(y));
      yr[c] = y;
      m = fmaxf(m, fabsf(y));
    };
#pragma unroll
    for (int t = 0; t < NB; ++t)
      if (t < nfull) emit((t << 6) + lane, xv[t]);
    if (lane < rem) emit((nfull << 6) + lane, xrem);
  }
  if (absmax) block_atomic_max_nonneg(absmax, m);
}

// The same for rows of exactly NB 64-element blocks (d = 64 NB: no leftover
// blocks, no tail), with the operations above in the same order: every
// load of a row goes out before its first use and no per-block branch
// splits them. ln_x86_row: the row's LayerNorm from its values xv, in place
// (y, fp16-rounded when round16), shared by the kernels below so that every
// pass over a row computes the same values.
template <int NB>
__device__ __forceinline__ void ln_x86_row(float (&xv)[NB], const float* __restrict__ gamma,
                                           const float* __restrict__ beta, float eps, int lane, int round16) {
  constexpr int d = NB * 64;
  const float inv_d = 1.0f / static_cast<float>(d);
  const float tsum = 0.0f, vtail = 0.0f;  // no tail elements

  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < NB; ++t) s = s + xv[t];
  float a = s + __shfl_down(s, 16);
  float v16 = a + __shfl_down(a, 32);
  const float mean = (__shfl(red16_lanes(v16), 0) + tsum) * inv_d;

  s = 0.0f;
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    const float df = xv[t] - mean;
    s = __builtin_fmaf(df, df, s);
  }
  a = s + __shfl_down(s, 16);
  v16 = a + __shfl_down(a, 32);
  const float ve = __builtin_fmaf(__shfl(red16_lanes(v16), 0) + vtail, inv_d, eps);
  const float sd = static_cast<float>(sqrt(static_cast<double>(ve)));
  const float inv_std = static_cast<float>(1.0 / static_cast<double>(sd));

  float gv[NB], bv[NB];
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    gv[t] = gamma[(t << 6) + lane];
    bv[t] = beta[(t << 6) + lane];
  }
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    float y = __builtin_fmaf((xv[t] - mean) * inv_std, gv[t], bv[t]);
    if (round16) y = static_cast<float>(static_cast<_Float16>(y));
    xv[t] = y;
  }
}

// Rows walked grid-stride (one atomic per block for each maximum). out may
// be null (the maxima alone); absmax gets max |y| of every row, tail_absmax
// (if not null) that of rows >= tail_row (LinearAmx's separately quantised
// last rows).
template <int NB>
__global__ __launch_bounds__(256) void layernorm_x86_rows_kernel(float* __restrict__ x,
                                                                  const float* __restrict__ resid,
                                                                  const float* __restrict__ gamma,
                                                                  const float* __restrict__ beta, float eps,
                                                                  float* __restrict__ out, int rows,
                                                                  float* __restrict__ absmax, int round16,
                                                                  float* __restrict__ tail_absmax, int tail_row) {
  constexpr int d = NB * 64;
  const int lane = threadIdx.x & 63;
  float m = 0.0f, mt = 0.0f;
  for (int row = blockIdx.x * 4 + (threadIdx.x >> 6); row < rows; row += gridDim.x * 4) {
    float* xr = x + static_cast<size_t>(row) * d;
    float xv[NB];
#pragma unroll
    for (int t = 0; t < NB; ++t) xv[t] = xr[(t << 6) + lane];
    if (resid) {
      const float* rr = resid + static_cast<size_t>(row) * d;
      float rv[NB];
#pragma unroll
      for (int t = 0; t < NB; ++t) rv[t] = rr[(t << 6) + lane];
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        xv[t] = xv[t] + rv[t];
        xr[(t << 6) + lane] = xv[t];
      }
    }
    ln_x86_row<NB>(xv, gamma, beta, eps, lane, round16);
    float rm = 0.0f;
#pragma unroll
    for (int t = 0; t < NB; ++t) rm = fmaxf(rm, fabsf(xv[t]));
    m = fmaxf(m, rm);
    if (row >= tail_row) mt = fmaxf(mt, rm);
    if (out) {
      float* yr = out + static_cast<size_t>(row) * d;
#pragma unroll
      for (int t = 0; t < NB; ++t) yr[(t << 6) + lane] = xv[t];
    }
  }
  if (absmax) block_atomic_max_nonneg(absmax, m);
  if (tail_absmax) block_atomic_max_nonneg(tail_absmax, mt);
}

// The same LayerNorm (no residual: x holds the sum already) quantised as
// QuantizeActPrefixAvx512 with the per-tensor scale of *absmax (rows >=
// tail_row: *tail_absmax), each code quant_i8 and the row's tail zeroed, as
// quant_tensor_kernel forms them: the codes of launch_layernorm_x86 then
// launch_quant_tensor, without the fp32 output. One wave per row.
template <int NB>
__global__ __launch_bounds__(256) void layernorm_x86_quant_kernel(const float* __restrict__ x,
                                                                   const float* __restrict__ gamma,
                                                                   const float* __restrict__ beta, float eps, int rows,
                                                                   const float* __restrict__ absmax,
                                                                   const float* __restrict__ tail_absmax, int tail_row,
                                                                   int8_t* __restrict__ q, int ldq,
                                                                   float* __restrict__ scales, int round16) {
  constexpr int d = NB * 64;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + static_cast<size_t>(row) * d;
  float xv[NB];
#pragma unroll
  for (int t = 0; t < NB; ++t) xv[t] = xr[(t << 6) + lane];
  ln_x86_row<NB>(xv, gamma, beta, eps, lane, round16);
  const float scale = act_scale_from_absmax(row >= tail_row ? *tail_absmax : *absmax);
  const float inv = 1.0f / scale;
  int8_t* qr = q + static_cast<size_t>(row) * ldq;
#pragma unroll
  for (int t = 0; t < NB; ++t) qr[(t << 6) + lane] = static_cast<int8_t>(quant_i8(xv[t], inv));
  for (int c = d + lane; c < ldq; c += 64) qr[c] = 0;
  if (lane == 0) scales[row] = scale;
}

// --------------------------------------------------------------- GELU
// GeluAvx512 elementwise; in place allowed. vec: x and out 16-byte aligned,
// four values per thread per step. absmax (optional): atomic max of |out|,
// one per block.
__global__ __launch_bounds__(256) void gelu_x86_kernel(const float* __restrict__ x, float* __restrict__ out, size_t n,
                                                       float* __restrict__ absmax, int vec) {
  float m = 0.0f;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  const size_t first = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  const size_t n4 = vec ? n / 4 : 0;
  for (size_t i = first; i < n4; i += stride) {
    const float4 v = reinterpret_cast<const float4*>(x)[i];
    const float4 y = make_float4(gelu_x86(v.x), gelu_x86(v.y), gelu_x86(v.z), gelu_x86(v.w));
    reinterpret_cast<float4*>(out)[i] = y;
    m = fmaxf(m, fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))));
  }
  for (size_t i = n4 * 4 + first; i < n; i += stride) {
    const float y = gelu_x86(x[i]);
    out[i] = y;
    m = fmaxf(m, fabsf(y));
  }
  if (absmax) block_atomic_max_nonneg(absmax, m);
}

// Elementwise expf_glibc (checks of the restated std::exp).
__global__ __launch_bounds__(256) void expf_glibc_kernel(const float* __restrict__ x, float* __restrict__ out,
                                                         size_t n) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    out[i] = expf_glibc(x[i]);
}

// --------------------------------------------------------------- RoPE
// ScaleInplace (x * scale, skipped when scale == 1) then
// RopeApplyVarlenAvx512 (reference src/kernels/rope.cpp:90-152): for the
// first-half index i, lo' = fnmadd(hi, s, lo * c) and hi' = fmadd(hi, c,
// lo * s), with c, s the tables' entries i of the token's position.
__global__ __launch_bounds__(256) void rope_x86_kernel(float* __restrict__ x, int ld, const int* __restrict__ pos,
                                                       int T, int heads, int head_dim, const float* __restrict__ cos_t,
                                                       const float* __restrict__ sin_t, int ldt, float scale) {
  const int half = head_dim >> 1;
  const size_t n = static_cast<size_t>(T) * heads * half;
  for (size_t e = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; e < n;
       e += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int i = static_cast<int>(e % half);
    const size_t th = e / half;
    const int h = static_cast<int>(th % heads);
    const int t = static_cast<int>(th / heads);
    float* xr = x + static_cast<size_t>(t) * ld + static_cast<size_t>(h) * head_dim;
    float lo = xr[i], hi = xr[i + half];
    if (scale != 1.0f) {
      lo = lo * scale;
      hi = hi * scale;
    }
    const size_t p = static_cast<size_t>(pos[t]) * ldt;
    const float c = cos_t[p + i], s = sin_t[p + i];
    const float lo_c = lo * c;
    const float lo_s = lo * s;
    xr[i] = __builtin_fmaf(-hi, s, lo_c);
    xr[i + half] = __builtin_fmaf(hi, c, lo_s);
  }
}

// ---------------------------------------------------------- attention
// AttentionVarlenAvx512 / RunOneHeadAvx512Impl (reference
// src/kernels/attention.cpp:240-430, 770-811). One wave per (sequence, head,
// 64 queries), one query per lane; the sequence's keys and values pass
// through LDS 16 rows at a time (8 KB per wave at head_dim 64, so the
// register file, not the LDS, bounds the waves per CU). Per query, as the
// reference:
//   score_j = red16 of the 16 lanes of fma(q[d], k_j[d], acc) over d
//   ascending in 16-wide steps (DotAvx512 and the 16-accumulator loop agree);
//   max over all keys;
//   keys of whole 16-key chunks: e = ExpAvx512Attn(score - max), summed per
//   lane j % 16 in chunk order, then red16; the last L % 16 keys: e =
//   std::exp(score - max) added one by one after that;
//   out[d] = fma(e_j * inv_sum, v_j[d], out[d]) over keys in order, zero
//   weights skipped.
// Scores are recomputed in each of the three passes (identical arithmetic,
// identical values), so no per-query score buffer is needed at any length.
template <int DH>
__device__ __forceinline__ float score_x86(const float (&q)[DH], const float* __restrict__ kr) {
  float acc[16];
#pragma unroll
  for (int l = 0; l < 16; ++l) acc[l] = 0.0f;
#pragma unroll
  for (int c = 0; c < DH / 16; ++c) {
#pragma unroll
    for (int l4 = 0; l4 < 4; ++l4) {
      const float4 k4 = *reinterpret_cast<const float4*>(kr + c * 16 + l4 * 4);
      acc[l4 * 4 + 0] = __builtin_fmaf(q[c * 16 + l4 * 4 + 0], k4.x, acc[l4 * 4 + 0]);
      acc[l4 * 4 + 1] = __builtin_fmaf(q[c * 16 + l4 * 4 + 1], k4.y, acc[l4 * 4 + 1]);
      acc[l4 * 4 + 2] = __builtin_fmaf(q[c * 16 + l4 * 4 + 2], k4.z, acc[l4 * 4 + 2]);
      acc[l4 * 4 + 3] = __builtin_fmaf(q[c * 16 + l4 * 4 + 3], k4.w, acc[l4 * 4 + 3]);
    }
  }
  return red16(acc);
}

constexpr int kX86Keys = 16;  // keys staged per LDS pass (one 16-key chunk of the reference)

// Scratch offset (floats) of sequence b's scores when every sequence b'
// before it holds heads x pad64(L_b') x L_b' of them: the wave sums those
// sizes 64 sequences at a time.
__device__ __forceinline__ size_t score_base(const int* __restrict__ cu, int b, int heads) {
  const int lane = threadIdx.x & 63;
  uint32_t pre = 0;
  for (int c = 0; c < b; c += 64) {
    const int bb = c + lane;
    uint32_t t = 0;
    if (bb < b) {
      const uint32_t L = static_cast<uint32_t>(cu[bb + 1] - cu[bb]);
      t = ((L + 63u) & ~63u) * L;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) t += __shfl_xor(t, off, 64);
    pre += t;
  }
  return static_cast<size_t>(pre) * static_cast<size_t>(heads);
}

// SC: the scores of pass 1 are stored in `scores` (this wave's region,
// key j of lane l at j * 64 + l) and pass 2 replaces each with its
// exponential, so passes 2 and 3 read what pass 1 and pass 2 computed
// instead of recomputing it: the same values, the same order of operations.
// Regions: sequence b at score_base, then head h at h x pad64(L) x L, then
// query tile t at t x 64 x L. Without SC every pass recomputes the scores.
// work: null (the grid is (query tiles, heads, sequences)), or one
// (sequence, head, 64-query tile) item per workgroup, longest sequences
// first so that their long items start early and the short ones fill in.
template <int DH, bool SC>
__global__ __launch_bounds__(64, 3) void attn_x86_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                      const float* __restrict__ v, int ld, const int* __restrict__ cu,
                                                      int heads, float* __restrict__ out, int ldo,
                                                      float* __restrict__ scores, const AttnWork* __restrict__ work,
                                                      float* __restrict__ part_max) {
  __shared__ __attribute__((aligned(16))) float ks[kX86Keys][DH];
  __shared__ __attribute__((aligned(16))) float vs[kX86Keys][DH];
  int b = blockIdx.z, h = blockIdx.y, q0 = blockIdx.x * 64;
  if (work) {
    const AttnWork w = work[blockIdx.x];
    b = w.seq;
    h = w.head;
    q0 = w.q0;
  }
  const int s0 = cu[b], L = cu[b + 1] - s0;
  // part_max (optional): slot blockIdx.x receives the largest |output| the
  // workgroup stores (0 for an item past its sequence).
  if (q0 >= L) {
    if (part_max && threadIdx.x == 0) part_max[blockIdx.x] = 0.0f;
    return;
  }
  const int lane = threadIdx.x;
  const int i = min(q0 + lane, L - 1);
  const bool active = q0 + lane < L;
  float* sc_w = nullptr;  // this lane's key-0 slot
  if constexpr (SC) {
    const size_t Lp = static_cast<size_t>((L + 63) & ~63);
    sc_w = scores + score_base(cu, b, heads) + static_cast<size_t>(h) * Lp * L +
           static_cast<size_t>(q0) * L + lane;
  }
  float qv[DH];
  {
    const float* qr = q + static_cast<size_t>(s0 + i) * ld + static_cast<size_t>(h) * DH;
#pragma unroll
    for (int d4 = 0; d4 < DH / 4; ++d4) {
      const float4 t = *reinterpret_cast<const float4*>(qr + d4 * 4);
      qv[d4 * 4 + 0] = t.x;
      qv[d4 * 4 + 1] = t.y;
      qv[d4 * 4 + 2] = t.z;
      qv[d4 * 4 + 3] = t.w;
    }
  }
  const int Lfull = L & ~15;
  // Stages rows [kc, kc + 16) of K and / or V into LDS, 16 bytes per lane per
  // step: item t is float4 t % (DH / 4) of row t / (DH / 4). Rows past the
  // sequence are not read (their LDS slots are never used).
  auto stage = [&](int kc, bool with_k, bool with_v) {
    __syncthreads();
    constexpr int kItems = kX86Keys * DH / 4;
#pragma unroll
    for (int t0 = 0; t0 < kItems; t0 += 64) {
      const int t = t0 + lane;
      const int r = t / (DH / 4), d4 = t % (DH / 4);
      if ((kItems % 64 == 0 || t < kItems) && kc + r < L) {
        const size_t o = static_cast<size_t>(s0 + kc + r) * ld + static_cast<size_t>(h) * DH + d4 * 4;
        if (with_k) *reinterpret_cast<float4*>(&ks[r][d4 * 4]) = *reinterpret_cast<const float4*>(k + o);
        if (with_v) *reinterpret_cast<float4*>(&vs[r][d4 * 4]) = *reinterpret_cast<const float4*>(v + o);
      }
    }
    __syncthreads();
  };

  // Pass 1: maximum score.
  float mx = -INFINITY;
  for (int kc = 0; kc < L; kc += kX86Keys) {
    stage(kc, true, false);
    const int nk = min(kX86Keys, L - kc);
    for (int jj = 0; jj < nk; ++jj) {
      const float sc = score_x86<DH>(qv, ks[jj]);
      if constexpr (SC) sc_w[static_cast<size_t>(kc + jj) * 64] = sc;
      mx = sc > mx ? sc : mx;
    }
  }

  // Pass 2: sum of exponentials.
  float vsum[16];
#pragma unroll
  for (int l = 0; l < 16; ++l) vsum[l] = 0.0f;
  float sum = 0.0f;
  bool summed = false;
  for (int kc = 0; kc < L; kc += kX86Keys) {
    if constexpr (!SC) stage(kc, true, false);
    const int nk = min(kX86Keys, L - kc);
    for (int jb = 0; jb < nk; jb += 16) {
      if (kc + jb + 16 <= L) {
        if constexpr (SC) {
          float* p = sc_w + static_cast<size_t>(kc + jb) * 64;
          float sv[16];
#pragma unroll
          for (int u = 0; u < 16; ++u) sv[u] = p[u * 64];
#pragma unroll
          for (int u = 0; u < 16; ++u) {
            const float e = exp_x86(sv[u] - mx);
            p[u * 64] = e;
            vsum[u] = vsum[u] + e;
          }
        } else {
#pragma unroll
          for (int u = 0; u < 16; ++u) vsum[u] = vsum[u] + exp_x86(score_x86<DH>(qv, ks[jb + u]) - mx);
        }
      } else {
        sum = red16(vsum);
        summed = true;
        for (int u = 0; kc + jb + u < L; ++u) {
          float e;
          if constexpr (SC) {
            float* p = sc_w + static_cast<size_t>(kc + jb + u) * 64;
            e = expf_glibc(*p - mx);
            *p = e;
          } else {
            e = expf_glibc(score_x86<DH>(qv, ks[jb + u]) - mx);
          }
          sum += e;
        }
      }
    }
  }
  if (!summed) sum = red16(vsum);
  const float inv = sum > 0.0f ? static_cast<float>(1.0 / static_cast<double>(sum)) : 0.0f;

  // Pass 3: weighted sum of V.
  float o[DH];
#pragma unroll
  for (int d = 0; d < DH; ++d) o[d] = 0.0f;
  for (int kc = 0; kc < L; kc += kX86Keys) {
    stage(kc, !SC, true);
    const int nk = min(kX86Keys, L - kc);
    float ec[kX86Keys];
    if constexpr (SC) {
#pragma unroll
      for (int jj = 0; jj < kX86Keys; ++jj) ec[jj] = jj < nk ? sc_w[static_cast<size_t>(kc + jj) * 64] : 0.0f;
    }
    for (int jj = 0; jj < nk; ++jj) {
      float e;
      if constexpr (SC) {
        e = ec[jj];
      } else {
        const float sc = score_x86<DH>(qv, ks[jj]) - mx;
        e = kc + jj < Lfull ? exp_x86(sc) : expf_glibc(sc);
      }
      const float w = e * inv;
      if (w == 0.0f) continue;
#pragma unroll
      for (int d4 = 0; d4 < DH / 4; ++d4) {
        const float4 t = *reinterpret_cast<const float4*>(&vs[jj][d4 * 4]);
        o[d4 * 4 + 0] = __builtin_fmaf(w, t.x, o[d4 * 4 + 0]);
        o[d4 * 4 + 1] = __builtin_fmaf(w, t.y, o[d4 * 4 + 1]);
        o[d4 * 4 + 2] = __builtin_fmaf(w, t.z, o[d4 * 4 + 2]);
        o[d4 * 4 + 3] = __builtin_fmaf(w, t.w, o[d4 * 4 + 3]);
      }
    }
  }
  float m = 0.0f;
  if (active) {
    float* orow = out + static_cast<size_t>(s0 + q0 + lane) * ldo + static_cast<size_t>(h) * DH;
#pragma unroll
    for (int d4 = 0; d4 < DH / 4; ++d4)
      *reinterpret_cast<float4*>(orow + d4 * 4) = float4{o[d4 * 4], o[d4 * 4 + 1], o[d4 * 4 + 2], o[d4 * 4 + 3]};
#pragma unroll
    for (int d = 0; d < DH; ++d) m = fmaxf(m, fabsf(o[d]));
  }
  if (part_max) {
    m = wave_max(m);
    if (lane == 0) part_max[blockIdx.x] = m;
  }
}

// ------------------------------------------------------- FP32 Linear
// LinearAvx512 (reference src/kernels/gemm_fp32.cpp:194-294):
// C[m, n] = bias[n] + red16 of the 16 lanes of fma(A[m, k], W[n, k], acc)
// over k ascending in 16-wide steps (a partial last step adds nothing to the
// lanes past K: fma(0, 0, acc) == acc for the +0-seeded accumulators).
// EPI: kF32Store, kF32Gelu (gelu_x86 of that value, as the reference's
// Linear followed by Gelu), kF32Resid (C += that value, ResidualAddInplace).
// A 16 x 16 tile of outputs per 256-thread workgroup, one per thread; A and
// W rows pass through LDS 64 columns at a time.
constexpr int kLinKc = 64;

template <int EPI>
__global__ __launch_bounds__(256) void linear_x86_kernel(const float* __restrict__ A, int lda,
                                                         const float* __restrict__ W, int ldw,
                                                         const float* __restrict__ bias, float* __restrict__ C,
                                                         int ldc, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) float as[16][kLinKc + 4];
  __shared__ __attribute__((aligned(16))) float ws[16][kLinKc + 4];
  const int tm = threadIdx.x >> 4, tn = threadIdx.x & 15;
  const int m0 = blockIdx.y * 16, n0 = blockIdx.x * 16;
  const int m = m0 + tm, n = n0 + tn;
  float acc[16];
#pragma unroll
  for (int l = 0; l < 16; ++l) acc[l] = 0.0f;
  for (int k0 = 0; k0 < K; k0 += kLinKc) {
    __syncthreads();
    // 256 threads copy 16 rows x 64 columns of A and of W (4 floats each).
    {
      const int r = threadIdx.x >> 4, c = (threadIdx.x & 15) * 4;
      const int ar = min(m0 + r, M - 1), wr = min(n0 + r, N - 1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int kk = k0 + c + e;
        as[r][c + e] = kk < K ? A[static_cast<size_t>(ar) * lda + kk] : 0.0f;
        ws[r][c + e] = kk < K ? W[static_cast<size_t>(wr) * ldw + kk] : 0.0f;
      }
    }
    __syncthreads();
    const int steps = min(kLinKc, K - k0);
    for (int s = 0; s < steps; s += 16) {
#pragma unroll
      for (int l4 = 0; l4 < 4; ++l4) {
        const float4 a4 = *reinterpret_cast<const float4*>(&as[tm][s + l4 * 4]);
        const float4 w4 = *reinterpret_cast<const float4*>(&ws[tn][s + l4 * 4]);
        acc[l4 * 4 + 0] = __builtin_fmaf(a4.x, w4.x, acc[l4 * 4 + 0]);
        acc[l4 * 4 + 1] = __builtin_fmaf(a4.y, w4.y, acc[l4 * 4 + 1]);
        acc[l4 * 4 + 2] = __builtin_fmaf(a4.z, w4.z, acc[l4 * 4 + 2]);
        acc[l4 * 4 + 3] = __builtin_fmaf(a4.w, w4.w, acc[l4 * 4 + 3]);
      }
    }
  }
  if (m >= M || n >= N) return;
  const float y = (bias ? bias[n] : 0.0f) + red16(acc);
  float* c = C + static_cast<size_t>(m) * ldc + n;
  if constexpr (EPI == kF32Gelu) {
    *c = gelu_x86(y);
  } else if constexpr (EPI == kF32Resid) {
    *c = *c + y;
  } else {
    *c = y;
  }
}

// The same sums with 32 x 32 outputs per 256-thread workgroup. Thread t owns
// the reference's accumulator lanes 4q .. 4q + 3 (q = t % 4) of a 4 x 4
// block of outputs (rows 4 (b / 8) + i, columns 4 (b % 8) + j, b = t / 4), so
// each 16-wide K step reads eight 16-byte LDS words for 64 FMAs instead of
// one word per FMA; every accumulator lane still takes its products in K
// order. The four threads of a block then add their lanes in red16's order
// (lanes l and l + 8 first: threads q and q ^ 2; then l and l + 4: q and
// q ^ 1), and thread q = 0 stores the block.
template <int EPI>
__global__ __launch_bounds__(256) void linear_x86_blk_kernel(const float* __restrict__ A, int lda,
                                                             const float* __restrict__ W, int ldw,
                                                             const float* __restrict__ bias, float* __restrict__ C,
                                                             int ldc, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) float as[32][kLinKc + 4];
  __shared__ __attribute__((aligned(16))) float ws[32][kLinKc + 4];
  const int t = threadIdx.x, q = t & 3, b = t >> 2, bm = b >> 3, bn = b & 7;
  const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  float acc[4][4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.0f;
  for (int k0 = 0; k0 < K; k0 += kLinKc) {
    __syncthreads();
    // 256 threads copy 32 rows x 64 columns of A and of W (8 floats each);
    // columns past K read as zero (fma(0, 0, acc) == acc).
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int idx = t + 256 * u;
      const int r = idx >> 4, c = (idx & 15) * 4;
      const int ar = min(m0 + r, M - 1), wr = min(n0 + r, N - 1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int kk = k0 + c + e;
        as[r][c + e] = kk < K ? A[static_cast<size_t>(ar) * lda + kk] : 0.0f;
        ws[r][c + e] = kk < K ? W[static_cast<size_t>(wr) * ldw + kk] : 0.0f;
      }
    }
    __syncthreads();
    const int steps = min(kLinKc, K - k0);
    for (int s0 = 0; s0 < steps; s0 += 16) {
      float4 a[4], w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const float4*>(&as[4 * bm + i][s0 + 4 * q]);
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = *reinterpret_cast<const float4*>(&ws[4 * bn + j][s0 + 4 * q]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[i][j][0] = __builtin_fmaf(a[i].x, w[j].x, acc[i][j][0]);
          acc[i][j][1] = __builtin_fmaf(a[i].y, w[j].y, acc[i][j][1]);
          acc[i][j][2] = __builtin_fmaf(a[i].z, w[j].z, acc[i][j][2]);
          acc[i][j][3] = __builtin_fmaf(a[i].w, w[j].w, acc[i][j][3]);
        }
    }
  }
  // red16: t3[l] = v[l + 8] + v[l] (l < 8), t6[l] = t3[l + 4] + t3[l]
  // (l < 4), then (t6[0] + t6[2]) + (t6[1] + t6[3]). Thread q holds lanes
  // 4q + e; after the first exchange thread 0 holds t3[0..3] and thread 1
  // t3[4..7], after the second thread 0 holds t6[0..3].
  float out[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float t3[4], t6[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) t3[e] = __shfl_xor(acc[i][j][e], 2, 4) + acc[i][j][e];
#pragma unroll
      for (int e = 0; e < 4; ++e) t6[e] = __shfl_xor(t3[e], 1, 4) + t3[e];
      out[i][j] = (t6[0] + t6[2]) + (t6[1] + t6[3]);
    }
  if (q != 0) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + 4 * bm + i;
    if (m >= M) break;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + 4 * bn + j;
      if (n >= N) break;
      const float y = (bias ? bias[n] : 0.0f) + out[i][j];
      float* c = C + static_cast<size_t>(m) * ldc + n;
      if constexpr (EPI == kF32Gelu) {
        *c = gelu_x86(y);
      } else if constexpr (EPI == kF32Resid) {
        *c = *c + y;
      } else {
        *c = y;
      }
    }
  }
}

// The same sums with 32 x 32 outputs per 256-thread workgroup, each thread
// holding two accumulator lanes (2q, 2q + 1; q = t % 8) of an 8 x 4 block
// of outputs (rows 8 (b / 8) + i, columns 4 (b % 8) + j, b = t / 8): a
// 16-wide K step reads 12 8-byte LDS words for 64 FMAs (the kernel above:
// eight 16-byte words), and the tiles arrive through 16-byte loads. The
// eight threads of a block then add their lanes in red16's order (lanes l
// and l + 8: threads q and q ^ 4; l and l + 4: q ^ 2; then t6[0] + t6[2] and
// t6[1] + t6[3]: q ^ 1), every thread ending with every sum, and thread q
// stores row q of the block. A, W 16-byte aligned, lda, ldw and K multiples
// of 4. LinearAvx512 of the lm head's dense: 4.10 -> 2.56 ms per forward.
template <int EPI>
__global__ __launch_bounds__(256) void linear_x86_wide_kernel(const float* __restrict__ A, int lda,
                                                              const float* __restrict__ W, int ldw,
                                                              const float* __restrict__ bias, float* __restrict__ C,
                                                              int ldc, int M, int N, int K) {
  constexpr int kPitch = kLinKc + 4;
  __shared__ __attribute__((aligned(16))) float as[32][kPitch];
  __shared__ __attribute__((aligned(16))) float ws[32][kPitch];
  const int t = threadIdx.x, q = t & 7, b = t >> 3, bm = b >> 3, bn = b & 7;
  const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  float acc[8][4][2];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j][0] = acc[i][j][1] = 0.0f;
  for (int k0 = 0; k0 < K; k0 += kLinKc) {
    __syncthreads();
    // A: 32 rows x 16 float4, W: 64 rows x 16 float4; columns past K are
    // zero (fma(0, 0, acc) == acc), rows past M / N repeat the last one.
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int idx = t + 256 * u, r = idx >> 4, c = (idx & 15) * 4;
      const int ar = min(m0 + r, M - 1);
      const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
      *reinterpret_cast<float4*>(&as[r][c]) =
          k0 + c < K ? *reinterpret_cast<const float4*>(A + static_cast<size_t>(ar) * lda + k0 + c) : z;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int idx = t + 256 * u, r = idx >> 4, c = (idx & 15) * 4;
      const int wr = min(n0 + r, N - 1);
      const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
      *reinterpret_cast<float4*>(&ws[r][c]) =
          k0 + c < K ? *reinterpret_cast<const float4*>(W + static_cast<size_t>(wr) * ldw + k0 + c) : z;
    }
    __syncthreads();
    const int steps = min(kLinKc, K - k0);
    for (int s0 = 0; s0 < steps; s0 += 16) {
      float2 av[8], wv[4];
#pragma unroll
      for (int i = 0; i < 8; ++i) av[i] = *reinterpret_cast<const float2*>(&as[8 * bm + i][s0 + 2 * q]);
#pragma unroll
      for (int j = 0; j < 4; ++j) wv[j] = *reinterpret_cast<const float2*>(&ws[4 * bn + j][s0 + 2 * q]);
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[i][j][0] = __builtin_fmaf(av[i].x, wv[j].x, acc[i][j][0]);
          acc[i][j][1] = __builtin_fmaf(av[i].y, wv[j].y, acc[i][j][1]);
        }
    }
  }
  float out[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float t3[2], t6[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) t3[e] = __shfl_xor(acc[i][j][e], 4, 8) + acc[i][j][e];
#pragma unroll
      for (int e = 0; e < 2; ++e) t6[e] = __shfl_xor(t3[e], 2, 8) + t3[e];
      const float a = t6[0] + __shfl_xor(t6[0], 1, 8);  // t6[0] + t6[2]
      const float bb = t6[1] + __shfl_xor(t6[1], 1, 8);  // t6[1] + t6[3]
      out[i][j] = a + bb;
    }
  {
    const int i = q;  // thread q stores row q of the block
    const int m = m0 + 8 * bm + i;
    float orow[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      float o = out[0][jj];
#pragma unroll
      for (int ii = 1; ii < 8; ++ii) o = ii == i ? out[ii][jj] : o;
      orow[jj] = o;
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int n = n0 + 4 * bn + jj;
      if (m >= M || n >= N) continue;
      const float y = (bias ? bias[n] : 0.0f) + orow[jj];
      float* c = C + static_cast<size_t>(m) * ldc + n;
      if constexpr (EPI == kF32Gelu) {
        *c = gelu_x86(y);
      } else if constexpr (EPI == kF32Resid) {
        *c = *c + y;
      } else {
        *c = y;
      }
    }
  }
}

int grid_for(size_t n, int block, int cap) {
  const size_t g = (n + block - 1) / block;
  return static_cast<int>(g < static_cast<size_t>(cap) ? g : cap);
}

}  // namespace

bool layernorm_x86_rows_ok(int d) { return d == 1280 || d == 320; }

hipError_t launch_layernorm_x86_quant(const float* x, const float* gamma, const float* beta, float eps, int rows,
                                      int d, const float* absmax, const float* tail_absmax, int tail_row, int8_t* q,
                                      int ldq, float* scales, int round16, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (!absmax || (tail_row < rows && !tail_absmax) || ldq < d) return hipErrorInvalidValue;
  const dim3 grid((rows + 3) / 4), block(256);
  if (d == 1280)
    hipLaunchKernelGGL(layernorm_x86_quant_kernel<20>, grid, block, 0, s, x, gamma, beta, eps, rows, absmax,
                       tail_absmax, tail_row, q, ldq, scales, round16);
  else if (d == 320)
    hipLaunchKernelGGL(layernorm_x86_quant_kernel<5>, grid, block, 0, s, x, gamma, beta, eps, rows, absmax,
                       tail_absmax, tail_row, q, ldq, scales, round16);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_layernorm_x86(float* x, const float* resid, const float* gamma, const float* beta, float eps,
                                float* out, int rows, int d, float* absmax, int round16, hipStream_t s,
                                float* tail_absmax, int tail_row) {
  if (rows <= 0 || d <= 0) return hipSuccess;
  const dim3 grid(grid_for(static_cast<size_t>(rows), 4, 1024)), block(256);  // rows walked grid-stride
  const int nb = d >> 6;
  if (d == 1280) {  // ESM-2 650M
    hipLaunchKernelGGL(layernorm_x86_rows_kernel<20>, grid, block, 0, s, x, resid, gamma, beta, eps, out, rows, absmax,
                       round16, tail_absmax, tail_row);
    return hipGetLastError();
  }
  if (d == 320) {  // ESM-2 8M
    hipLaunchKernelGGL(layernorm_x86_rows_kernel<5>, grid, block, 0, s, x, resid, gamma, beta, eps, out, rows, absmax,
                       round16, tail_absmax, tail_row);
    return hipGetLastError();
  }
  if (!out || tail_absmax) return hipErrorInvalidValue;  // the generic kernel stores every row
  if (nb <= 5)
    hipLaunchKernelGGL(layernorm_x86_kernel<5>, grid, block, 0, s, x, resid, gamma, beta, eps, out, rows, d, absmax,
                       round16);
  else if (nb <= 20)
    hipLaunchKernelGGL(layernorm_x86_kernel<20>, grid, block, 0, s, x, resid, gamma, beta, eps, out, rows, d, absmax,
                       round16);
  else if (nb <= 40)
    hipLaunchKernelGGL(layernorm_x86_kernel<40>, grid, block, 0, s, x, resid, gamma, beta, eps, out, rows, d, absmax,
                       round16);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_gelu_x86(const float* x, float* out, size_t n, float* absmax, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const int vec = (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) % 16 == 0;
  hipLaunchKernelGGL(gelu_x86_kernel, dim3(grid_for(vec ? n / 4 : n, 256, 1024)), dim3(256), 0, s, x, out, n, absmax,
                     vec);
  return hipGetLastError();
}

hipError_t launch_expf_glibc(const float* x, float* out, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(expf_glibc_kernel, dim3(grid_for(n, 256, 8192)), dim3(256), 0, s, x, out, n);
  return hipGetLastError();
}

hipError_t launch_rope_x86(float* x, int ld, const int* pos, int T, int heads, int head_dim, const float* cos_t,
                           const float* sin_t, int ldt, float scale, hipStream_t s) {
  const size_t n = static_cast<size_t>(T) * heads * (head_dim / 2);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(rope_x86_kernel, dim3(grid_for(n, 256, 16384)), dim3(256), 0, s, x, ld, pos, T, heads, head_dim,
                     cos_t, sin_t, ldt, scale);
  return hipGetLastError();
}

bool attention_x86_supported(int head_dim) { return head_dim == 16 || head_dim == 32 || head_dim == 64; }

size_t attention_x86_score_floats(const int* cu, int batch, int heads) {
  size_t n = 0;
  for (int b = 0; b < batch; ++b) {
    const size_t L = static_cast<size_t>(cu[b + 1] - cu[b]);
    n += ((L + 63) & ~static_cast<size_t>(63)) * L;
  }
  return n * static_cast<size_t>(heads);
}

hipError_t launch_attention_x86(const float* q, const float* k, const float* v, int ld, int head_dim, const int* cu,
                                int batch, int heads, int max_len, float* out, int ldo, hipStream_t s,
                                float* scores, const AttnWork* work, int nwork, float* part_max) {
  if (batch <= 0 || max_len <= 0) return hipSuccess;
  if (work && nwork <= 0) return hipSuccess;
  if (part_max && !work) return hipErrorInvalidValue;  // one slot per work item
  const dim3 grid = work ? dim3(nwork) : dim3((max_len + 63) / 64, heads, batch), block(64);
#define ESM_ATTN_X86(DH)                                                                                           \
  if (scores)                                                                                                      \
    hipLaunchKernelGGL((attn_x86_kernel<DH, true>), grid, block, 0, s, q, k, v, ld, cu, heads, out, ldo, scores,   \
                       work, part_max);                                                                            \
  else                                                                                                             \
    hipLaunchKernelGGL((attn_x86_kernel<DH, false>), grid, block, 0, s, q, k, v, ld, cu, heads, out, ldo, nullptr, \
                       work, part_max);
  switch (head_dim) {
    case 16: ESM_ATTN_X86(16) break;
    case 32: ESM_ATTN_X86(32) break;
    case 64: ESM_ATTN_X86(64) break;
    default: return hipErrorInvalidValue;
  }
#undef ESM_ATTN_X86
  return hipGetLastError();
}

hipError_t launch_linear_x86(const float* A, int lda, const float* W, int ldw, const float* bias, float* C, int ldc,
                             int M, int N, int K, int epi, hipStream_t s) {
  if (M <= 0 || N <= 0) return hipSuccess;
  const bool vec = K % 4 == 0 && lda % 4 == 0 && ldw % 4 == 0 && reinterpret_cast<uintptr_t>(A) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(W) % 16 == 0;
  if (vec && M >= 32 && N >= 32) {
    const dim3 grid((N + 31) / 32, (M + 31) / 32), block(256);
    switch (epi) {
      case kF32Store:
        hipLaunchKernelGGL(linear_x86_wide_kernel<kF32Store>, grid, block, 0, s, A, lda, W, ldw, bias, C, ldc, M, N,
                           K);
        break;
      case kF32Gelu:
        hipLaunchKernelGGL(linear_x86_wide_kernel<kF32Gelu>, grid, block, 0, s, A, lda, W, ldw, bias, C, ldc, M, N, K);
        break;
      case kF32Resid:
        hipLaunchKernelGGL(linear_x86_wide_kernel<kF32Resid>, grid, block, 0, s, A, lda, W, ldw, bias, C, ldc, M, N,
                           K);
        break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  if (M >= 32 && N >= 32) {
    const dim3 grid((N + 31) / 32, (M + 31) / 32), block(256);
    switch (epi) {
      case kF32Store:
        hipLaunchKernelGGL(linear_x86_blk_kernel<kF32Store>, grid, block, 0, s, A, lda, W, ldw, bias, C, ldc, M, N, K);
        break;
      case kF32Gelu:
        hipLaunchKernelGGL(linear_x86_blk_kernel<kF32Gelu>, grid, block, 0, s, A, lda, W, ldw, bias, C, ldc, M, N, K);
        break;
      case kF32Resid:
        hipLaunchKernelGGL(linear_x86_blk_kernel<kF32Resid>, grid, block, 0, s, A, lda, W, ldw, bias, C, ldc, M, N, K);
        break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const dim3 grid((N + 15) / 16, (M + 15) / 16), block(256);
  switch (epi) {
    case kF32Store:
      hipLaunchKernelGGL(linear_x86_kernel<kF32Store>, grid, block, 0, s, A, lda, W, ldw, bias, C, ldc, M, N, K);
      break;
    case kF32Gelu:
      hipLaunchKernelGGL(linear_x86_kernel<kF32Gelu>, grid, block, 0, s, A, lda, W, ldw, bias, C, ldc, M, N, K);
      break;
    case kF32Resid:
      hipLaunchKernelGGL(linear_x86_kernel<kF32Resid>, grid, block, 0, s, A, lda, W, ldw, bias, C, ldc, M, N, K);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace esm_gfx950
