// W8A8 INT8 GEMM for gfx950: v_mfma_i32_16x16x64_i8 with int32
// accumulation and fused epilogues (dequant + bias, GELU, residual add,
// QKV split with Q-scale and rotary embedding).
//
// Replaces the inner product of esm::kernels::LinearInt8
// (reference src/kernels/gemm_int8.cpp:510-555 LinearVnni and
// src/kernels/gemm_amx.cpp:218-309 LinearAmx). The reference dequantises
// with out = fma(float(acc), w_scale[n] * act_scale, bias[n])
// (gemm_int8.cpp:109-126); the epilogue here uses the same expression with
// a per-row activation scale, which equals the per-tensor scale when every
// row carries the tensor's scale.
//
// Tiling: a 256-thread workgroup owns a 128x128 output tile; its four
// waves (2x2) each own 64x64 = 4x4 MFMA blocks. K advances 128 bytes per
// stage; A and W stages are staged through LDS (double-buffered) with a
// 144-byte row pitch so the 16 rows read by one ds_read_b128 quarter-wave
// land on disjoint banks. Tiles are ordered so each XCD (workgroup id mod
// 8) walks a contiguous, M-grouped slice of the tile space, which keeps the
// A rows and W columns it shares inside that XCD's L2.
#include "common.hpp"
#include "kernels.hpp"

namespace esm_gfx950 {
namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 128;            // bytes of K per stage
constexpr int kPitch = BK + 16;    // LDS row pitch in bytes
constexpr int kThreads = 256;
constexpr int kStage = (BM + BN) * kPitch;
constexpr int kGroupM = 8;

__device__ __forceinline__ int xcd_remap(int id, int num) {
  constexpr int X = 8;
  const int per = num / X, rem = num % X;
  const int xcd = id % X, local = id / X;
  return xcd * per + min(xcd, rem) + local;
}

// Global -> registers for one 128-row x 128-byte stage. Rows past the
// matrix edge re-read the last valid row (results are discarded); K bytes
// past the end read as zero.
__device__ __forceinline__ void load_stage(const int8_t* __restrict__ base,
                                           int ld, int rows, int row0, int k0,
                                           int K, i32x4 (&r)[4]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = t + kThreads * i;
    const int row = idx >> 3;
    const int c = (idx & 7) * 16;
    int gr = row0 + row;
    gr = gr < rows ? gr : rows - 1;
    const int kk = k0 + c;
    if (kk < K) {
      r[i] = *reinterpret_cast<const i32x4*>(base + static_cast<size_t>(gr) * ld + kk);
    } else {
      r[i] = i32x4{0, 0, 0, 0};
    }
  }
}

__device__ __forceinline__ void store_stage(int8_t* s, const i32x4 (&r)[4]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = t + kThreads * i;
    const int row = idx >> 3;
    const int c = (idx & 7) * 16;
    *reinterpret_cast<i32x4*>(s + row * kPitch + c) = r[i];
  }
}

template <int EPI>
__device__ __forceinline__ void epilogue(const GemmI8Args& p,
                                         const i32x4 (&acc)[4][4], int rb,
                                         int cb, int lr, int lg) {
  if constexpr (EPI == kEpiI32) {
#pragma unroll
    for (int bm = 0; bm < 4; ++bm)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = rb + bm * 16 + lg * 4 + r;
        if (row >= p.M) continue;
#pragma unroll
        for (int bn = 0; bn < 4; ++bn) {
          const int col = cb + bn * 16 + lr;
          if (col < p.N) p.C_i32[static_cast<size_t>(row) * p.ldc + col] = acc[bm][bn][r];
        }
      }
    return;
  } else {
    float ws[4], bs[4];
#pragma unroll
    for (int bn = 0; bn < 4; ++bn) {
      const int col = cb + bn * 16 + lr;
      const bool ok = col < p.N;
      ws[bn] = ok ? p.w_scale[col] : 0.0f;
      bs[bn] = (ok && p.bias) ? p.bias[col] : 0.0f;
    }
    if constexpr (EPI == kEpiQkvRope) {
      // The wave's 64 columns are exactly one head of Q, K or V. Lane
      // column lr of block bn holds head dim bn*16+lr, so the rotary pairs
      // (i, i+32) sit in blocks (0,2) and (1,3) of the same lane and row.
      const int which = cb / p.d_model;
      const int hcol = cb - which * p.d_model;
#pragma unroll
      for (int bm = 0; bm < 4; ++bm)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rb + bm * 16 + lg * 4 + r;
          if (row >= p.M) continue;
          const float as = p.a_scale[row];
          float v[4];
#pragma unroll
          for (int bn = 0; bn < 4; ++bn)
            v[bn] = __builtin_fmaf(static_cast<float>(acc[bm][bn][r]), as * ws[bn], bs[bn]);
          const size_t o = static_cast<size_t>(row) * p.d_model + hcol + lr;
          if (which == 2) {
#pragma unroll
            for (int bn = 0; bn < 4; ++bn) p.v_out[o + bn * 16] = f32_to_f16_bits(v[bn]);
            continue;
          }
          if (which == 0) {
#pragma unroll
            for (int bn = 0; bn < 4; ++bn) v[bn] *= p.q_scale;
          }
          const int ps = p.pos[row];
          const float* ct = p.rope_cos + static_cast<size_t>(ps) * 64;
          const float* st = p.rope_sin + static_cast<size_t>(ps) * 64;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int i = h * 16 + lr;
            const float x1 = v[h], x2 = v[h + 2];
            v[h] = x1 * ct[i] - x2 * st[i];
            v[h + 2] = x2 * ct[i + 32] + x1 * st[i + 32];
          }
          uint16_t* dst = which == 0 ? p.q_out : p.k_out;
#pragma unroll
          for (int bn = 0; bn < 4; ++bn) dst[o + bn * 16] = f32_to_bf16_bits(v[bn]);
        }
      return;
    } else {
      float tmax = 0.0f;
#pragma unroll
      for (int bm = 0; bm < 4; ++bm)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rb + bm * 16 + lg * 4 + r;
          const bool rok = row < p.M;
          const float as = rok ? p.a_scale[row] : 0.0f;
          float rmax = 0.0f;
#pragma unroll
          for (int bn = 0; bn < 4; ++bn) {
            const int col = cb + bn * 16 + lr;
            float v = __builtin_fmaf(static_cast<float>(acc[bm][bn][r]), as * ws[bn], bs[bn]);
            if constexpr (EPI == kEpiF32Gelu || EPI == kEpiF32GeluQ) v = gelu_erf(v);
            if (rok && col < p.N) {
              const size_t o = static_cast<size_t>(row) * p.ldc + col;
              if constexpr (EPI == kEpiF32Resid) {
                p.C_f32[o] += v;
              } else if constexpr (EPI == kEpiF32GeluQ) {
                p.C_f16[o] = f32_to_f16_bits(v);
                rmax = fmaxf(rmax, fabsf(v));
              } else {
                p.C_f32[o] = v;
                rmax = fmaxf(rmax, fabsf(v));
              }
            }
          }
          if constexpr (EPI == kEpiF32Gelu || EPI == kEpiF32GeluQ || EPI == kEpiF32) {
            if (p.row_absmax) {
              // Lanes sharing lg hold the same row; reduce over the 16 of them.
#pragma unroll
              for (int off = 8; off >= 1; off >>= 1)
                rmax = fmaxf(rmax, __shfl_xor(rmax, off, kWave));
              if (lr == 0 && rok) atomic_max_nonneg(p.row_absmax + row, rmax);
            }
            tmax = fmaxf(tmax, rmax);
          }
        }
      if constexpr (EPI == kEpiF32Gelu || EPI == kEpiF32GeluQ || EPI == kEpiF32) {
        if (p.tensor_absmax) {
          tmax = wave_max(tmax);
          if ((threadIdx.x & 63) == 0) atomic_max_nonneg(p.tensor_absmax, tmax);
        }
      }
    }
  }
}

template <int EPI>
__global__ __launch_bounds__(kThreads, 2) void gemm_i8_kernel(const GemmI8Args p) {
  __shared__ __attribute__((aligned(16))) int8_t smem[2 * kStage];

  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int pid = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  const int per_group = kGroupM * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in_group = pid - group * per_group;
  const int m0 = (first_m + in_group % gsize) * BM;
  const int n0 = (in_group / gsize) * BN;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 15, lg = lane >> 4;

  i32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

  i32x4 ra[4], rb[4];
  const int nk = (p.K + BK - 1) / BK;
  load_stage(p.A, p.lda, p.M, m0, 0, p.K, ra);
  load_stage(p.W, p.ldw, p.N, n0, 0, p.K, rb);
  store_stage(smem, ra);
  store_stage(smem + BM * kPitch, rb);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int8_t* cur = smem + (kt & 1) * kStage;
    const bool more = kt + 1 < nk;
    if (more) {
      load_stage(p.A, p.lda, p.M, m0, (kt + 1) * BK, p.K, ra);
      load_stage(p.W, p.ldw, p.N, n0, (kt + 1) * BK, p.K, rb);
    }
    const int8_t* sa = cur + (wm * 64 + lr) * kPitch + lg * 16;
    const int8_t* sb = cur + BM * kPitch + (wn * 64 + lr) * kPitch + lg * 16;
#pragma unroll
    for (int kk = 0; kk < BK / 64; ++kk) {
      i32x4 fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        fa[i] = *reinterpret_cast<const i32x4*>(sa + i * 16 * kPitch + kk * 64);
        fb[i] = *reinterpret_cast<const i32x4*>(sb + i * 16 * kPitch + kk * 64);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      int8_t* nxt = smem + ((kt + 1) & 1) * kStage;
      store_stage(nxt, ra);
      store_stage(nxt + BM * kPitch, rb);
    }
    __syncthreads();
  }

  epilogue<EPI>(p, acc, m0 + wm * 64, n0 + wn * 64, lr, lg);
}

}  // namespace

hipError_t launch_gemm_i8(const GemmI8Args& p, int epi, hipStream_t s) {
  if (p.M <= 0 || p.N <= 0) return hipSuccess;
  const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const dim3 grid(tiles), block(kThreads);
  switch (epi) {
    case kEpiI32: hipLaunchKernelGGL(gemm_i8_kernel<kEpiI32>, grid, block, 0, s, p); break;
    case kEpiF32: hipLaunchKernelGGL(gemm_i8_kernel<kEpiF32>, grid, block, 0, s, p); break;
    case kEpiF32Gelu: hipLaunchKernelGGL(gemm_i8_kernel<kEpiF32Gelu>, grid, block, 0, s, p); break;
    case kEpiF32Resid: hipLaunchKernelGGL(gemm_i8_kernel<kEpiF32Resid>, grid, block, 0, s, p); break;
    case kEpiQkvRope: hipLaunchKernelGGL(gemm_i8_kernel<kEpiQkvRope>, grid, block, 0, s, p); break;
    case kEpiF32GeluQ: hipLaunchKernelGGL(gemm_i8_kernel<kEpiF32GeluQ>, grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace esm_gfx950
