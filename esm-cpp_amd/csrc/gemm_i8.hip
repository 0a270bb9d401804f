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
// Tiling (TileCfg): a 256-thread workgroup owns a 256x128 output tile; its
// four waves (2x2) each own 128x64 = 8x4 MFMA blocks of 16x16, so a wave
// reads 12 fragments (192 B per lane) from LDS per 32 MFMAs. K advances 64
// bytes per stage; A and W stages go global -> registers -> LDS, double-
// buffered, with an 80-byte row pitch so the 16 rows read by one
// ds_read_b128 quarter-wave land on disjoint banks. 60 KB of LDS and <= 256
// VGPRs per wave let two workgroups share a CU (two waves per SIMD), so one
// wave's LDS reads and barrier overlap the other's MFMAs. Tiles are ordered
// so each XCD (workgroup id mod 8) walks a contiguous, M-grouped slice of
// the tile space, which keeps the A rows and W columns it shares inside
// that XCD's L2.
#include "common.hpp"
#include "kernels.hpp"

namespace esm_gfx950 {
namespace {

template <int WAVES_M_, int WAVES_N_, int WM_, int WN_, int BK_>
struct TileCfg {
  static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
  static constexpr int WM = WM_, WN = WN_;  // 16x16 MFMA blocks per wave
  static constexpr int BM = WAVES_M * WM * 16;
  static constexpr int BN = WAVES_N * WN * 16;
  static constexpr int BK = BK_;            // bytes of K per stage
  static constexpr int THREADS = WAVES_M * WAVES_N * 64;
  static constexpr int PITCH = BK + 16;     // LDS row pitch in bytes
  static constexpr int STAGE = (BM + BN) * PITCH;
  static constexpr int CHUNKS = BK / 16;    // 16-byte chunks per staged row
  static constexpr int A_LOADS = BM * CHUNKS / THREADS;
  static constexpr int B_LOADS = BN * CHUNKS / THREADS;
  static_assert(BM * CHUNKS % THREADS == 0 && BN * CHUNKS % THREADS == 0, "tile/threads mismatch");
  static_assert(BK % 64 == 0, "BK must be a multiple of the MFMA K (64)");
};

using Cfg = TileCfg<2, 2, 8, 4, 64>;  // 256 x 128 tile, waves of 128 x 64
constexpr int kGroupM = 8;

__device__ __forceinline__ int xcd_remap(int id, int num) {
  constexpr int X = 8;
  const int per = num / X, rem = num % X;
  const int xcd = id % X, local = id / X;
  return xcd * per + min(xcd, rem) + local;
}

// Global -> registers for one stage of ROWS rows x C::BK bytes. Rows past
// the matrix edge re-read the last valid row (results are discarded); K
// bytes past the end read as zero.
template <class C, int LOADS>
__device__ __forceinline__ void load_stage(const int8_t* __restrict__ base, int ld, int rows, int row0,
                                           int k0, int K, i32x4 (&r)[LOADS]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int idx = t + C::THREADS * i;
    const int row = idx / C::CHUNKS;
    const int c = (idx % C::CHUNKS) * 16;
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

template <class C, int LOADS>
__device__ __forceinline__ void store_stage(int8_t* s, const i32x4 (&r)[LOADS]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int idx = t + C::THREADS * i;
    *reinterpret_cast<i32x4*>(s + (idx / C::CHUNKS) * C::PITCH + (idx % C::CHUNKS) * 16) = r[i];
  }
}

template <class C, int EPI>
__device__ __forceinline__ void epilogue(const GemmI8Args& p,
                                         const i32x4 (&acc)[C::WM][C::WN], int rb,
                                         int cb, int lr, int lg) {
  constexpr int WM = C::WM, WN = C::WN;
  if constexpr (EPI == kEpiI32) {
#pragma unroll
    for (int bm = 0; bm < WM; ++bm)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = rb + bm * 16 + lg * 4 + r;
        if (row >= p.M) continue;
#pragma unroll
        for (int bn = 0; bn < WN; ++bn) {
          const int col = cb + bn * 16 + lr;
          if (col < p.N) p.C_i32[static_cast<size_t>(row) * p.ldc + col] = acc[bm][bn][r];
        }
      }
    return;
  } else {
    float ws[WN], bs[WN];
#pragma unroll
    for (int bn = 0; bn < WN; ++bn) {
      const int col = cb + bn * 16 + lr;
      const bool ok = col < p.N;
      ws[bn] = ok ? p.w_scale[col] : 0.0f;
      bs[bn] = (ok && p.bias) ? p.bias[col] : 0.0f;
    }
    if constexpr (EPI == kEpiQkvRopeF32) {
      static_assert(WN == 4, "QKV epilogue needs 64-column (one head) waves");
      if (cb >= p.N) return;
      // fp32 Q|K|V row of width 3*d_model: the wave's 64 columns are one
      // head of Q, K or V; rotary pairs (i, i+32) are blocks (0,2), (1,3).
      const int which = cb / p.d_model;
#pragma unroll
      for (int bm = 0; bm < WM; ++bm)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rb + bm * 16 + lg * 4 + r;
          if (row >= p.M) continue;
          const float as = p.a_scale[row];
          float v[WN];
#pragma unroll
          for (int bn = 0; bn < WN; ++bn)
            v[bn] = __builtin_fmaf(static_cast<float>(acc[bm][bn][r]), as * ws[bn], bs[bn]);
          if (which < 2) {
            if (which == 0) {
#pragma unroll
              for (int bn = 0; bn < WN; ++bn) v[bn] *= p.q_scale;
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
          }
          float* dst = p.C_f32 + static_cast<size_t>(row) * p.ldc + cb + lr;
#pragma unroll
          for (int bn = 0; bn < WN; ++bn) dst[bn * 16] = v[bn];
        }
      return;
    } else if constexpr (EPI == kEpiQkvRope) {
      static_assert(WN == 4, "QKV epilogue needs 64-column (one head) waves");
      // With an odd head count the last tile's second wave lies past N.
      if (cb >= p.N) return;
      // The wave's 64 columns are exactly one head of Q, K or V. Lane
      // column lr of block bn holds head dim bn*16+lr, so the rotary pairs
      // (i, i+32) sit in blocks (0,2) and (1,3) of the same lane and row.
      const int which = cb / p.d_model;
      const int hcol = cb - which * p.d_model;
#pragma unroll
      for (int bm = 0; bm < WM; ++bm)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rb + bm * 16 + lg * 4 + r;
          if (row >= p.M) continue;
          const float as = p.a_scale[row];
          float v[WN];
#pragma unroll
          for (int bn = 0; bn < WN; ++bn)
            v[bn] = __builtin_fmaf(static_cast<float>(acc[bm][bn][r]), as * ws[bn], bs[bn]);
          const size_t o = static_cast<size_t>(row) * p.d_model + hcol + lr;
          if (which == 2) {
#pragma unroll
            for (int bn = 0; bn < WN; ++bn) p.v_out[o + bn * 16] = f32_to_f16_bits(v[bn]);
            continue;
          }
          if (which == 0) {
#pragma unroll
            for (int bn = 0; bn < WN; ++bn) v[bn] *= p.q_scale;
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
          if (p.qk_fp16) {
#pragma unroll
            for (int bn = 0; bn < WN; ++bn) dst[o + bn * 16] = f32_to_f16_bits(v[bn]);
          } else {
#pragma unroll
            for (int bn = 0; bn < WN; ++bn) dst[o + bn * 16] = f32_to_bf16_bits(v[bn]);
          }
        }
      return;
    } else {
      float tmax = 0.0f;
#pragma unroll
      for (int bm = 0; bm < WM; ++bm)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rb + bm * 16 + lg * 4 + r;
          const bool rok = row < p.M;
          const float as = rok ? p.a_scale[row] : 0.0f;
          float rmax = 0.0f;
#pragma unroll
          for (int bn = 0; bn < WN; ++bn) {
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

template <class C, int EPI>
__global__ __launch_bounds__(C::THREADS, 2) void gemm_i8_kernel(const GemmI8Args p) {
  __shared__ __attribute__((aligned(16))) int8_t smem[2 * C::STAGE];

  const int tiles_m = (p.M + C::BM - 1) / C::BM;
  const int tiles_n = (p.N + C::BN - 1) / C::BN;
  const int pid = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  const int per_group = kGroupM * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in_group = pid - group * per_group;
  const int m0 = (first_m + in_group % gsize) * C::BM;
  const int n0 = (in_group / gsize) * C::BN;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
  const int lr = lane & 15, lg = lane >> 4;

  i32x4 acc[C::WM][C::WN];
#pragma unroll
  for (int i = 0; i < C::WM; ++i)
#pragma unroll
    for (int j = 0; j < C::WN; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

  i32x4 ra[C::A_LOADS], rb[C::B_LOADS];
  const int nk = (p.K + C::BK - 1) / C::BK;
  load_stage<C>(p.A, p.lda, p.M, m0, 0, p.K, ra);
  load_stage<C>(p.W, p.ldw, p.N, n0, 0, p.K, rb);
  store_stage<C>(smem, ra);
  store_stage<C>(smem + C::BM * C::PITCH, rb);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int8_t* cur = smem + (kt & 1) * C::STAGE;
    const bool more = kt + 1 < nk;
    if (more) {
      load_stage<C>(p.A, p.lda, p.M, m0, (kt + 1) * C::BK, p.K, ra);
      load_stage<C>(p.W, p.ldw, p.N, n0, (kt + 1) * C::BK, p.K, rb);
    }
    const int8_t* sa = cur + (wm * C::WM * 16 + lr) * C::PITCH + lg * 16;
    const int8_t* sb = cur + C::BM * C::PITCH + (wn * C::WN * 16 + lr) * C::PITCH + lg * 16;
#pragma unroll
    for (int kk = 0; kk < C::BK / 64; ++kk) {
      i32x4 fa[C::WM], fb[C::WN];
#pragma unroll
      for (int j = 0; j < C::WN; ++j)
        fb[j] = *reinterpret_cast<const i32x4*>(sb + j * 16 * C::PITCH + kk * 64);
#pragma unroll
      for (int i = 0; i < C::WM; ++i)
        fa[i] = *reinterpret_cast<const i32x4*>(sa + i * 16 * C::PITCH + kk * 64);
#pragma unroll
      for (int i = 0; i < C::WM; ++i)
#pragma unroll
        for (int j = 0; j < C::WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      int8_t* nxt = smem + ((kt + 1) & 1) * C::STAGE;
      store_stage<C>(nxt, ra);
      store_stage<C>(nxt + C::BM * C::PITCH, rb);
    }
    __syncthreads();
  }

  epilogue<C, EPI>(p, acc, m0 + wm * C::WM * 16, n0 + wn * C::WN * 16, lr, lg);
}

}  // namespace

hipError_t launch_gemm_i8(const GemmI8Args& p, int epi, hipStream_t s) {
  if (p.M <= 0 || p.N <= 0) return hipSuccess;
  const int tiles = ((p.M + Cfg::BM - 1) / Cfg::BM) * ((p.N + Cfg::BN - 1) / Cfg::BN);
  const dim3 grid(tiles), block(Cfg::THREADS);
  switch (epi) {
    case kEpiI32: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiI32>), grid, block, 0, s, p); break;
    case kEpiF32: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiF32>), grid, block, 0, s, p); break;
    case kEpiF32Gelu: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiF32Gelu>), grid, block, 0, s, p); break;
    case kEpiF32Resid: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiF32Resid>), grid, block, 0, s, p); break;
    case kEpiQkvRope: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiQkvRope>), grid, block, 0, s, p); break;
    case kEpiF32GeluQ: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiF32GeluQ>), grid, block, 0, s, p); break;
    case kEpiQkvRopeF32: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiQkvRopeF32>), grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace esm_gfx950
