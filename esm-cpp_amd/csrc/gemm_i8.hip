// W8A8 INT8 GEMM for gfx950 with int32 accumulation and fused epilogues
// (dequant + bias, GELU, residual add, QKV split with Q-scale and rotary
// embedding). Two kernels:
//   - gemm_i8_v3_kernel (namespace v3 below): the main path whenever K is a
//     multiple of 128 and rows are 16-byte aligned -- v_mfma_i32_32x32x32_i8,
//     256x256 or 320x256 tiles, direct global -> LDS stage loads;
//   - gemm_i8_kernel (TileCfg, described next): the general fallback for any
//     other shape, v_mfma_i32_16x16x64_i8.
//
// Replaces the inner product of esm::kernels::LinearInt8
// (reference src/kernels/gemm_int8.cpp:510-555 LinearVnni and
// src/kernels/gemm_amx.cpp:218-309 LinearAmx). The reference dequantises
// with out = fma(float(acc), w_scale[n] * act_scale, bias[n])
// (gemm_int8.cpp:109-126); the epilogue here uses the same expression with
// a per-row activation scale, which equals the per-tensor scale when every
// row carries the tensor's scale.
//
// Fallback tiling (TileCfg): a 256-thread workgroup owns a 256x128 output tile; its
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
#include <atomic>
#include <cmath>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "x86_math.hpp"

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

// Output tile of this workgroup: ids are first spread so that each XCD
// (workgroup id mod 8) owns a contiguous range, then walked in groups of
// kGroupM row tiles so consecutive tiles on one XCD share W columns and A rows
// in that XCD's L2.
__device__ __forceinline__ void tile_origin_of(int id, int M, int N, int BM, int BN, int* m0, int* n0) {
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  const int pid = xcd_remap(id, tiles_m * tiles_n);
  const int per_group = kGroupM * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in_group = pid - group * per_group;
  *m0 = (first_m + in_group % gsize) * BM;
  *n0 = (in_group / gsize) * BN;
}

__device__ __forceinline__ void tile_origin(int M, int N, int BM, int BN, int* m0, int* n0) {
  tile_origin_of(blockIdx.x, M, N, BM, BN, m0, n0);
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

// Epilogue of one wave's WM x WN blocks of 16x16 int32 accumulators; the
// block (bm, bn) element r of lane (lr, lg) is row rb + bm*16 + lg*4 + r,
// column cb + bn*16 + lr.
template <int WM, int WN, int EPI>
__device__ __forceinline__ void epilogue(const GemmI8Args& p, const i32x4 (&acc)[WM][WN], int rb,
                                         int cb, int lr, int lg) {
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
      static_assert(WN % 4 == 0, "QKV epilogue needs whole 64-column heads per wave");
      // fp32 Q|K|V row of width 3*d_model. Each group of four blocks is one
      // head of Q, K or V; lane column lr of block g*4+j holds head dim
      // j*16+lr, so the rotary pairs (i, i+32) are blocks (0,2) and (1,3).
#pragma unroll
      for (int g = 0; g < WN / 4; ++g) {
        const int hc = cb + g * 64;
        if (hc >= p.N) break;
        const int which = hc / p.d_model;
#pragma unroll
        for (int bm = 0; bm < WM; ++bm)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = rb + bm * 16 + lg * 4 + r;
            if (row >= p.M) continue;
            const float as = p.a_scale[row];
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
              v[j] = __builtin_fmaf(static_cast<float>(acc[bm][g * 4 + j][r]), as * ws[g * 4 + j], bs[g * 4 + j]);
            if (which < 2) {
              if (which == 0) {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] *= p.q_scale;
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
            float* dst = p.C_f32 + static_cast<size_t>(row) * p.ldc + hc + lr;
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[j * 16] = v[j];
          }
      }
      return;
    } else if constexpr (EPI == kEpiQkvRope) {
      static_assert(WN % 4 == 0, "QKV epilogue needs whole 64-column heads per wave");
      // Same head-group layout as above; Q/K stored bf16 or fp16, V fp16,
      // each as [M, d_model].
#pragma unroll
      for (int g = 0; g < WN / 4; ++g) {
        const int hc = cb + g * 64;
        if (hc >= p.N) break;
        const int which = hc / p.d_model;
        const int hcol = hc - which * p.d_model;
#pragma unroll
        for (int bm = 0; bm < WM; ++bm)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = rb + bm * 16 + lg * 4 + r;
            if (row >= p.M) continue;
            const float as = p.a_scale[row];
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
              v[j] = __builtin_fmaf(static_cast<float>(acc[bm][g * 4 + j][r]), as * ws[g * 4 + j], bs[g * 4 + j]);
            const size_t o = static_cast<size_t>(row) * p.d_model + hcol + lr;
            if (which == 2) {
#pragma unroll
              for (int j = 0; j < 4; ++j) p.v_out[o + j * 16] = f32_to_f16_bits(v[j]);
              continue;
            }
            if (which == 0) {
#pragma unroll
              for (int j = 0; j < 4; ++j) v[j] *= p.q_scale;
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
              for (int j = 0; j < 4; ++j) dst[o + j * 16] = f32_to_f16_bits(v[j]);
            } else {
#pragma unroll
              for (int j = 0; j < 4; ++j) dst[o + j * 16] = f32_to_bf16_bits(v[j]);
            }
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
            if constexpr (EPI == kEpiF32GeluAs) v = 0.5f * gelu2_as(v);
            if constexpr (EPI == kEpiF32GeluX86) v = gelu_x86(v);
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
          if constexpr (EPI == kEpiF32Gelu || EPI == kEpiF32GeluQ || EPI == kEpiF32GeluAs || EPI == kEpiF32GeluX86 ||
                        EPI == kEpiF32) {
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
      if constexpr (EPI == kEpiF32Gelu || EPI == kEpiF32GeluQ || EPI == kEpiF32GeluAs || EPI == kEpiF32GeluX86 ||
                    EPI == kEpiF32) {
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

  int m0, n0;
  tile_origin(p.M, p.N, C::BM, C::BN, &m0, &n0);

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

  epilogue<C::WM, C::WN, EPI>(p, acc, m0 + wm * C::WM * 16, n0 + wn * C::WN * 16, lr, lg);
}


// ---------------------------------------------------------------------------
// Pipelined kernel for K % 128 == 0 (every ESM-2 linear): 256x256 workgroup
// tile, eight waves (2 x 4) of 128x64, two waves per SIMD, on
// v_mfma_i32_32x32x32_i8 (4 x 2 blocks of 32x32 per wave).
//
// Staging: K advances 128 bytes per stage; each stage moves global -> LDS
// with global_load_lds_dwordx4, one instruction per 8 rows x 128 bytes, so
// every request is a whole 128-byte cache line (L2 -> CU throughput on this
// part measured 2.3x that of 64-byte row pieces). Lane l of the instruction
// writes LDS bytes [16l, 16l+16) of its 1 KB block; it loads row l/8 of the
// block and 16-byte chunk (l%8) ^ (l/8) ^ (block & 1), so the LDS copy holds
// chunk c of row r at position c ^ r ^ (block & 1). That XOR keeps the
// 32x32x32 fragment reads (32 rows x one chunk per half-wave) on distinct
// banks. Two 64 KB stages ping-pong with one barrier per stage: the barrier
// publishes stage kt (each wave waited for its own loads) and retires the
// reads of stage kt-1, whose buffer then receives stage kt+1 while stage
// kt's 64 MFMAs per wave run.
namespace v3 {

constexpr int WAVES_M = 2;  // waves down the tile
constexpr int BN = 256;     // tile width
constexpr int BK = 128;

// Tile height: BLK_M 32x32 row blocks per wave, BM = 64 * BLK_M rows (1: 64,
// 2: 128, 4: 256, 5: 320). For grids that fill the CUs the launcher picks the
// height that needs the fewer rows' worth of workgroup rounds (a 256-row grid
// that spills a few tiles into one more round often fits in fewer rounds as
// 320-row tiles), 320 on a tie; small-M grids take shorter tiles so that
// more CUs share the rows (gemm_i8_tile_rows).
// Wave layout: BLK_N 32x32 column blocks per wave, WAVES_N = 8 / BLK_N waves
// across the 256 columns. Every launch uses BLK_N 2: eight waves, two per
// SIMD. (BLK_N 4, four waves of 128x128 with the accumulators in AGPRs, reads
// 29% fewer LDS bytes per MFMA but ran 11-27% slower: one wave per SIMD
// leaves the matrix core idle at every barrier and LDS wait.)
template <int BLK_M_, int BLK_N_ = 2>
struct Tile {
  static constexpr int BLK_M = BLK_M_, BLK_N = BLK_N_;
  static constexpr int WAVES_N = 8 / BLK_N;
  static constexpr int kWaves = WAVES_M * WAVES_N;
  static constexpr int kThreads = kWaves * 64;
  static_assert(WAVES_N * BLK_N * 32 == BN, "waves x blocks must cover the 256 tile columns");
  static constexpr int BM = WAVES_M * BLK_M * 32;
  static constexpr int kBlocks = (BM + BN) / 8;  // 1 KB blocks per stage
  static constexpr int kPer = kBlocks / kWaves;
  static constexpr int kStage = kBlocks * 1024;  // 64 KB (BM 256) / 72 KB (BM 320)
  // Stage buffers: three for the short tiles (40 / 48 KB each), so the loads
  // run two stages ahead of the MFMAs; the tall tiles' two fill the LDS.
  static constexpr int kNStage = BLK_M <= 2 ? 3 : 2;
  // RoPE cos / sin rows of a tile staged in LDS, transposed: [32 dims][BM
  // rows + pad], so that a lane reads four consecutive rows of one dim at once.
  static constexpr int kRopeTPitch = BM + 4;
  static_assert(kBlocks % kWaves == 0, "load blocks per wave");
};

// One 16-byte-per-lane global -> LDS load (global_load_lds_dwordx4), issued
// from inline asm: M0 holds the wave's LDS destination (uniform), and one
// wait state separates the M0 write from the load. Issued through the
// compiler builtin instead, the compiler's wait insertion would hold the
// fragment reads of the other stage buffer until these loads complete (it
// cannot tell the two buffers apart), which serialises the double buffer.
// Completion is awaited explicitly: s_waitcnt vmcnt(0) and a barrier before
// a stage is read. The load is addressed as a wave-uniform base (SGPRs) plus
// a 32-bit lane offset: one VGPR per load instead of a 64-bit address pair.
// `lds` is the destination's LDS byte address.
__device__ __forceinline__ void dma16_async_so(const int8_t* base, uint32_t off, uint32_t lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0v)
               : "memory", "m0");
#endif
}

// LDS byte address of a __shared__ object (one address-space cast, made
// once, instead of a null-checked cast per load).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

__device__ __forceinline__ i32x16 mfma32(i32x4 a, i32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// Byte offset of (row R, 16-byte chunk c) in a stage.
__device__ __forceinline__ int soff(int R, int c) {
  const int b = R >> 3, r = R & 7;
  return b * 1024 + ((r << 3) + (c ^ r ^ (b & 1))) * 16;
}

// Epilogue of one wave's BLK_M x BLK_N blocks of 32x32 int32 accumulators.
// Element r of block (i, j) in lane l is tile row lr0 + i*32 + (r/4)*8 + r%4
// (lr0 = wm*BLK_M*32 + (l/32)*4) and tile column lc0 + j*32 (lc0 =
// wn*BLK_N*32 + l%32): each store instruction writes 128 contiguous bytes of
// two rows. Addresses are 32-bit offsets from the tile's origin (uniform), so
// no per-element 64-bit arithmetic is needed. FULL: the tile lies inside M x N
// and no element needs a bounds check.
// s_as / s_ws / s_bs: the tile's activation scales (by tile row), weight
// scales and bias (by tile column), staged in LDS at kernel start. s_cosT /
// s_sinT: the tile rows' RoPE tables (first half of each row; the model's
// tables repeat it in the second half), staged after the main loop.
// base + off elements, with the byte offset formed in 32 bits so that the
// store adds one 32-bit lane offset to a uniform 64-bit base.
template <class T>
__device__ __forceinline__ T* at(T* base, uint32_t off) {
  return reinterpret_cast<T*>(reinterpret_cast<char*>(base) + off * static_cast<uint32_t>(sizeof(T)));
}

// Element of tile row R (wave-uniform) at the lane's byte offset: the row
// address is scalar (SGPRs), the lane offset a loop-invariant VGPR, and a
// constant column step becomes the store's immediate offset, so a store
// needs no per-element address arithmetic.
template <class T>
__device__ __forceinline__ T* row_at(T* tile, uint32_t ldc, int R, uint32_t lane_byte) {
  char* row = reinterpret_cast<char*>(tile) + static_cast<size_t>(static_cast<uint32_t>(R) * ldc) * sizeof(T);
  return reinterpret_cast<T*>(row + lane_byte);
}

// Buffer resource over a tile's output (or residual input): the epilogues
// address every access as this base plus a 32-bit lane offset (VGPR, the
// same for every row) plus the row's 32-bit byte offset (SGPR), which the
// buffer instructions add themselves -- no per-access address arithmetic.
// Offsets stay far below the 4 GiB record range. Word 3 selects a 32-bit
// data format (raw, untyped accesses).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, 0x00020000);
}
constexpr int kBufNT = 2;  // buffer access aux bits: non-temporal

// One 64-column head of Q (WHICH 0), K (1) or V (2): blocks (2g, 2g+1) of the
// wave, so lane column l32 holds head dims l32 and 32 + l32 -- exactly a
// rotary pair. hc: the head's first column relative to the tile origin.
// QS: multiply Q by p.q_scale (skipped when the model folded it into the Q
// weights, p.q_scale == 1, so the product would be exact anyway).
// kEpiQkvSplit: the Q columns' weight scales and bias arrive already
// multiplied by p.q_prescale (see the kernel's scale staging).
template <int BLK_M, int BLK_N, int EPI, bool FULL, int WHICH, bool QS = true>
__device__ __forceinline__ void qkv_head(const GemmI8Args& p, const i32x16 (&acc)[BLK_M][BLK_N], int g, int hc,
                                         int wr0, int lr0, int l32, const float* s_as, const float (&ws)[BLK_N],
                                         const float (&bs)[BLK_N], const float* s_cosT, const float* s_sinT, int m0,
                                         int n0) {
  constexpr int kRopeTPitch = Tile<BLK_M, BLK_N>::kRopeTPitch;
  const uint32_t ldc = p.ldc;
  const uint32_t dm = p.d_model;
  // Row offsets: the lane's first row (lr0) times the stride once; the rest
  // of each row index is a compile-time constant times a uniform stride.
  const uint32_t lane_b =
      (static_cast<uint32_t>(lr0 - wr0) * ldc + static_cast<uint32_t>(hc + l32)) * 4u;  // 4-byte outputs
  const uint32_t lane_d = static_cast<uint32_t>(lr0) * dm + static_cast<uint32_t>(n0 + hc - WHICH * p.d_model + l32);
  // kEpiQkvSplit layout of a [M, 3 d] word row: Q words [0, d), K hi / lo
  // fp16 planes in words [d, 2d), V's in [2d, 3d). Every head keeps 64
  // positions per part in the order (dim 0, dim 32, dim 1, dim 33, ...): the
  // lane's rotary pair (l32, 32 + l32) lands at positions 2 l32, 2 l32 + 1.
  // lane_s: the lane's byte offset from the tile's first row at column 0.
  const uint32_t head_dim0 = static_cast<uint32_t>(n0 + hc - WHICH * p.d_model);  // head's first dim
  const uint32_t col_s = WHICH == 0 ? head_dim0 + 2u * l32 : WHICH * dm + head_dim0 / 2u + l32;
  const uint32_t lane_s = (static_cast<uint32_t>(lr0 - wr0) * ldc + col_s) * 4u;
#pragma unroll
  for (int i = 0; i < BLK_M; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int lr = lr0 + i * 32 + q * 8;  // rows lr .. lr+3 hold elements r = 4q .. 4q+3
      const float4 as4 = *reinterpret_cast<const float4*>(s_as + lr);
      float4 c4, s4;
      if constexpr (WHICH < 2) {
        c4 = *reinterpret_cast<const float4*>(s_cosT + l32 * kRopeTPitch + lr);
        s4 = *reinterpret_cast<const float4*>(s_sinT + l32 * kRopeTPitch + lr);
      }
      const float asv[4] = {as4.x, as4.y, as4.z, as4.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int r = 4 * q + u;
        if (!FULL && m0 + lr + u >= p.M) continue;
        float x1 = __builtin_fmaf(static_cast<float>(acc[i][2 * g][r]), asv[u] * ws[2 * g], bs[2 * g]);
        float x2 = __builtin_fmaf(static_cast<float>(acc[i][2 * g + 1][r]), asv[u] * ws[2 * g + 1], bs[2 * g + 1]);
        if constexpr (WHICH == 0 && QS) {
          x1 *= p.q_scale;
          x2 *= p.q_scale;
        }
        if constexpr (WHICH < 2) {
          const float c = u == 0 ? c4.x : u == 1 ? c4.y : u == 2 ? c4.z : c4.w;
          const float sn = u == 0 ? s4.x : u == 1 ? s4.y : u == 2 ? s4.z : s4.w;
          // Explicit fused forms: every instantiation (full / edge tile)
          // rounds a row identically, whatever the compiler would contract.
          float y1 = __builtin_fmaf(x1, c, -(x2 * sn));
          if constexpr (EPI == kEpiQkvRopeF32) {
            if (p.rope_x86) y1 = __builtin_fmaf(-x2, sn, x1 * c);
          }
          const float y2 = __builtin_fmaf(x2, c, x1 * sn);
          x1 = y1;
          x2 = y2;
        }
        // Offsets from the tile origin: unsigned 32-bit, so the store adds a
        // lane offset to a uniform base.
        const uint32_t dr = static_cast<uint32_t>(i * 32 + q * 8 + u);
        if constexpr (EPI == kEpiQkvRopeF32) {
          float* tile = p.C_f32 + static_cast<size_t>(m0) * ldc + n0;
          float* dst = row_at(tile, ldc, wr0 + static_cast<int>(dr), lane_b);
          dst[0] = x1;
          dst[32] = x2;
        } else if constexpr (EPI == kEpiQkvSplit) {
          // Q: x already carries q_prescale (a power of two folded into the
          // staged scales and bias: fma(acc, a*(w*2^e), b*2^e) and every later
          // product and fma are the unfolded values times 2^e exactly).
          // Buffer stores relative to the tile's first row: the lane offset
          // lane_s (VGPR) plus the row's byte offset (SGPR).
          const __amdgpu_buffer_rsrc_t rows = tile_rsrc(reinterpret_cast<uint32_t*>(p.C_f32) +
                                                        static_cast<size_t>(m0) * ldc);
          const uint32_t soff = (static_cast<uint32_t>(wr0) + dr) * ldc * 4u;
          if constexpr (WHICH == 0) {
            // Q words, the rotary pair adjacent: one 8-byte store per lane.
            const uint32_t w1 = split_f16_word(x1), w2 = split_f16_word(x2);
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{w1, w2}, rows, lane_s, soff, kBufNT);
          } else {
            // K / V: the pair's fp16 hi parts in the hi plane, lo parts in
            // the lo plane (d / 2 words further), each pair converted at
            // once (the values pinned in registers first, so the conversion
            // rounds these fp32 values and no fused form of them).
            asm("" : "+v"(x1), "+v"(x2));
            uint32_t hw, lw;
            split_pair(x1, x2, &hw, &lw);
            __builtin_amdgcn_raw_buffer_store_b32(hw, rows, lane_s, soff, kBufNT);
            __builtin_amdgcn_raw_buffer_store_b32(lw, rows, lane_s, soff + dm * 2u, kBufNT);
          }
        } else {
          // [M, d_model] outputs; column of the head inside its Q / K / V part.
          const uint32_t o = lane_d + dr * dm;
          if constexpr (WHICH == 2) {
            uint16_t* vb = p.v_out + static_cast<size_t>(m0) * dm;
            *at(vb, o) = f32_to_f16_bits(x1);
            *at(vb, o + 32) = f32_to_f16_bits(x2);
          } else {
            uint16_t* dst = (WHICH == 0 ? p.q_out : p.k_out) + static_cast<size_t>(m0) * dm;
            *at(dst, o) = p.qk_fp16 ? f32_to_f16_bits(x1) : f32_to_bf16_bits(x1);
            *at(dst, o + 32) = p.qk_fp16 ? f32_to_f16_bits(x2) : f32_to_bf16_bits(x2);
          }
        }
      }
    }
}

// MAX: also reduce |out| into p.row_absmax / p.tensor_absmax (whichever is set).
// c_i32: the int32 output (kEpiI32), p.C_i32 or, for a split-K launch, the
// split's own plane of it.
template <int BLK_M, int BLK_N, int EPI, bool FULL, bool MAX>
__device__ __forceinline__ void epilogue32(const GemmI8Args& p, const i32x16 (&acc)[BLK_M][BLK_N], int wm, int wn,
                                           int l32, int hi, const float* s_as, const float* s_ws,
                                           const float* s_bs, const float* s_cosT, const float* s_sinT, int m0,
                                           int n0, int32_t* c_i32, bool nan_risk) {
  const int lr0 = wm * BLK_M * 32 + hi * 4;
  const int lc0 = wn * BLK_N * 32 + l32;
  const uint32_t ldc = p.ldc;
  auto col_ok = [&](int lc) { return FULL || n0 + lc < p.N; };
  // Tile rows split into a wave-uniform part (wm's rows + block offsets) and
  // the lane's half-wave offset hi * 4, which joins the lane's column in a
  // per-lane byte offset.
  const int wr0 = wm * BLK_M * 32;
  if constexpr (EPI == kEpiI32) {
    int32_t* tile = c_i32 + static_cast<size_t>(m0) * ldc + n0;
    const uint32_t lane_b = (static_cast<uint32_t>(hi * 4) * ldc + static_cast<uint32_t>(lc0)) * 4u;
#pragma unroll
    for (int i = 0; i < BLK_M; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dr = i * 32 + (r >> 2) * 8 + (r & 3);
        int32_t* dst = row_at(tile, ldc, wr0 + dr, lane_b);
#pragma unroll
        for (int j = 0; j < BLK_N; ++j)
          if ((FULL || m0 + lr0 + dr < p.M) && col_ok(lc0 + j * 32))
            __builtin_nontemporal_store(acc[i][j][r], dst + j * 32);
      }
    return;
  } else {
    float ws[BLK_N], bs[BLK_N];
#pragma unroll
    for (int j = 0; j < BLK_N; ++j) {
      ws[j] = s_ws[lc0 + j * 32];
      bs[j] = s_bs[lc0 + j * 32];
    }
    if constexpr (EPI == kEpiQkvRopeF32 || EPI == kEpiQkvRope || EPI == kEpiQkvSplit) {
      static_assert(BLK_N % 2 == 0, "QKV epilogue needs whole 64-column heads per wave");
#pragma unroll
      for (int g = 0; g < BLK_N / 2; ++g) {
        const int hc = wn * BLK_N * 32 + g * 64;  // uniform: the wave index is
        if (!FULL && n0 + hc >= p.N) break;
        const int which = (n0 + hc) / p.d_model;
        if (which == 0 && p.q_scale == 1.0f)
          qkv_head<BLK_M, BLK_N, EPI, FULL, 0, false>(p, acc, g, hc, wr0, lr0, l32, s_as, ws, bs, s_cosT, s_sinT, m0,
                                                      n0);
        else if (which == 0)
          qkv_head<BLK_M, BLK_N, EPI, FULL, 0>(p, acc, g, hc, wr0, lr0, l32, s_as, ws, bs, s_cosT, s_sinT, m0, n0);
        else if (which == 1)
          qkv_head<BLK_M, BLK_N, EPI, FULL, 1>(p, acc, g, hc, wr0, lr0, l32, s_as, ws, bs, s_cosT, s_sinT, m0, n0);
        else
          qkv_head<BLK_M, BLK_N, EPI, FULL, 2>(p, acc, g, hc, wr0, lr0, l32, s_as, ws, bs, s_cosT, s_sinT, m0, n0);
      }
      return;
    } else if constexpr (EPI == kEpiF32R24) {
      // The lane's two columns (l32 and 32 + l32 of the wave's 64) round to
      // 24 bits (+0x80, then the top three bytes). Their high halves go out
      // as one 4-byte word at stored positions 2 l32, 2 l32 + 1 of the group:
      // whole 128-byte rows of the high plane per half-wave. The low plane
      // interleaves row pairs (rows 2k and 2k + 1 share 2 ldc bytes; byte
      // (r & ~1) ldc + 4 (p / 2) + 2 (r & 1) + (p & 1) holds row r, stored
      // position p), so the lane's rows R and R + 1 (R even) go out as one
      // 4-byte word and each half-wave store writes a whole 128-byte line.
      static_assert(BLK_N == 2, "the 24-bit layout pairs a lane's two 32-column blocks");
      const int gc = wn * 64;  // the wave's column group inside the tile
      if (!FULL && n0 + gc >= p.N) return;
      const __amdgpu_buffer_rsrc_t rh = tile_rsrc(p.C_f16 + static_cast<size_t>(m0) * ldc + n0 + gc);
      const __amdgpu_buffer_rsrc_t rl = tile_rsrc(p.C_u8 + static_cast<size_t>(m0) * ldc + 2 * (n0 + gc));
      const uint32_t lane_h = (static_cast<uint32_t>(hi * 4) * ldc + static_cast<uint32_t>(2 * l32)) * 2u;
      const uint32_t lane_l = static_cast<uint32_t>(hi * 4) * ldc + static_cast<uint32_t>(4 * l32);
      // A NaN's bit pattern must not take the rounding add (it could carry
      // into the sign or leave an infinity). fma(float(acc), a_scale *
      // w_scale, bias) can be NaN only when a scale or bias is not finite or
      // a scale product overflows; the prologue checks the tile's scales and
      // biases (nan_risk), and only such a tile maps NaN to the quiet NaN
      // value by value.
      auto pass = [&](auto fix_nan) {
#pragma unroll
        for (int i = 0; i < BLK_M; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int lr = lr0 + i * 32 + q * 8;
            const float4 as4 = *reinterpret_cast<const float4*>(s_as + lr);
            const float asv[4] = {as4.x, as4.y, as4.z, as4.w};
#pragma unroll
            for (int u2 = 0; u2 < 4; u2 += 2) {
              uint32_t lo[2];  // the low bytes of rows R and R + 1 at positions 2 l32, 2 l32 + 1
#pragma unroll
              for (int h = 0; h < 2; ++h) {
                const int u = u2 + h, r = 4 * q + u;
                const float v0 = __builtin_fmaf(static_cast<float>(acc[i][0][r]), asv[u] * ws[0], bs[0]);
                const float v1 = __builtin_fmaf(static_cast<float>(acc[i][1][r]), asv[u] * ws[1], bs[1]);
                uint32_t b0 = __float_as_uint(v0) + 0x80u, b1 = __float_as_uint(v1) + 0x80u;
                if constexpr (decltype(fix_nan)::value) {
                  b0 = __builtin_isnan(v0) ? 0x7fc00000u : b0;
                  b1 = __builtin_isnan(v1) ? 0x7fc00000u : b1;
                }
                lo[h] = __builtin_amdgcn_perm(b1, b0, 0x0c0c0501u);
                const uint32_t R = static_cast<uint32_t>(wr0 + i * 32 + q * 8 + u);
                if (FULL || m0 + lr + u < p.M)
                  __builtin_amdgcn_raw_buffer_store_b32(__builtin_amdgcn_perm(b1, b0, 0x07060302u), rh, lane_h,
                                                        R * ldc * 2u, kBufNT);
              }
              const uint32_t R0 = static_cast<uint32_t>(wr0 + i * 32 + q * 8 + u2);
              if (FULL || m0 + lr + u2 + 1 < p.M) {
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_amdgcn_perm(lo[1], lo[0], 0x05040100u), rl, lane_l,
                                                      R0 * ldc, kBufNT);
              } else if (m0 + lr + u2 < p.M) {
                // The last row of an odd row count: its own two bytes only.
                __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(lo[0]), rl, lane_l, R0 * ldc, kBufNT);
              }
            }
          }
      };
      if (__builtin_expect(nan_risk, 0))
        pass(std::true_type{});
      else
        pass(std::false_type{});
      return;
    } else if constexpr (EPI == kEpiF32Resid) {
      // C += result, in groups of four rows x BLK_N columns (8 values per
      // lane): the C values of group g + kDist are loaded while group g is
      // formed and stored, so the reads stay in flight behind the work
      // (scheduling barriers keep the compiler from hoisting them all, which
      // would need 160 more registers). The sum is C + v, the residual add's
      // operands and rounding.
      constexpr int kGroups = BLK_M * 4, kDist = BLK_M >= 5 ? 3 : 4;
      const __amdgpu_buffer_rsrc_t rt = tile_rsrc(p.C_f32 + static_cast<size_t>(m0) * ldc + n0);
      const uint32_t lane_b = (static_cast<uint32_t>(hi * 4) * ldc + static_cast<uint32_t>(lc0)) * 4u;
      // Byte offset of tile row R (uniform) plus column block j.
      auto roff = [&](int R, int j) { return static_cast<uint32_t>(R) * ldc * 4u + static_cast<uint32_t>(j * 128); };
      float res[kDist + 1][4][BLK_N];
      auto load_group = [&](int g, float(&r)[4][BLK_N]) {
        const int dr0 = (g >> 2) * 32 + (g & 3) * 8;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const bool rok = FULL || m0 + lr0 + dr0 + u < p.M;
#pragma unroll
          for (int j = 0; j < BLK_N; ++j)
            r[u][j] = (rok && col_ok(lc0 + j * 32))
                          ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rt, lane_b, roff(wr0 + dr0 + u, j), 0))
                          : 0.0f;
        }
      };
#pragma unroll
      for (int g = 0; g < kDist && g < kGroups; ++g) load_group(g, res[g]);
#pragma unroll
      for (int g = 0; g < kGroups; ++g) {
        if (g + kDist < kGroups) load_group(g + kDist, res[(g + kDist) % (kDist + 1)]);
        const int i = g >> 2, q = g & 3;
        const int lr = lr0 + i * 32 + q * 8;
        const float4 as4 = *reinterpret_cast<const float4*>(s_as + lr);
        const float asv[4] = {as4.x, as4.y, as4.z, as4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const bool rok = FULL || m0 + lr + u < p.M;
#pragma unroll
          for (int j = 0; j < BLK_N; ++j) {
            const float v = __builtin_fmaf(static_cast<float>(acc[i][j][4 * q + u]), asv[u] * ws[j], bs[j]);
            if (rok && col_ok(lc0 + j * 32))
              __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(res[g % (kDist + 1)][u][j] + v), rt, lane_b,
                                                    roff(wr0 + i * 32 + q * 8 + u, j), kBufNT);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      return;
    } else {
      float tmax = 0.0f;
      const uint32_t lane_c = static_cast<uint32_t>(lr0) * ldc + static_cast<uint32_t>(lc0);
      const uint32_t lane_b = (static_cast<uint32_t>(hi * 4) * ldc + static_cast<uint32_t>(lc0)) * 4u;
#pragma unroll
      for (int i = 0; i < BLK_M; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int lr = lr0 + i * 32 + q * 8;
          const float4 as4 = *reinterpret_cast<const float4*>(s_as + lr);
          const float asv[4] = {as4.x, as4.y, as4.z, as4.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int r = 4 * q + u;
            const bool rok = FULL || m0 + lr + u < p.M;
            float rmax = 0.0f;
#pragma unroll
            for (int j = 0; j < BLK_N; ++j) {
              float v = __builtin_fmaf(static_cast<float>(acc[i][j][r]), asv[u] * ws[j], bs[j]);
              if constexpr (EPI == kEpiF32Gelu || EPI == kEpiF32GeluQ) v = gelu_erf(v);
              if constexpr (EPI == kEpiF32GeluAs) v = 0.5f * gelu2_as(v);
              if constexpr (EPI == kEpiF32GeluX86) v = gelu_x86(v);
              if (rok && col_ok(lc0 + j * 32)) {
                const uint32_t off = lane_c + static_cast<uint32_t>(i * 32 + q * 8 + u) * ldc + j * 32;
                if constexpr (EPI == kEpiF32GeluQ) {
                  uint16_t* base = p.C_f16 + static_cast<size_t>(m0) * ldc + n0;
                  *at(base, off) = f32_to_f16_bits(v);
                } else {
                  float* tile = p.C_f32 + static_cast<size_t>(m0) * ldc + n0;
                  __builtin_nontemporal_store(v, row_at(tile, ldc, wr0 + i * 32 + q * 8 + u, lane_b) + j * 32);
                }
                if constexpr (MAX) rmax = fmaxf(rmax, fabsf(v));
              }
            }
            if constexpr (MAX) {
              if (p.row_absmax) {
                // The 32 lanes of a half-wave hold the same row.
#pragma unroll
                for (int o = 16; o >= 1; o >>= 1) rmax = fmaxf(rmax, __shfl_xor(rmax, o, kWave));
                if (l32 == 0 && rok) atomic_max_nonneg(p.row_absmax + m0 + lr + u, rmax);
              }
              tmax = fmaxf(tmax, rmax);
            }
          }
        }
      if constexpr (MAX) {
        // One atomic per workgroup (every wave reaches this point).
        if (p.tensor_absmax) block_atomic_max_nonneg<Tile<BLK_M, BLK_N>::kWaves>(p.tensor_absmax, tmax);
      }
    }
  }
}

template <int BLK_M, int BLK_N, int EPI>
__global__ __launch_bounds__((Tile<BLK_M, BLK_N>::kThreads), 1) void gemm_i8_v3_kernel(const GemmI8Args p) {
  using TL = Tile<BLK_M, BLK_N>;
  constexpr int BM = TL::BM, kPer = TL::kPer, kStage = TL::kStage, kRopeTPitch = TL::kRopeTPitch;
  constexpr int kNStage = TL::kNStage;
  constexpr int kThreads = TL::kThreads, WAVES_N = TL::WAVES_N;
  __shared__ __attribute__((aligned(1024))) int8_t smem[kNStage * kStage];
  __shared__ float s_as[BM], s_ws[BN], s_bs[BN];
  __shared__ int s_pos[BM];
  constexpr bool kRope = EPI == kEpiQkvRopeF32 || EPI == kEpiQkvRope || EPI == kEpiQkvSplit;

  // Split-K (int32 output only): workgroup b takes tile b mod tiles and the
  // (b / tiles)-th of p.splits contiguous ranges of K stages, and writes its
  // partial sums to that split's [M, ldc] plane of C_i32.
  int m0, n0, split = 0;
  int32_t* c_i32 = p.C_i32;
  if (EPI == kEpiI32 && p.splits > 1) {
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    split = blockIdx.x / tiles;
    tile_origin_of(blockIdx.x - split * tiles, p.M, p.N, BM, BN, &m0, &n0);
    c_i32 += static_cast<size_t>(split) * p.M * p.ldc;
  } else {
    tile_origin(p.M, p.N, BM, BN, &m0, &n0);
  }
  const int splits = EPI == kEpiI32 ? max(p.splits, 1) : 1;
  const int nk_all = p.K / BK;
  const int kb0 = nk_all * split / splits;
  const int nk = nk_all * (split + 1) / splits - kb0;
  const int8_t* const pA = p.A + kb0 * BK;
  const int8_t* const pW = p.W + kb0 * BK;
  // The wave index is uniform across the wave; readfirstlane tells the
  // compiler so, keeping per-wave decisions (Q/K/V head, RoPE) scalar.
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int l32 = lane & 31, hi = lane >> 5;

  // Load blocks wave*kPer .. +kPer of each stage: blocks [0, BM/8) are A row
  // groups, the rest W row groups. Rows past the edge re-read the last valid
  // row (their products are never stored).
  // Source of block i: a wave-uniform base (A or W) plus a 32-bit lane
  // offset (operands are far below 4 GiB).
  uint32_t goff[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int b = wave * kPer + i;
    const int r = lane >> 3;
    const int c = (lane & 7) ^ r ^ (b & 1);
    const bool is_a = b < BM / 8;
    const int row = is_a ? min(m0 + b * 8 + r, p.M - 1) : min(n0 + (b - BM / 8) * 8 + r, p.N - 1);
    goff[i] = static_cast<uint32_t>(row) * static_cast<uint32_t>(is_a ? p.lda : p.ldw) + c * 16;
  }
  auto gbase = [&](int i) { return wave * kPer + i < BM / 8 ? pA : pW; };
  const uint32_t ldst = lds_addr(smem) + static_cast<uint32_t>(wave * kPer * 1024);
  // Stage 0 first, so that its loads and the scale loads below are in flight
  // together.
#pragma unroll
  for (int i = 0; i < kPer; ++i) dma16_async_so(gbase(i), goff[i], ldst + i * 1024);

  // kEpiF32R24: whether a value of the tile can be NaN (a scale or bias not
  // finite, or a scale above 2^60, so that a product of two could overflow).
  // Each wave's verdict goes to LDS here and is combined before the
  // epilogue.
  __shared__ int s_risk[TL::kWaves];
  if constexpr (EPI != kEpiI32) {
    // Per-row activation scales and per-column weight scales / bias of the
    // tile, read once here instead of per element in the epilogue, every
    // item's loads issued before the first LDS write. The epilogue (and the
    // RoPE staging) read them after the main loop's barriers, each of which
    // follows an lgkmcnt(0) wait, so no barrier of their own is needed.
    constexpr int kItems = (BM + BN + kThreads - 1) / kThreads;
    float va[kItems], vb[kItems];
    int vp[kItems];
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
      const int t = threadIdx.x + k * kThreads;
      va[k] = vb[k] = 0.0f;
      vp[k] = 0;
      if (t < BM) {
        const int row = m0 + t;
        if (row < p.M) {
          va[k] = p.a_scale[row];
          if constexpr (kRope) vp[k] = p.pos[row];
        }
      } else if (t < BM + BN) {
        const int col = n0 + t - BM;
        if (col < p.N) {
          va[k] = p.w_scale[col];
          if (p.bias) vb[k] = p.bias[col];
        }
      }
    }
    int risk = 0;
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
      const int t = threadIdx.x + k * kThreads;
      if (t < BM) {
        s_as[t] = va[k];
        if constexpr (EPI == kEpiF32R24) risk |= !(__builtin_fabsf(va[k]) <= 0x1p60f);
        if constexpr (kRope) s_pos[t] = vp[k];
      } else if (t < BM + BN) {
        const int c = t - BM;
        float w = va[k], b = vb[k];
        if constexpr (EPI == kEpiQkvSplit) {
          // Q columns: q_prescale (a power of two) folded in here, exactly.
          if (n0 + c < p.d_model) {
            w *= p.q_prescale;
            b *= p.q_prescale;
          }
        }
        s_ws[c] = w;
        s_bs[c] = b;
        if constexpr (EPI == kEpiF32R24) risk |= !(__builtin_fabsf(w) <= 0x1p60f) | !(__builtin_fabsf(b) <= 0x1p127f);
      }
    }
    if constexpr (EPI == kEpiF32R24) {
      const bool wave_risk = __builtin_amdgcn_ballot_w64(risk != 0) != 0;
      if (lane == 0) s_risk[wave] = wave_risk;
    }
  }

  // The accumulators start as the first products (the first sub-step's
  // MFMAs take a zero C operand), so no register is cleared beforehand.
  i32x16 acc[BLK_M][BLK_N];

  // Fragments are double-buffered in registers: the reads of K sub-step
  // q + 1 (32 bytes of K) are issued between the MFMAs of sub-step q, one
  // read after each MFMA, so the LDS latency runs under the matrix cores
  // instead of in front of them. Across a stage boundary the first sub-step
  // of the next stage is read during the last sub-step's MFMAs, after the
  // barrier that publishes that stage.
  // Row R + 32 i of a stage sits 4 KB after row R (same r = R & 7 and
  // parity of R >> 3), so one lane offset per 16-byte chunk addresses every
  // fragment of a sub-step, the block index becoming an immediate offset.
  const int arow = wm * BLK_M * 32 + l32;       // A fragment rows (+ i*32)
  const int brow = BM + wn * BLK_N * 32 + l32;  // W fragment rows (+ j*32)
  constexpr int kSub = BK / 32;                 // MFMA sub-steps per stage
  int aoff[kSub], boff[kSub];
#pragma unroll
  for (int q = 0; q < kSub; ++q) {
    aoff[q] = soff(arow, 2 * q + hi);
    boff[q] = soff(brow, 2 * q + hi);
  }
  auto read_frags = [&](const int8_t* buf, int q, i32x4(&fa)[BLK_M], i32x4(&fb)[BLK_N]) {
#pragma unroll
    for (int i = 0; i < BLK_M; ++i) fa[i] = *reinterpret_cast<const i32x4*>(buf + aoff[q] + i * 4096);
#pragma unroll
    for (int j = 0; j < BLK_N; ++j) fb[j] = *reinterpret_cast<const i32x4*>(buf + boff[q] + j * 4096);
  };
  auto mfmas = [&](const i32x4(&fa)[BLK_M], const i32x4(&fb)[BLK_N]) {
#pragma unroll
    for (int i = 0; i < BLK_M; ++i)
#pragma unroll
      for (int j = 0; j < BLK_N; ++j) acc[i][j] = mfma32(fa[i], fb[j], acc[i][j]);
  };
  auto mfmas_first = [&](const i32x4(&fa)[BLK_M], const i32x4(&fb)[BLK_N]) {
    const i32x16 zero = {};
#pragma unroll
    for (int i = 0; i < BLK_M; ++i)
#pragma unroll
      for (int j = 0; j < BLK_N; ++j) acc[i][j] = mfma32(fa[i], fb[j], zero);
  };
  // Order the reads issued during a sub-step's MFMAs: read, MFMA, read,
  // MFMA ... then the remaining MFMAs.
  // Short tiles (BLK_M 1) issue more reads than MFMAs per sub-step; the
  // reads left over go last.
  constexpr int kReads = BLK_M + BLK_N, kMfmas = BLK_M * BLK_N;
  constexpr int kPairs = kReads < kMfmas ? kReads : kMfmas;
  auto interleave = [&]() {
#pragma unroll
    for (int u = 0; u < kPairs; ++u) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    }
    if constexpr (kMfmas > kPairs) __builtin_amdgcn_sched_group_barrier(0x008, kMfmas - kPairs, 0);
    if constexpr (kReads > kPairs) __builtin_amdgcn_sched_group_barrier(0x100, kReads - kPairs, 0);
  };
  i32x4 fa0[BLK_M], fb0[BLK_N], fa1[BLK_M], fb1[BLK_N];
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  // Stages 1 .. kNStage - 1 go to the free buffers.
#pragma unroll
  for (int st = 1; st < kNStage; ++st) {
    if (st < nk) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) dma16_async_so(gbase(i) + st * BK, goff[i], ldst + st * kStage + i * 1024);
    }
  }
  read_frags(smem, 0, fa0, fb0);
  static_assert(kSub == 4, "the sub-step rotation below assumes four 32-byte sub-steps per stage");
  // Buffer of stage kt (kt mod kNStage), kept as a wave-uniform counter.
  // Stage 0 is the loop body with its first sub-step's MFMAs starting the
  // accumulators.
  int bcur = 0;
  auto stage = [&](int kt, auto first) {
    const int8_t* cur = smem + bcur * kStage;
    const int bnext = bcur + 1 == kNStage ? 0 : bcur + 1;
    read_frags(cur, 1, fa1, fb1);
    if constexpr (decltype(first)::value)
      mfmas_first(fa0, fb0);
    else
      mfmas(fa0, fb0);
    interleave();
    read_frags(cur, 2, fa0, fb0);
    mfmas(fa1, fb1);
    interleave();
    read_frags(cur, 3, fa1, fb1);
    mfmas(fa0, fb0);
    interleave();
    // Stage kt + 1 has landed (own loads, then the barrier for everyone
    // else's) and every wave has finished reading stage kt, whose buffer
    // then receives stage kt + kNStage. With three buffers stage kt + 2's
    // loads, issued one iteration earlier, may still be in flight: vector
    // memory operations complete in order, so waiting until at most those
    // kPer remain means stage kt + 1's have landed. The body has no other
    // branch: the last iteration reads sub-step 0 of a stale buffer into
    // fa0 / fb0 and never uses it (a branch around those reads would split
    // the last sub-step's MFMAs over two blocks, and the accumulators'
    // copies at the join spill).
    if (kNStage == 3 && kt + 2 < nk)
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kPer) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (kt + kNStage < nk) {
      const uint32_t dst = ldst + bcur * kStage;
#pragma unroll
      for (int i = 0; i < kPer; ++i) dma16_async_so(gbase(i) + (kt + kNStage) * BK, goff[i], dst + i * 1024);
    }
    read_frags(smem + bnext * kStage, 0, fa0, fb0);
    mfmas(fa1, fb1);
    interleave();
    bcur = bnext;
  };
  stage(0, std::true_type{});
  for (int kt = 1; kt < nk; ++kt) stage(kt, std::false_type{});

  const float* s_cosT = nullptr;
  const float* s_sinT = nullptr;
  if constexpr (kRope) {
    if (n0 < 2 * p.d_model) {
      // The tile holds Q or K columns: stage its rows' RoPE cos / sin,
      // transposed, in the now idle operand buffers. Item u copies half a
      // table row (cos for even u, sin for odd u) of tile row u / 2.
      static_assert(2 * 32 * kRopeTPitch * 4 <= kNStage * kStage, "RoPE staging fits in the operand buffers");
      float* cosT = reinterpret_cast<float*>(smem);
      float* sinT = cosT + 32 * kRopeTPitch;
      __syncthreads();
      // Each thread copies items threadIdx.x + k * kThreads; every item's
      // loads are issued before the first LDS write, so the table reads'
      // latency is paid once.
      constexpr int kItems = (2 * BM + kThreads - 1) / kThreads;
      float4 v[kItems][8];
#pragma unroll
      for (int k = 0; k < kItems; ++k) {
        const int u = threadIdx.x + k * kThreads;
        const int uc = u < 2 * BM ? u : 0;
        const float4* src = reinterpret_cast<const float4*>((uc & 1 ? p.rope_sin : p.rope_cos) +
                                                            static_cast<size_t>(s_pos[uc >> 1]) * 64);
#pragma unroll
        for (int c4 = 0; c4 < 8; ++c4) v[k][c4] = src[c4];
      }
#pragma unroll
      for (int k = 0; k < kItems; ++k) {
        const int u = threadIdx.x + k * kThreads;
        if (u < 2 * BM) {
          float* dst = (u & 1 ? sinT : cosT) + (u >> 1);
#pragma unroll
          for (int c4 = 0; c4 < 8; ++c4) {
            dst[(4 * c4 + 0) * kRopeTPitch] = v[k][c4].x;
            dst[(4 * c4 + 1) * kRopeTPitch] = v[k][c4].y;
            dst[(4 * c4 + 2) * kRopeTPitch] = v[k][c4].z;
            dst[(4 * c4 + 3) * kRopeTPitch] = v[k][c4].w;
          }
        }
      }
      __syncthreads();
      s_cosT = cosT;
      s_sinT = sinT;
    }
  }
  bool nan_risk = false;
  if constexpr (EPI == kEpiF32R24) {
    int any = 0;
#pragma unroll
    for (int w = 0; w < TL::kWaves; ++w) any |= s_risk[w];
    nan_risk = any != 0;
  }
  constexpr bool kMaxable =
      EPI == kEpiF32Gelu || EPI == kEpiF32GeluQ || EPI == kEpiF32GeluAs || EPI == kEpiF32GeluX86 || EPI == kEpiF32;
  const bool full = m0 + BM <= p.M && n0 + BN <= p.N;
  if (kMaxable && (p.row_absmax || p.tensor_absmax)) {
    if (full)
      epilogue32<BLK_M, BLK_N, EPI, true, kMaxable>(p, acc, wm, wn, l32, hi, s_as, s_ws, s_bs, s_cosT, s_sinT, m0, n0,
          c_i32, nan_risk);
    else
      epilogue32<BLK_M, BLK_N, EPI, false, kMaxable>(p, acc, wm, wn, l32, hi, s_as, s_ws, s_bs, s_cosT, s_sinT, m0, n0,
          c_i32, nan_risk);
  } else {
    if (full)
      epilogue32<BLK_M, BLK_N, EPI, true, false>(p, acc, wm, wn, l32, hi, s_as, s_ws, s_bs, s_cosT, s_sinT, m0, n0,
          c_i32, nan_risk);
    else
      epilogue32<BLK_M, BLK_N, EPI, false, false>(p, acc, wm, wn, l32, hi, s_as, s_ws, s_bs, s_cosT, s_sinT, m0, n0,
          c_i32, nan_risk);
  }
}

// Split-K dequant: C[m, n] = fma(float(sum over the S planes of P[m, n]),
// a_scale[m] * w_scale[n], bias[n]), the kEpiF32 epilogue's expression on the
// exact int32 sum. Four columns per thread (N and ldc multiples of 4).
// ACCUM: C[m, n] += that value instead (the kEpiF32Resid epilogue's C + v).
template <bool ACCUM>
__global__ __launch_bounds__(256) void splitk_dequant_kernel(const int32_t* __restrict__ P, int S, int M, int N,
                                                             const float* __restrict__ a_scale,
                                                             const float* __restrict__ w_scale,
                                                             const float* __restrict__ bias, float* __restrict__ C,
                                                             int ldc) {
  const int n4 = N / 4;
  const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<size_t>(M) * n4) return;
  const int m = static_cast<int>(i / n4), c = static_cast<int>(i % n4) * 4;
  const size_t plane = static_cast<size_t>(M) * N;
  const int32_t* src = P + static_cast<size_t>(m) * N + c;
  int4 acc = *reinterpret_cast<const int4*>(src);
  for (int k = 1; k < S; ++k) {
    const int4 v = *reinterpret_cast<const int4*>(src + k * plane);
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  const float as = a_scale[m];
  const float4 ws = *reinterpret_cast<const float4*>(w_scale + c);
  const float4 b = bias ? *reinterpret_cast<const float4*>(bias + c) : make_float4(0.f, 0.f, 0.f, 0.f);
  float4 out;
  out.x = __builtin_fmaf(static_cast<float>(acc.x), as * ws.x, b.x);
  out.y = __builtin_fmaf(static_cast<float>(acc.y), as * ws.y, b.y);
  out.z = __builtin_fmaf(static_cast<float>(acc.z), as * ws.z, b.z);
  out.w = __builtin_fmaf(static_cast<float>(acc.w), as * ws.w, b.w);
  if constexpr (ACCUM) {
    const float4 r = *reinterpret_cast<const float4*>(C + static_cast<size_t>(m) * ldc + c);
    out.x = r.x + out.x;
    out.y = r.y + out.y;
    out.z = r.z + out.z;
    out.w = r.w + out.w;
  }
  __builtin_nontemporal_store(out.x, C + static_cast<size_t>(m) * ldc + c);
  __builtin_nontemporal_store(out.y, C + static_cast<size_t>(m) * ldc + c + 1);
  __builtin_nontemporal_store(out.z, C + static_cast<size_t>(m) * ldc + c + 2);
  __builtin_nontemporal_store(out.w, C + static_cast<size_t>(m) * ldc + c + 3);
}

}  // namespace v3
}  // namespace

namespace {

hipError_t launch_v1(const GemmI8Args& p, int epi, hipStream_t s) {
  const int tiles = ((p.M + Cfg::BM - 1) / Cfg::BM) * ((p.N + Cfg::BN - 1) / Cfg::BN);
  const dim3 grid(tiles), block(Cfg::THREADS);
  switch (epi) {
    case kEpiI32: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiI32>), grid, block, 0, s, p); break;
    case kEpiF32: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiF32>), grid, block, 0, s, p); break;
    case kEpiF32Gelu: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiF32Gelu>), grid, block, 0, s, p); break;
    case kEpiF32Resid: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiF32Resid>), grid, block, 0, s, p); break;
    case kEpiQkvRope: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiQkvRope>), grid, block, 0, s, p); break;
    case kEpiF32GeluQ: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiF32GeluQ>), grid, block, 0, s, p); break;
    case kEpiF32GeluAs: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiF32GeluAs>), grid, block, 0, s, p); break;
    case kEpiF32GeluX86: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiF32GeluX86>), grid, block, 0, s, p); break;
    case kEpiQkvRopeF32: hipLaunchKernelGGL((gemm_i8_kernel<Cfg, kEpiQkvRopeF32>), grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int BLK_M, int BLK_N = 2>
hipError_t launch_v3_tile(const GemmI8Args& p, int epi, hipStream_t s) {
  using namespace v3;
  constexpr int BM = Tile<BLK_M, BLK_N>::BM;
  const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const dim3 grid(tiles * (epi == kEpiI32 ? std::max(p.splits, 1) : 1)), block(Tile<BLK_M, BLK_N>::kThreads);
  switch (epi) {
    case kEpiI32: hipLaunchKernelGGL((gemm_i8_v3_kernel<BLK_M, BLK_N, kEpiI32>), grid, block, 0, s, p); break;
    case kEpiF32: hipLaunchKernelGGL((gemm_i8_v3_kernel<BLK_M, BLK_N, kEpiF32>), grid, block, 0, s, p); break;
    case kEpiF32Gelu: hipLaunchKernelGGL((gemm_i8_v3_kernel<BLK_M, BLK_N, kEpiF32Gelu>), grid, block, 0, s, p); break;
    case kEpiF32Resid: hipLaunchKernelGGL((gemm_i8_v3_kernel<BLK_M, BLK_N, kEpiF32Resid>), grid, block, 0, s, p); break;
    case kEpiQkvRope: hipLaunchKernelGGL((gemm_i8_v3_kernel<BLK_M, BLK_N, kEpiQkvRope>), grid, block, 0, s, p); break;
    case kEpiF32GeluQ: hipLaunchKernelGGL((gemm_i8_v3_kernel<BLK_M, BLK_N, kEpiF32GeluQ>), grid, block, 0, s, p); break;
    case kEpiF32GeluAs:
      hipLaunchKernelGGL((gemm_i8_v3_kernel<BLK_M, BLK_N, kEpiF32GeluAs>), grid, block, 0, s, p);
      break;
    case kEpiF32GeluX86:
      hipLaunchKernelGGL((gemm_i8_v3_kernel<BLK_M, BLK_N, kEpiF32GeluX86>), grid, block, 0, s, p);
      break;
    case kEpiQkvRopeF32:
      hipLaunchKernelGGL((gemm_i8_v3_kernel<BLK_M, BLK_N, kEpiQkvRopeF32>), grid, block, 0, s, p);
      break;
    case kEpiQkvSplit: hipLaunchKernelGGL((gemm_i8_v3_kernel<BLK_M, BLK_N, kEpiQkvSplit>), grid, block, 0, s, p); break;
    case kEpiF32R24:
      if (p.N % 64 != 0 || !p.C_f16 || !p.C_u8 || p.ldc % 2 != 0) return hipErrorInvalidValue;
      hipLaunchKernelGGL((gemm_i8_v3_kernel<BLK_M, BLK_N, kEpiF32R24>), grid, block, 0, s, p);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

std::atomic<int> g_tile_rows{0};

}  // namespace

// CUs of the current device (queried once per device).
int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  cus[dev].store(n, std::memory_order_relaxed);
  return n;
}

namespace {

long tiles_of(int M, int N, int BM) {
  return static_cast<long>((M + BM - 1) / BM) * ((N + v3::BN - 1) / v3::BN);
}

// Workgroup rounds times tile height: the rows' worth of tile time the grid
// needs when every round costs one tile's time.
long tile_cost(int M, int N, int BM, int cus) { return (tiles_of(M, N, BM) + cus - 1) / cus * BM; }

}  // namespace

int gemm_i8_tile_rows(int M, int N, int K, int epi, int cus) {
  const int forced = g_tile_rows.load(std::memory_order_relaxed);
  if (forced != 0) return forced;
  const int all = device_cus();
  if (cus <= 0) cus = all;
  // Ties go to 320 rows: at equal rounds the taller tile re-reads less of
  // A and W (fc1 at config 4: 270 vs 282 us). The erff GELU and bf16/fp32
  // RoPE epilogues stay at 256 rows: at BLK_M = 5 they exceed 256 VGPRs. The
  // split-word QKV epilogue spills 72 bytes there too, but runs faster at
  // 320 rows all the same (216 vs 224 us at config 4). Rounds are counted
  // over the whole device: concurrent launches fill each other's last round.
  const bool tall_ok =
      epi == kEpiI32 || epi == kEpiF32 || epi == kEpiF32Resid || epi == kEpiQkvSplit || epi == kEpiF32R24 ||
      epi == kEpiF32GeluAs;
  if (tiles_of(M, N, 256) >= cus)
    return tall_ok && tile_cost(M, N, 320, all) <= tile_cost(M, N, 256, all) ? 320 : 256;
  // The 256-row grid leaves CUs idle (one workgroup per CU): shorter tiles
  // spread the rows over more CUs. Estimated time of a grid = rounds x
  // (stages + fixed cost) x the per-stage time of the tile height, the
  // per-stage times relative to the 256-row tile's.
  static constexpr int kRows[3] = {64, 128, 256};
  static constexpr double kStage[3] = {0.45, 0.62, 1.0};
  constexpr double kFixed = 3.0;  // prologue + epilogue, in stages
  const double stages = K / v3::BK + kFixed;
  int best = 256;
  double best_t = 0.0;
  for (int i = 2; i >= 0; --i) {
    const long rounds = (tiles_of(M, N, kRows[i]) + cus - 1) / cus;
    const double t = static_cast<double>(rounds) * stages * kStage[i];
    if (i == 2 || t < best_t * 0.97) {
      best = kRows[i];
      best_t = t;
    }
  }
  return best;
}

namespace {

std::atomic<int> g_split_k{0};

// Estimated time, in units of one 256-row tile's K stage (about 2 us here),
// of a grid of `tiles` workgroups on `cus` CUs running `stages` K stages each
// at tile height rows (64, 128 or 256), as in gemm_i8_tile_rows.
double grid_units(long tiles, int stages, int rows, int cus) {
  const double per = rows == 64 ? 0.45 : rows == 128 ? 0.62 : 1.0;
  const long rounds = (tiles + cus - 1) / cus;
  return static_cast<double>(rounds) * (stages + 3.0) * per;
}

}  // namespace

int gemm_i8_split_k(int M, int N, int K, int cus, bool fused, int* rows) {
  const int all = device_cus();
  if (cus <= 0) cus = all;
  *rows = gemm_i8_tile_rows(M, N, K, kEpiF32, cus);
  const int forced = g_split_k.load(std::memory_order_relaxed);
  if (forced == 1 || N % 4 != 0) return 1;
  const int nk = K / v3::BK;
  if (forced >= 2) return nk >= forced ? forced : 1;
  if (*rows == 320 || tiles_of(M, N, *rows) >= cus) return 1;
  // The dequant pass reads S int32 planes and writes the fp32 result: at
  // about 4 TB/s plus a launch, in the same units. Fused into the reader, it
  // costs the S - 1 planes read beyond the fp32 result it replaces.
  constexpr double kUnitUs = 2.05;
  auto pass_units = [&](int S) {
    if (fused) return (S - 1.0) * static_cast<double>(M) * N * 4.0 / 4.0e6 / kUnitUs;
    const double bytes = (S + 1.0) * static_cast<double>(M) * N * 4.0;
    return (bytes / 4.0e6 + 4.0) / kUnitUs;
  };
  double best = grid_units(tiles_of(M, N, *rows), nk, *rows, cus);
  int best_s = 1, best_rows = *rows;
  static constexpr int kRows[3] = {64, 128, 256};
  for (int r : kRows)
    for (int S = 2; S <= 4 && nk / S >= 4; ++S) {
      const double t = grid_units(tiles_of(M, N, r) * S, (nk + S - 1) / S, r, cus) + pass_units(S);
      if (t < best * 0.9) {
        best = t;
        best_s = S;
        best_rows = r;
      }
    }
  *rows = best_rows;
  return best_s;
}

bool set_gemm_split_k(int splits) {
  if (splits < 0 || splits > 4) return false;
  g_split_k.store(splits, std::memory_order_relaxed);
  return true;
}

namespace {

hipError_t launch_v3_rows(const GemmI8Args& p, int epi, int rows, hipStream_t s) {
  switch (rows) {
    case 64: return launch_v3_tile<1>(p, epi, s);
    case 128: return launch_v3_tile<2>(p, epi, s);
    case 320: return launch_v3_tile<5>(p, epi, s);
    default: return launch_v3_tile<4>(p, epi, s);
  }
}

hipError_t launch_v3(const GemmI8Args& p, int epi, hipStream_t s) {
  const bool accum = epi == kEpiF32Resid;
  if ((epi == kEpiF32 || accum) && p.splitk_ws && !p.row_absmax && !p.tensor_absmax && p.ldc % 4 == 0) {
    int rows = 0;
    const int S = gemm_i8_split_k(p.M, p.N, p.K, p.cus, false, &rows);
    if (S > 1 && static_cast<size_t>(S) * p.M * p.N <= p.splitk_ws_elems) {
      GemmI8Args q = p;
      q.C_i32 = p.splitk_ws;
      q.ldc = p.N;
      q.splits = S;
      const hipError_t e = launch_v3_rows(q, kEpiI32, rows, s);
      if (e != hipSuccess) return e;
      const size_t quads = static_cast<size_t>(p.M) * (p.N / 4);
      const dim3 grid(static_cast<unsigned>((quads + 255) / 256)), block(256);
      if (accum)
        hipLaunchKernelGGL(v3::splitk_dequant_kernel<true>, grid, block, 0, s, p.splitk_ws, S, p.M, p.N, p.a_scale,
                           p.w_scale, p.bias, p.C_f32, p.ldc);
      else
        hipLaunchKernelGGL(v3::splitk_dequant_kernel<false>, grid, block, 0, s, p.splitk_ws, S, p.M, p.N, p.a_scale,
                           p.w_scale, p.bias, p.C_f32, p.ldc);
      return hipGetLastError();
    }
  }
  return launch_v3_rows(p, epi, gemm_i8_tile_rows(p.M, p.N, p.K, epi, p.cus), s);
}

}  // namespace

bool gemm_i8_pipelined_ok(const GemmI8Args& p) {
  // The stage loads address A and W with 32-bit lane offsets.
  constexpr uint64_t kOffsetLimit = 1ull << 32;
  return p.K > 0 && p.K % v3::BK == 0 && p.lda % 16 == 0 && p.ldw % 16 == 0 && p.lda >= p.K && p.ldw >= p.K &&
         reinterpret_cast<uintptr_t>(p.A) % 16 == 0 && reinterpret_cast<uintptr_t>(p.W) % 16 == 0 &&
         static_cast<uint64_t>(p.M) * static_cast<uint64_t>(p.lda) <= kOffsetLimit &&
         static_cast<uint64_t>(p.N) * static_cast<uint64_t>(p.ldw) <= kOffsetLimit;
}

hipError_t launch_gemm_i8_variant(const GemmI8Args& p, int epi, int variant, hipStream_t s) {
  if (p.M <= 0 || p.N <= 0) return hipSuccess;
  // The split epilogue folds q_prescale into the staged Q scales, which is
  // exact only for a power of two.
  int e = 0;
  if (epi == kEpiQkvSplit && std::frexp(p.q_prescale, &e) != 0.5f) return hipErrorInvalidValue;
  if (variant == 2) {
    if (!gemm_i8_pipelined_ok(p)) return hipErrorInvalidValue;
    return launch_v3(p, epi, s);
  }
  return launch_v1(p, epi, s);
}

hipError_t launch_gemm_i8(const GemmI8Args& p, int epi, hipStream_t s) {
  return launch_gemm_i8_variant(p, epi, gemm_i8_pipelined_ok(p) ? 2 : 1, s);
}

hipError_t launch_gemm_i8_partials(const GemmI8Args& p, int splits, int rows, hipStream_t s) {
  if (p.M <= 0 || p.N <= 0) return hipSuccess;
  if (!gemm_i8_pipelined_ok(p) || splits < 1 || splits > p.K / v3::BK || !p.C_i32) return hipErrorInvalidValue;
  GemmI8Args q = p;
  q.splits = splits;
  return launch_v3_rows(q, kEpiI32, rows, s);
}

bool set_gemm_tile_rows(int rows) {
  if (rows != 0 && rows != 64 && rows != 128 && rows != 256 && rows != 320) return false;
  g_tile_rows.store(rows, std::memory_order_relaxed);
  return true;
}

}  // namespace esm_gfx950
