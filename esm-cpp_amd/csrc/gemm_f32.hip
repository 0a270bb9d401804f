// FP32 GEMM C = A W^T + bias on gfx950 fp32 MFMA (v_mfma_f32_16x16x4f32),
// with optional GELU or residual-add epilogue.
//
// Replaces esm::kernels::Linear (reference src/kernels/gemm_fp32.cpp:33-46
// LinearRef, :272-294 LinearAvx512) for the all-fp32 8M model and for the
// fp32 lm head (dense d->d, tied decoder d->vocab; src/model.cpp:1192-1239).
// Products are exact fp32 products accumulated in fp32, so results differ
// from the sequential reference sum only by summation order.
//
// Tiling: 128x128 workgroup tile, four waves of 64x64, 32-wide K stages in
// LDS (row pitch 36 floats). Within a stage, lane group g (lane / 16) owns
// the eight consecutive k values [8g, 8g+8): MFMA step j multiplies A and W
// at k = 8g + j for every lane group, which keeps A and W consistent and
// lets each lane fetch its k values with two 16-byte LDS reads.
#include "common.hpp"
#include "kernels.hpp"

namespace esm_gfx950 {
namespace {

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int kPitch = BK + 4;  // floats
constexpr int kThreads = 256;
constexpr int kStage = (BM + BN) * kPitch;

template <bool VEC>
__device__ __forceinline__ void load_stage(const float* __restrict__ base, int ld, int rows,
                                           int row0, int k0, int K, float4 (&r)[4]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = t + kThreads * i;
    const int row = idx >> 3;
    const int c = (idx & 7) * 4;
    int gr = row0 + row;
    gr = gr < rows ? gr : rows - 1;
    const int kk = k0 + c;
    const float* src = base + static_cast<size_t>(gr) * ld + kk;
    if constexpr (VEC) {
      r[i] = kk < K ? *reinterpret_cast<const float4*>(src) : make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
      r[i].x = kk + 0 < K ? src[0] : 0.f;
      r[i].y = kk + 1 < K ? src[1] : 0.f;
      r[i].z = kk + 2 < K ? src[2] : 0.f;
      r[i].w = kk + 3 < K ? src[3] : 0.f;
    }
  }
}

__device__ __forceinline__ void store_stage(float* s, const float4 (&r)[4]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = t + kThreads * i;
    *reinterpret_cast<float4*>(s + (idx >> 3) * kPitch + (idx & 7) * 4) = r[i];
  }
}

template <int EPI, bool VEC>
__global__ __launch_bounds__(kThreads, 2) void gemm_f32_kernel(const GemmF32Args p) {
  __shared__ __attribute__((aligned(16))) float smem[2 * kStage];
  const int tiles_n = (p.N + BN - 1) / BN;
  const int m0 = (blockIdx.x / tiles_n) * BM;
  const int n0 = (blockIdx.x % tiles_n) * BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 15, lg = lane >> 4;

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  float4 ra[4], rb[4];
  const int nk = (p.K + BK - 1) / BK;
  load_stage<VEC>(p.A, p.lda, p.M, m0, 0, p.K, ra);
  load_stage<VEC>(p.W, p.ldw, p.N, n0, 0, p.K, rb);
  store_stage(smem, ra);
  store_stage(smem + BM * kPitch, rb);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const float* cur = smem + (kt & 1) * kStage;
    const bool more = kt + 1 < nk;
    if (more) {
      load_stage<VEC>(p.A, p.lda, p.M, m0, (kt + 1) * BK, p.K, ra);
      load_stage<VEC>(p.W, p.ldw, p.N, n0, (kt + 1) * BK, p.K, rb);
    }
    float fa[4][8], fb[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float* pa = cur + (wm * 64 + i * 16 + lr) * kPitch + lg * 8;
      const float* pb = cur + BM * kPitch + (wn * 64 + i * 16 + lr) * kPitch + lg * 8;
      const float4 a0 = *reinterpret_cast<const float4*>(pa);
      const float4 a1 = *reinterpret_cast<const float4*>(pa + 4);
      const float4 b0 = *reinterpret_cast<const float4*>(pb);
      const float4 b1 = *reinterpret_cast<const float4*>(pb + 4);
      fa[i][0] = a0.x; fa[i][1] = a0.y; fa[i][2] = a0.z; fa[i][3] = a0.w;
      fa[i][4] = a1.x; fa[i][5] = a1.y; fa[i][6] = a1.z; fa[i][7] = a1.w;
      fb[i][0] = b0.x; fb[i][1] = b0.y; fb[i][2] = b0.z; fb[i][3] = b0.w;
      fb[i][4] = b1.x; fb[i][5] = b1.y; fb[i][6] = b1.z; fb[i][7] = b1.w;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 4; ++n)
          acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i][j], fb[n][j], acc[i][n], 0, 0, 0);
    if (more) {
      float* nxt = smem + ((kt + 1) & 1) * kStage;
      store_stage(nxt, ra);
      store_stage(nxt + BM * kPitch, rb);
    }
    __syncthreads();
  }

  const int rb0 = m0 + wm * 64, cb0 = n0 + wn * 64;
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int col = cb0 + n * 16 + lr;
    if (col >= p.N) continue;
    const float b = p.bias ? p.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = rb0 + i * 16 + lg * 4 + r;
        if (row >= p.M) continue;
        float v = acc[i][n][r] + b;
        float* dst = p.C + static_cast<size_t>(row) * p.ldc + col;
        if constexpr (EPI == kF32Gelu) v = gelu_erf(v);
        if constexpr (EPI == kF32Resid) {
          *dst += v;
        } else {
          *dst = v;
        }
      }
  }
}

// ---- Split-fp16 GEMM (fp32 accuracy on fp16 MFMA), same 128x128 tile and
// wave layout as above on v_mfma_f32_16x16x32_f16: each lane holds eight
// consecutive k of one row for A and W, so one MFMA covers a 32-wide K stage.
// A (fp32) is split into hi / lo fp16 planes while it is staged in LDS; W's
// planes come split. LDS rows are 64 bytes (four 16-byte chunks), chunk c of
// row r stored at position c ^ ((r / 4) mod 4): the 16-byte fragment reads
// of 16 rows at one chunk then cover all 64 banks once, and so do the stage
// writes of four consecutive rows (an 80-byte padded pitch kept the reads
// conflict-free but made every write pass conflict).
constexpr int kX3Pitch = 64;                    // bytes per 32-half row
constexpr int kX3Plane = 128 * kX3Pitch;        // one 128-row plane
constexpr int kX3Stage = 4 * kX3Plane;          // A hi, A lo, W hi, W lo

// Byte offset of 16-byte chunk c of row r in a plane.
__device__ __forceinline__ int x3_off(int r, int c) { return r * kX3Pitch + ((c ^ ((r >> 2) & 3)) << 4); }

__device__ __forceinline__ uint2 pack_f16x4(float a, float b, float c, float d) {
  return make_uint2(static_cast<uint32_t>(f32_to_f16_bits(a)) | (static_cast<uint32_t>(f32_to_f16_bits(b)) << 16),
                    static_cast<uint32_t>(f32_to_f16_bits(c)) | (static_cast<uint32_t>(f32_to_f16_bits(d)) << 16));
}

// One K stage of the tile from global memory: A 128 rows x 32 floats (four
// float4 per thread), W planes 128 rows x 32 halves each (two 16-byte pieces
// per plane per thread). Rows past the edge re-read the last valid row;
// their results are never stored.
__device__ __forceinline__ void x3_load(const GemmX3Args& p, int m0, int n0, int k0, f32x4 (&ra)[4],
                                        i32x4 (&rh)[2], i32x4 (&rl)[2]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = t + kThreads * i;
    const int row = min(m0 + (idx >> 3), p.M - 1);
    ra[i] = *reinterpret_cast<const f32x4*>(p.A + static_cast<size_t>(row) * p.lda + k0 + (idx & 7) * 4);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = t + kThreads * i;
    const int row = min(n0 + (idx >> 2), p.N - 1);
    const size_t off = static_cast<size_t>(row) * p.ldw + k0 + (idx & 3) * 8;
    rh[i] = *reinterpret_cast<const i32x4*>(p.w_hi + off);
    rl[i] = *reinterpret_cast<const i32x4*>(p.w_lo + off);
  }
}

// The stage into LDS: A split into hi / lo planes, W planes as loaded.
__device__ __forceinline__ void x3_store(uint8_t* st, const f32x4 (&ra)[4], const i32x4 (&rh)[2],
                                         const i32x4 (&rl)[2]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = t + kThreads * i;
    const int off = x3_off(idx >> 3, (idx & 7) >> 1) + (idx & 1) * 8;
    const f32x4 x = ra[i];
    const float hx = f16_bits_to_f32(f32_to_f16_bits(x[0])), hy = f16_bits_to_f32(f32_to_f16_bits(x[1]));
    const float hz = f16_bits_to_f32(f32_to_f16_bits(x[2])), hw = f16_bits_to_f32(f32_to_f16_bits(x[3]));
    *reinterpret_cast<uint2*>(st + off) = pack_f16x4(hx, hy, hz, hw);
    *reinterpret_cast<uint2*>(st + kX3Plane + off) = pack_f16x4(x[0] - hx, x[1] - hy, x[2] - hz, x[3] - hw);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = t + kThreads * i;
    const int off = x3_off(idx >> 2, idx & 3);
    *reinterpret_cast<i32x4*>(st + 2 * kX3Plane + off) = rh[i];
    *reinterpret_cast<i32x4*>(st + 3 * kX3Plane + off) = rl[i];
  }
}

template <int EPI>
__global__ __launch_bounds__(kThreads, 2) void gemm_x3_kernel(const GemmX3Args p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kX3Stage];
  const int tiles_n = (p.N + BN - 1) / BN;
  const int m0 = (blockIdx.x / tiles_n) * BM;
  const int n0 = (blockIdx.x % tiles_n) * BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 15, lg = lane >> 4;

  f32x4 ra[4];
  i32x4 rh[2], rl[2];
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = p.K / 32;
  x3_load(p, m0, n0, 0, ra, rh, rl);
  x3_store(smem, ra, rh, rl);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const uint8_t* cur = smem + (kt & 1) * kX3Stage;
    const bool more = kt + 1 < nk;
    if (more) x3_load(p, m0, n0, (kt + 1) * 32, ra, rh, rl);
    f16x8 ah[4], al[4], bh[4], bl[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ao = x3_off(wm * 64 + i * 16 + lr, lg);
      const int bo = x3_off(wn * 64 + i * 16 + lr, lg);
      ah[i] = *reinterpret_cast<const f16x8*>(cur + ao);
      al[i] = *reinterpret_cast<const f16x8*>(cur + kX3Plane + ao);
      bh[i] = *reinterpret_cast<const f16x8*>(cur + 2 * kX3Plane + bo);
      bl[i] = *reinterpret_cast<const f16x8*>(cur + 3 * kX3Plane + bo);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bh[n], acc[i][n], 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bh[n], c, 0, 0, 0);
        acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bl[n], c, 0, 0, 0);
      }
    if (more) x3_store(smem + ((kt + 1) & 1) * kX3Stage, ra, rh, rl);
    __syncthreads();
  }

  const int rb0 = m0 + wm * 64, cb0 = n0 + wn * 64;
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int col = cb0 + n * 16 + lr;
    if (col >= p.N) continue;
    const float b = p.bias ? p.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = rb0 + i * 16 + lg * 4 + r;
        if (row >= p.M) continue;
        float v = __builtin_fmaf(acc[i][n][r], p.w_unscale, b);
        if constexpr (EPI == kF32Gelu) v = gelu_erf(v);
        float* dst = p.C + static_cast<size_t>(row) * p.ldc + col;
        if constexpr (EPI == kF32Resid) {
          *dst += v;
        } else {
          *dst = v;
        }
      }
  }
}

// ---- Narrow fp32 GEMM, N <= 48 (the tied decoder, d -> 33 logits): one wave
// per 16 rows covers all 48 (padded) columns with v_mfma_f32_16x16x4f32.
// Lane (r, g) = (lane % 16, lane / 16) loads a float4 of row r of A at
// k = k0 + 4g and of rows r, r + 16, r + 32 of W; MFMA step j then multiplies
// A[r][k0 + 4g + j] with W[c][k0 + 4g + j] for every lane group g, which sums
// all 16 k of the stage over the four steps. W (N x K, 169 KB for the ESM
// decoder) is re-read from L2 by every wave. K % 16 == 0.
__global__ __launch_bounds__(256) void gemm_narrow_kernel(const GemmF32Args p) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 16;
  if (row0 >= p.M) return;
  const int r = lane & 15, g = lane >> 4;
  const float* arow = p.A + static_cast<size_t>(min(row0 + r, p.M - 1)) * p.lda + 4 * g;
  const float* wrow[3];
  bool wok[3];
#pragma unroll
  for (int nb = 0; nb < 3; ++nb) {
    const int c = nb * 16 + r;
    wok[nb] = c < p.N;
    wrow[nb] = p.W + static_cast<size_t>(min(c, p.N - 1)) * p.ldw + 4 * g;
  }
  f32x4 acc[3];
#pragma unroll
  for (int nb = 0; nb < 3; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 a = *reinterpret_cast<const f32x4*>(arow);
  f32x4 b[3];
#pragma unroll
  for (int nb = 0; nb < 3; ++nb) b[nb] = *reinterpret_cast<const f32x4*>(wrow[nb]);
  for (int k0 = 0; k0 < p.K; k0 += 16) {
    f32x4 an = a, bn[3] = {b[0], b[1], b[2]};
    if (k0 + 16 < p.K) {
      an = *reinterpret_cast<const f32x4*>(arow + k0 + 16);
#pragma unroll
      for (int nb = 0; nb < 3; ++nb) bn[nb] = *reinterpret_cast<const f32x4*>(wrow[nb] + k0 + 16);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int nb = 0; nb < 3; ++nb)
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], wok[nb] ? b[nb][j] : 0.0f, acc[nb], 0, 0, 0);
    a = an;
#pragma unroll
    for (int nb = 0; nb < 3; ++nb) b[nb] = bn[nb];
  }
  // Output element i of block nb in lane (r, g): row row0 + 4g + i, column nb*16 + r.
#pragma unroll
  for (int nb = 0; nb < 3; ++nb) {
    const int col = nb * 16 + r;
    if (col >= p.N) continue;
    const float bias = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = row0 + 4 * g + i;
      if (row < p.M) p.C[static_cast<size_t>(row) * p.ldc + col] = acc[nb][i] + bias;
    }
  }
}

}  // namespace

hipError_t launch_gemm_narrow(const GemmF32Args& p, hipStream_t s) {
  if (p.M <= 0 || p.N <= 0) return hipSuccess;
  if (p.N > 48 || p.K <= 0 || p.K % 16 != 0 || p.lda % 4 != 0 || p.ldw % 4 != 0) return hipErrorInvalidValue;
  const int waves = (p.M + 15) / 16;
  hipLaunchKernelGGL(gemm_narrow_kernel, dim3((waves + 3) / 4), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_gemm_x3(const GemmX3Args& p, int epi, hipStream_t s) {
  if (p.M <= 0 || p.N <= 0) return hipSuccess;
  if (p.K <= 0 || p.K % 32 != 0 || p.lda % 4 != 0 || p.ldw % 8 != 0) return hipErrorInvalidValue;
  const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const dim3 grid(tiles), block(kThreads);
  switch (epi) {
    case kF32Store: hipLaunchKernelGGL((gemm_x3_kernel<kF32Store>), grid, block, 0, s, p); break;
    case kF32Gelu: hipLaunchKernelGGL((gemm_x3_kernel<kF32Gelu>), grid, block, 0, s, p); break;
    case kF32Resid: hipLaunchKernelGGL((gemm_x3_kernel<kF32Resid>), grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gemm_f32(const GemmF32Args& p, int epi, hipStream_t s) {
  if (p.M <= 0 || p.N <= 0) return hipSuccess;
  const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const dim3 grid(tiles), block(kThreads);
  const bool vec = (p.K % 4 == 0) && (p.lda % 4 == 0) && (p.ldw % 4 == 0);
#define ESM_F32_LAUNCH(E)                                                          \
  if (vec) hipLaunchKernelGGL((gemm_f32_kernel<E, true>), grid, block, 0, s, p);   \
  else hipLaunchKernelGGL((gemm_f32_kernel<E, false>), grid, block, 0, s, p);
  switch (epi) {
    case kF32Store: ESM_F32_LAUNCH(kF32Store) break;
    case kF32Gelu: ESM_F32_LAUNCH(kF32Gelu) break;
    case kF32Resid: ESM_F32_LAUNCH(kF32Resid) break;
    default: return hipErrorInvalidValue;
  }
#undef ESM_F32_LAUNCH
  return hipGetLastError();
}

}  // namespace esm_gfx950
