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

}  // namespace

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
