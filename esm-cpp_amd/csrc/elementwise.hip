// HBM-bound row and elementwise kernels of the packed ESM-2 encoder path:
// LayerNorm (optionally fused with per-token int8 quantisation), activation
// quantisation (per token or per tensor), absmax, GELU, residual add, Q
// scale, rotary embedding, token embedding and dtype casts.
//
// Reference counterparts: LayerNormRef src/kernels/layernorm.cpp:23-44,
// activation quant src/kernels/gemm_int8.cpp:391-508 and
// src/quant/pack.cpp:119-147, GeluRef src/kernels/gelu.cpp:30-35,
// ResidualAddInplaceRef / ScaleInplaceRef src/kernels/residual.cpp:23-29,
// RopeApplyVarlenRef src/kernels/rope.cpp:47-70, Embed src/model.cpp:737-778.
#include "common.hpp"
#include "kernels.hpp"

namespace esm_gfx950 {
namespace {

constexpr int kRowsPerBlock = 4;  // one wave per row, 4 waves per block

// Each value rounded to the nearest fp16 (ties to even) and widened back:
// the reference's first-block fc1 escape (RoundToFp16Inplace, src/model.cpp:
// 912-930, VCVTPS2PH round-to-nearest).
__device__ __forceinline__ float4 round_f16(float4 y) {
  y.x = static_cast<float>(static_cast<_Float16>(y.x));
  y.y = static_cast<float>(static_cast<_Float16>(y.y));
  y.z = static_cast<float>(static_cast<_Float16>(y.z));
  y.w = static_cast<float>(static_cast<_Float16>(y.w));
  return y;
}

// Lane's NV float4 chunks of a row (chunk j at column (j*64 + lane)*4). Every
// load is issued before any value is used: a chunk past `cols` re-reads
// column 0 (in bounds) and is then zeroed, so no load sits in a branch that
// would make the wave wait for it before issuing the next.
// load_row_raw issues the loads alone and mask_row zeroes the chunks past
// `cols` once they are used, so a caller can keep a row's loads in flight.
template <int NV>
__device__ __forceinline__ void load_row_raw(const float* __restrict__ xr, int cols, int lane, float4 (&v)[NV]) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    v[j] = *reinterpret_cast<const float4*>(xr + (c < cols ? c : 0));
  }
}

template <int NV>
__device__ __forceinline__ void mask_row(int cols, int lane, float4 (&v)[NV]) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const bool ok = (j * 64 + lane) * 4 < cols;
    v[j].x = ok ? v[j].x : 0.0f;
    v[j].y = ok ? v[j].y : 0.0f;
    v[j].z = ok ? v[j].z : 0.0f;
    v[j].w = ok ? v[j].w : 0.0f;
  }
}

template <int NV>
__device__ __forceinline__ void load_row_vec(const float* __restrict__ xr, int cols, int lane, float4 (&v)[NV]) {
  load_row_raw<NV>(xr, cols, lane, v);
  mask_row<NV>(cols, lane, v);
}

// ---- LayerNorm with the row cached in registers (d % 4 == 0, d <= NV*256).
// The LayerNorm of the row in v (residual already added), in place; returns
// the row's largest |output|.
template <int NV>
__device__ __forceinline__ float ln_core(const float* __restrict__ gamma, const float* __restrict__ beta, float eps,
                                         int d, int lane, int round16, float4 (&v)[NV]) {
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) sum += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  const float mean = wave_sum(sum) / static_cast<float>(d);
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    const float a = v[j].x - mean, b = v[j].y - mean, e = v[j].z - mean, f = v[j].w - mean;
    const float t = (a * a + b * b) + (e * e + f * f);
    sq += c < d ? t : 0.0f;
  }
  const float var = wave_sum(sq) / static_cast<float>(d);
  const float inv_std = 1.0f / sqrtf(var + eps);
  float4 g[NV], bt[NV];
  load_row_vec<NV>(gamma, d, lane, g);
  load_row_vec<NV>(beta, d, lane, bt);
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    float4 y;
    y.x = (v[j].x - mean) * inv_std * g[j].x + bt[j].x;
    y.y = (v[j].y - mean) * inv_std * g[j].y + bt[j].y;
    y.z = (v[j].z - mean) * inv_std * g[j].z + bt[j].z;
    y.w = (v[j].w - mean) * inv_std * g[j].w + bt[j].w;
    if (round16) y = round_f16(y);
    v[j] = y;
    if (c < d) amax = fmaxf(amax, fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))));
  }
  return amax;
}

// One wave's row: the residual update, the LayerNorm into v, and the row's
// absolute maximum (returned). With resid != null the row is first updated
// in place, x += resid (the residual add that precedes the next LayerNorm,
// reference src/model.cpp:1013 and :1063), and the LayerNorm runs on the
// sum; SPLIT: the residual arrives as split-K partial sums (SplitResid). The
// kernels below share ln_core, so every pass over a row computes the same
// values.
template <int NV, bool SPLIT>
__device__ __forceinline__ float ln_row(float* __restrict__ x, const float* __restrict__ resid,
                                        const float* __restrict__ gamma, const float* __restrict__ beta, float eps,
                                        int row, int rows, int d, int lane, int round16, const SplitResid& split,
                                        float4 (&v)[NV]) {
  float* xr = x + static_cast<size_t>(row) * d;
  load_row_vec<NV>(xr, d, lane, v);
  if (SPLIT || resid) {
    float4 r[NV];
    if constexpr (SPLIT) {
      // The residual's GEMM epilogue on its summed split-K partial sums:
      // fma(float(acc), a_scale * w_scale, bias), the same expression and
      // operands. The row's a_scale is read here, before `scales` (which it
      // may be) receives this row's new scale.
      const float as = split.a_scale[row];
      const size_t plane = static_cast<size_t>(rows) * d;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int c = (j * 64 + lane) * 4;
        const int cc = c < d ? c : 0;
        const int32_t* src = split.planes + static_cast<size_t>(row) * d + cc;
        int4 acc = *reinterpret_cast<const int4*>(src);
        for (int k = 1; k < split.splits; ++k) {
          const int4 t = *reinterpret_cast<const int4*>(src + k * plane);
          acc.x += t.x;
          acc.y += t.y;
          acc.z += t.z;
          acc.w += t.w;
        }
        const float4 ws = *reinterpret_cast<const float4*>(split.w_scale + cc);
        const float4 bs = split.bias ? *reinterpret_cast<const float4*>(split.bias + cc) : make_float4(0.f, 0.f, 0.f, 0.f);
        r[j].x = c < d ? __builtin_fmaf(static_cast<float>(acc.x), as * ws.x, bs.x) : 0.0f;
        r[j].y = c < d ? __builtin_fmaf(static_cast<float>(acc.y), as * ws.y, bs.y) : 0.0f;
        r[j].z = c < d ? __builtin_fmaf(static_cast<float>(acc.z), as * ws.z, bs.z) : 0.0f;
        r[j].w = c < d ? __builtin_fmaf(static_cast<float>(acc.w), as * ws.w, bs.w) : 0.0f;
      }
    } else {
      load_row_vec<NV>(resid + static_cast<size_t>(row) * d, d, lane, r);
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      v[j].x += r[j].x;
      v[j].y += r[j].y;
      v[j].z += r[j].z;
      v[j].w += r[j].w;
      const int c = (j * 64 + lane) * 4;
      if (c < d) *reinterpret_cast<float4*>(xr + c) = v[j];
    }
  }
  return ln_core<NV>(gamma, beta, eps, d, lane, round16, v);
}


// !QUANT: the LayerNorm stored to out (if not null). With a per-tensor
// absmax the grid is bounded and walks the rows (one atomic per block: the
// atomics on the one address serialise in L2), every wave reaching the
// block's reduction.
// QUANT: int8 codes and the row's scale; the scale from the row's own
// maximum (per-token), or with tensor_absmax from that device value, each
// code then quant_i8 as the per-tensor quantisation kernel forms it.
template <int NV, bool QUANT, bool SPLIT = false>
__global__ __launch_bounds__(256) void layernorm_vec_kernel(
    float* __restrict__ x, const float* __restrict__ resid, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, float* __restrict__ out,
    int rows, int d, float* tensor_absmax, int8_t* __restrict__ q, int ldq,
    float* scales, int round16, SplitResid split = SplitResid()) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float4 v[NV];
  if (!QUANT && tensor_absmax && !SPLIT && !resid && !out) {
    // The maximum alone: the wave's next row is loaded while this one is
    // reduced, so each wave keeps a row's loads in flight.
    float am = 0.f;
    const int step = gridDim.x * kRowsPerBlock;
    int row = blockIdx.x * kRowsPerBlock + wave;
    float4 nv[NV];
    if (row < rows) load_row_raw<NV>(x + static_cast<size_t>(row) * d, d, lane, nv);
    for (; row < rows; row += step) {
#pragma unroll
      for (int j = 0; j < NV; ++j) v[j] = nv[j];
      mask_row<NV>(d, lane, v);
      if (row + step < rows) load_row_raw<NV>(x + static_cast<size_t>(row + step) * d, d, lane, nv);
      am = fmaxf(am, ln_core<NV>(gamma, beta, eps, d, lane, round16, v));
    }
    block_atomic_max_nonneg(tensor_absmax, am);
    return;
  }
  if (!QUANT && tensor_absmax) {
    float am = 0.f;
    for (int base = blockIdx.x * kRowsPerBlock; base < rows; base += gridDim.x * kRowsPerBlock) {
      const int row = base + wave;
      if (row < rows) {
        am = fmaxf(am, ln_row<NV, SPLIT>(x, resid, gamma, beta, eps, row, rows, d, lane, round16, split, v));
        if (out) {
#pragma unroll
          for (int j = 0; j < NV; ++j) {
            const int c = (j * 64 + lane) * 4;
            if (c < d) *reinterpret_cast<float4*>(out + static_cast<size_t>(row) * d + c) = v[j];
          }
        }
      }
    }
    block_atomic_max_nonneg(tensor_absmax, am);
    return;
  }
  const int row = blockIdx.x * kRowsPerBlock + wave;
  if (row >= rows) return;
  const float amax = ln_row<NV, SPLIT>(x, resid, gamma, beta, eps, row, rows, d, lane, round16, split, v);
  if constexpr (QUANT) {
    int8_t* qr = q + static_cast<size_t>(row) * ldq;
    if (tensor_absmax) {
      const float scale = act_scale_from_absmax(*tensor_absmax);
      const float inv = 1.0f / scale;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int c = (j * 64 + lane) * 4;
        if (c < d)
          *reinterpret_cast<uint32_t*>(qr + c) = (static_cast<uint32_t>(quant_i8(v[j].x, inv)) & 0xffu) |
                                                 ((static_cast<uint32_t>(quant_i8(v[j].y, inv)) & 0xffu) << 8) |
                                                 ((static_cast<uint32_t>(quant_i8(v[j].z, inv)) & 0xffu) << 16) |
                                                 (static_cast<uint32_t>(quant_i8(v[j].w, inv)) << 24);
      }
      for (int c = d + lane; c < ldq; c += 64) qr[c] = 0;
      if (lane == 0) scales[row] = scale;
    } else {
      const float scale = act_scale_from_absmax(wave_max(amax));
      const float inv = 1.0f / scale;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int c = (j * 64 + lane) * 4;
        if (c < d) *reinterpret_cast<uint32_t*>(qr + c) = quant_pack4(v[j], inv);
      }
      for (int c = d + lane; c < ldq; c += 64) qr[c] = 0;
      if (lane == 0) scales[row] = scale;
    }
  } else {
    if (out) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int c = (j * 64 + lane) * 4;
        if (c < d) *reinterpret_cast<float4*>(out + static_cast<size_t>(row) * d + c) = v[j];
      }
    }
  }
}

// ---- Generic LayerNorm for any d (three passes over the row in cache).
__global__ __launch_bounds__(256) void layernorm_any_kernel(
    float* __restrict__ x, const float* __restrict__ resid, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, float* __restrict__ out,
    int rows, int d, float* tensor_absmax, int round16) {
  const int lane = threadIdx.x & 63;
  // As layernorm_vec_kernel: with a per-tensor absmax a wave past the last
  // row recomputes that row, stores nothing and joins the block's reduction.
  const int row0 = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const bool live = row0 < rows;
  if (!live && !tensor_absmax) return;
  const int row = live ? row0 : rows - 1;
  float* xr = x + static_cast<size_t>(row) * d;
  if (resid && live) {
    const float* rr = resid + static_cast<size_t>(row) * d;
    for (int c = lane; c < d; c += 64) xr[c] += rr[c];
  }
  float sum = 0.f;
  for (int c = lane; c < d; c += 64) sum += xr[c];
  const float mean = wave_sum(sum) / static_cast<float>(d);
  float sq = 0.f;
  for (int c = lane; c < d; c += 64) {
    const float a = xr[c] - mean;
    sq += a * a;
  }
  const float var = wave_sum(sq) / static_cast<float>(d);
  const float inv_std = 1.0f / sqrtf(var + eps);
  float amax = 0.f;
  float* yr = out + static_cast<size_t>(row) * d;
  for (int c = lane; c < d; c += 64) {
    float y = (xr[c] - mean) * inv_std * gamma[c] + beta[c];
    if (round16) y = static_cast<float>(static_cast<_Float16>(y));
    if (live) yr[c] = y;
    amax = fmaxf(amax, fabsf(y));
  }
  if (tensor_absmax) block_atomic_max_nonneg(tensor_absmax, live ? amax : 0.0f);
}

template <int KIND>
__device__ __forceinline__ float load_as_f32(const void* p, size_t i) {
  if constexpr (KIND == 0) return static_cast<const float*>(p)[i];
  if constexpr (KIND == 1) return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// ---- Per-row quantisation: one wave per row.
template <int KIND>
__global__ __launch_bounds__(256) void quant_rows_kernel(
    const void* __restrict__ x, int ldx, int rows, int cols,
    int8_t* __restrict__ q, int ldq, float* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t base = static_cast<size_t>(row) * ldx;
  float amax = 0.f;
  for (int c = lane; c < cols; c += 64) amax = fmaxf(amax, fabsf(load_as_f32<KIND>(x, base + c)));
  const float scale = act_scale_from_absmax(wave_max(amax));
  const float inv = 1.0f / scale;
  int8_t* qr = q + static_cast<size_t>(row) * ldq;
  for (int c = lane; c < cols; c += 64) qr[c] = static_cast<int8_t>(quant_i8(load_as_f32<KIND>(x, base + c), inv));
  for (int c = cols + lane; c < ldq; c += 64) qr[c] = 0;
  if (lane == 0) scales[row] = scale;
}

// Vectorised fp32 per-row quantisation (cols % 4 == 0, cols <= NV*256).
template <int NV>
__global__ __launch_bounds__(256) void quant_rows_vec_kernel(
    const float* __restrict__ x, int ldx, int rows, int cols,
    int8_t* __restrict__ q, int ldq, float* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + static_cast<size_t>(row) * ldx;
  float4 v[NV];
  load_row_vec<NV>(xr, cols, lane, v);
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
  const float scale = act_scale_from_absmax(wave_max(amax));
  const float inv = 1.0f / scale;
  int8_t* qr = q + static_cast<size_t>(row) * ldq;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    if (c < cols) {
      *reinterpret_cast<uint32_t*>(qr + c) = quant_pack4(v[j], inv);
    }
  }
  for (int c = cols + lane; c < ldq; c += 64) qr[c] = 0;
  if (lane == 0) scales[row] = scale;
}

// GELU fused with per-row quantisation (cols % 4 == 0, cols <= NV*256): the
// fc1 output row is read once, GELU'd in registers, its absmax taken, and it
// is written as int8 with the row's scale. The registers hold 2 gelu(x)
// (gelu2_as); halving the absmax and the reciprocal scale are exact, so the
// bytes and the scale are those of quantising gelu(x) itself. FULL: cols ==
// NV*256, no column masking.
template <int NV, bool FULL>
__global__ __launch_bounds__(256) void gelu_quant_rows_kernel(
    const float* __restrict__ x, int ldx, int rows, int cols,
    int8_t* __restrict__ q, int ldq, float* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + static_cast<size_t>(row) * ldx;
  float4 v[NV];
  if constexpr (FULL) {
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = *reinterpret_cast<const float4*>(xr + (j * 64 + lane) * 4);
  } else {
    load_row_vec<NV>(xr, cols, lane, v);  // gelu(0) == 0: zeroed chunks stay zero
  }
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    v[j].x = gelu2_as(v[j].x);
    v[j].y = gelu2_as(v[j].y);
    v[j].z = gelu2_as(v[j].z);
    v[j].w = gelu2_as(v[j].w);
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
  }
  const float scale = act_scale_from_absmax(0.5f * wave_max(amax));
  const float inv = 0.5f * (1.0f / scale);
  int8_t* qr = q + static_cast<size_t>(row) * ldq;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    if (FULL || c < cols) *reinterpret_cast<uint32_t*>(qr + c) = quant_pack4(v[j], inv);
  }
  for (int c = cols + lane; c < ldq; c += 64) qr[c] = 0;
  if (lane == 0) scales[row] = scale;
}

// The same pass over the INT8 GEMM's 24-bit fc1 output (kEpiF32R24): a
// high plane xh of bits 31..16 (row pitch ldx) and a low plane xl of bits
// 15..8 that interleaves row pairs (byte (r & ~1) ldx + 4 (p / 2) + 2 (r & 1)
// + (p & 1) holds row r, stored position p); stored position 2 i + j of each
// aligned 64-column group holds column 32 j + i. WAVES waves share a row (1:
// four rows per block; 2: two rows; 4: one row, several waves' maxima
// meeting in LDS), each wave NV * 512 stored positions, eight consecutive
// ones per lane per step: one 16-byte high load, and one 16-byte low load
// that holds them for both rows of the pair (the pair's two rows are read
// by the same block, or for WAVES 4 by two blocks on the same XCD, so the
// line comes from HBM once), give columns 4 k .. 4 k + 3 and 32 + 4 k ..
// (k = position / 8 within the group), whose int8 values go out as two
// 4-byte words. cols % 64 == 0.
template <int NV, int WAVES>
__global__ __launch_bounds__(256) void gelu_quant_rows_r24_kernel(
    const uint16_t* __restrict__ xh, const uint8_t* __restrict__ xl, int ldx, int rows, int cols,
    int8_t* __restrict__ q, int ldq, float* __restrict__ scales) {
  static_assert(WAVES == 1 || WAVES == 2 || WAVES == 4, "one, two or four waves per row");
  __shared__ float s_max[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // WAVES 4 (one row per block): blocks 16 g + 8 h + x take row 16 g + 2 x +
  // h, so a row pair's two blocks land on XCD x (the dispatcher sends block
  // b to XCD b mod 8) and share that XCD's L2.
  const int row = WAVES == 4 ? (blockIdx.x & ~15) + 2 * (blockIdx.x & 7) + ((blockIdx.x >> 3) & 1)
                             : blockIdx.x * (kRowsPerBlock / WAVES) + wave / WAVES;
  if (WAVES == 1 && row >= rows) return;
  // Several waves per row: every wave reaches the barrier below; a row past
  // the end reads row 0 and stores nothing.
  const bool live = row < rows;
  const int part = wave % WAVES;
  const int rr = live ? row : 0;
  const uint16_t* hr = xh + static_cast<size_t>(rr) * ldx;
  const uint8_t* lr = xl + static_cast<size_t>(rr & ~1) * ldx;
  const uint32_t odd = static_cast<uint32_t>(rr & 1);
  uint4 hv[NV], lv[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int p0 = (part * NV + j) * 512 + lane * 8;
    const int pc = p0 < cols ? p0 : 0;  // in bounds; zeroed below
    hv[j] = *reinterpret_cast<const uint4*>(hr + pc);
    lv[j] = *reinterpret_cast<const uint4*>(lr + 2 * pc);
  }
  float v[NV][8];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const bool ok = (part * NV + j) * 512 + lane * 8 < cols;
    const uint32_t hw[4] = {hv[j].x, hv[j].y, hv[j].z, hv[j].w};
    const uint32_t lw[4] = {lv[j].x, lv[j].y, lv[j].z, lv[j].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // bytes: 0, this row's low byte of position e (word e / 2, byte
      // (e & 1) + 2 odd), the high plane's 16 bits of e
      const uint32_t sel = 0x0cu | ((static_cast<uint32_t>(e & 1) + 2u * odd) << 8) | ((4u + 2u * (e & 1)) << 16) |
                           ((5u + 2u * (e & 1)) << 24);
      // Past the row's end the input is zeroed before the GELU (gelu2_as(0)
      // is +0), a select rather than a branch around the GELU, so that the
      // eight independent GELUs of a vector stay in one basic block and
      // their latencies overlap.
      const float x = __uint_as_float(__builtin_amdgcn_perm(hw[e >> 1], lw[e >> 1], sel));
      v[j][e] = gelu2_as(ok ? x : 0.0f);
      amax = fmaxf(amax, fabsf(v[j][e]));
    }
  }
  amax = wave_max(amax);
  if constexpr (WAVES > 1) {
    if (lane == 0) s_max[wave] = amax;
    __syncthreads();
    const int w0 = wave - part;
    amax = s_max[w0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) amax = fmaxf(amax, s_max[w0 + w]);
    if (!live) return;
  }
  const float scale = act_scale_from_absmax(0.5f * amax);
  const float inv = 0.5f * (1.0f / scale);
  int8_t* qr = q + static_cast<size_t>(row) * ldq;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int p0 = (part * NV + j) * 512 + lane * 8;
    if (p0 < cols) {
      const int c = (p0 & ~63) + ((p0 & 63) >> 1);  // column of position p0: group start + 4 k
      *reinterpret_cast<uint32_t*>(qr + c) = quant_pack4(make_float4(v[j][0], v[j][2], v[j][4], v[j][6]), inv);
      *reinterpret_cast<uint32_t*>(qr + c + 32) =
          quant_pack4(make_float4(v[j][1], v[j][3], v[j][5], v[j][7]), inv);
    }
  }
  if (part == 0) {
    for (int c = cols + lane; c < ldq; c += 64) qr[c] = 0;
    if (lane == 0) scales[row] = scale;
  }
}

// The same pass with a row split over the block's four waves, for rows
// wider than 5120 (ESM-2 3B's d_ff of 10240): wave w holds columns
// [w * NV * 256, (w + 1) * NV * 256), the waves' maxima meet in LDS, and each
// wave quantises its own part. One wave per 10240-wide row needs 160
// registers per lane for the row (three waves per SIMD); split four ways it
// needs 40 (seven): configuration 5's forward measured 87.6 against 88.7 ms.
// At 5120 columns the split measured 160 against 162 us and left the
// configuration-4 forward unchanged, so that width keeps the one-wave kernel.
// Bytes and scales are those of gelu_quant_rows_kernel (the maximum does not
// depend on the order it is taken in).
template <int NV>
__global__ __launch_bounds__(256) void gelu_quant_rows_split_kernel(
    const float* __restrict__ x, int ldx, int rows, int cols,
    int8_t* __restrict__ q, int ldq, float* __restrict__ scales) {
  __shared__ float s_max[kRowsPerBlock];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x;  // uniform: the whole block takes one row
  const int c0 = wave * NV * 256;
  const float* xr = x + static_cast<size_t>(row) * ldx;
  // Every load is issued before the first use; chunks past the row re-read
  // its start (in bounds) and are zeroed (gelu(0) == 0 keeps them zero).
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = c0 + (j * 64 + lane) * 4;
    v[j] = *reinterpret_cast<const float4*>(xr + (c < cols ? c : 0));
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const bool ok = c0 + (j * 64 + lane) * 4 < cols;
    v[j].x = ok ? v[j].x : 0.0f;
    v[j].y = ok ? v[j].y : 0.0f;
    v[j].z = ok ? v[j].z : 0.0f;
    v[j].w = ok ? v[j].w : 0.0f;
  }
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    v[j].x = gelu2_as(v[j].x);
    v[j].y = gelu2_as(v[j].y);
    v[j].z = gelu2_as(v[j].z);
    v[j].w = gelu2_as(v[j].w);
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
  }
  amax = wave_max(amax);
  if (lane == 0) s_max[wave] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
  const float scale = act_scale_from_absmax(0.5f * amax);
  const float inv = 0.5f * (1.0f / scale);
  int8_t* qr = q + static_cast<size_t>(row) * ldq;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = c0 + (j * 64 + lane) * 4;
    if (c < cols) *reinterpret_cast<uint32_t*>(qr + c) = quant_pack4(v[j], inv);
  }
  for (int c = cols + threadIdx.x; c < ldq; c += 256) qr[c] = 0;
  if (threadIdx.x == 0) scales[row] = scale;
}

// ---- Per-tensor quantisation with a device-resident absmax.
__global__ __launch_bounds__(256) void quant_tensor_kernel(
    const float* __restrict__ x, int ldx, int rows, int cols,
    const float* __restrict__ absmax, int8_t* __restrict__ q, int ldq,
    float* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float scale = act_scale_from_absmax(*absmax);
  const float inv = 1.0f / scale;
  const float* xr = x + static_cast<size_t>(row) * ldx;
  int8_t* qr = q + static_cast<size_t>(row) * ldq;
  int c0 = 0;
  if ((cols | ldx | ldq) % 4 == 0) {
    // Four values per lane per step: one 16-byte load, quant_i8 of each
    // (its NaN rule included), one packed 4-byte store.
    for (int c = lane * 4; c < cols; c += 256) {
      const float4 v = *reinterpret_cast<const float4*>(xr + c);
      *reinterpret_cast<uint32_t*>(qr + c) =
          (static_cast<uint32_t>(quant_i8(v.x, inv)) & 0xffu) | ((static_cast<uint32_t>(quant_i8(v.y, inv)) & 0xffu) << 8) |
          ((static_cast<uint32_t>(quant_i8(v.z, inv)) & 0xffu) << 16) | (static_cast<uint32_t>(quant_i8(v.w, inv)) << 24);
    }
    c0 = cols;
  }
  for (int c = c0 + lane; c < cols; c += 64) qr[c] = static_cast<int8_t>(quant_i8(xr[c], inv));
  for (int c = cols + lane; c < ldq; c += 64) qr[c] = 0;
  if (lane == 0) scales[row] = scale;
}

__device__ __forceinline__ float absmax4(float m, const float4& v) {
  return fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
}

// max |x[i]| over n values into *absmax (NaNs ignored, as fmaxf does). A
// 16-byte aligned x is read as float4, eight loads in flight per thread.
__global__ __launch_bounds__(256) void absmax_kernel(const float* __restrict__ x,
                                                     size_t n, float* absmax) {
  float m = 0.f;
  const size_t tid = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  size_t done = 0;
  if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const size_t n4 = n / 4;
    constexpr int kU = 8;
    size_t i = tid;
    for (; i + (kU - 1) * stride < n4; i += kU * stride) {
      float4 v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) v[u] = x4[i + u * stride];
#pragma unroll
      for (int u = 0; u < kU; ++u) m = absmax4(m, v[u]);
    }
    for (; i < n4; i += stride) m = absmax4(m, x4[i]);
    done = n4 * 4;
  }
  for (size_t i = done + tid; i < n; i += stride) m = fmaxf(m, fabsf(x[i]));
  block_atomic_max_nonneg(absmax, m);
}

// One workgroup of 1024 threads: the largest of n non-negative floats.
__global__ __launch_bounds__(1024) void max_of_kernel(const float* __restrict__ x, size_t n, float* out) {
  __shared__ float s_max[16];
  float m = 0.0f;
  for (size_t i = threadIdx.x; i < n; i += 1024) m = fmaxf(m, x[i]);
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = s_max[0];
#pragma unroll
    for (int w = 1; w < 16; ++w) r = fmaxf(r, s_max[w]);
    *out = r;
  }
}

__global__ void fill_kernel(float* x, size_t n, float v) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    x[i] = v;
}

__global__ void observe_gather_kernel(const float* __restrict__ x, const uint32_t* __restrict__ pos, int count,
                                      int gelu, float* __restrict__ out) {
  const int w = blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= count) return;
  float v = x[pos[w]];
  if (gelu) v = 0.5f * gelu2_as(v);
  out[w] = fabsf(v);
}

// The same over kEpiF32R24's planes (xh bits 31..16 with row pitch cols;
// xl bits 15..8 with row pairs interleaved; stored position 2 i + j of each
// 64-column group holds column 32 j + i): |GELU(x)| of the 24-bit values the
// GELU + quantisation pass reads.
__global__ void observe_gather_r24_kernel(const uint16_t* __restrict__ xh, const uint8_t* __restrict__ xl, int cols,
                                          const uint32_t* __restrict__ pos, int count, float* __restrict__ out) {
  const int w = blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= count) return;
  const uint32_t i = pos[w], r = i / static_cast<uint32_t>(cols), c = i - r * static_cast<uint32_t>(cols);
  const uint32_t p = (c & ~63u) + 2u * (c & 31u) + ((c >> 5) & 1u);  // stored position of column c
  const size_t at = static_cast<size_t>(r) * cols + p;
  const size_t lo = static_cast<size_t>(r & ~1u) * cols + 4u * (p >> 1) + 2u * (r & 1u) + (p & 1u);
  const float v = __uint_as_float((static_cast<uint32_t>(xh[at]) << 16) | (static_cast<uint32_t>(xl[lo]) << 8));
  out[w] = fabsf(0.5f * gelu2_as(v));
}

__global__ void gelu_kernel(const float* __restrict__ x, float* __restrict__ out, size_t n) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    out[i] = gelu_erf(x[i]);
}

__global__ void residual_kernel(float* __restrict__ y, const float* __restrict__ x, size_t n) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    y[i] += x[i];
}

__global__ void scale_kernel(float* __restrict__ x, size_t n, float s) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    x[i] *= s;
}

// One thread per (token, head, i < head_dim/2) rotary pair.
__global__ void rope_f32_kernel(float* __restrict__ x, int ld, const int* __restrict__ pos,
                                int T, int heads, int dh, const float* __restrict__ cos_tab,
                                const float* __restrict__ sin_tab, int tab_ld, float pre_scale) {
  const int half = dh / 2;
  const size_t total = static_cast<size_t>(T) * heads * half;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int c = static_cast<int>(i % half);
    const size_t th = i / half;
    const int h = static_cast<int>(th % heads);
    const int t = static_cast<int>(th / heads);
    const int p = pos[t];
    float* xr = x + static_cast<size_t>(t) * ld + static_cast<size_t>(h) * dh;
    const float* cr = cos_tab + static_cast<size_t>(p) * tab_ld;
    const float* sr = sin_tab + static_cast<size_t>(p) * tab_ld;
    const float x1 = xr[c] * pre_scale, x2 = xr[c + half] * pre_scale;
    // Same fused forms as the QKV GEMM epilogue's rotation.
    xr[c] = __builtin_fmaf(x1, cr[c], -(x2 * sr[c]));
    xr[c + half] = __builtin_fmaf(x2, cr[c + half], x1 * sr[c + half]);
  }
}

__global__ void embed_kernel(const int* __restrict__ ids, const float* __restrict__ tok_scale,
                             const float* __restrict__ embed, int T, int d, int mask_id,
                             float* __restrict__ out) {
  const size_t total = static_cast<size_t>(T) * d;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int t = static_cast<int>(i / d);
    const int c = static_cast<int>(i % d);
    const int id = ids[t];
    const float s = tok_scale[t];
    out[i] = (id == mask_id || s == 0.0f) ? 0.0f : embed[static_cast<size_t>(id) * d + c] * s;
  }
}

// One wave per token row, float4 copies (d % 4 == 0): the same values as
// embed_kernel without its per-element index division.
__global__ __launch_bounds__(256) void embed_rows_kernel(const int* __restrict__ ids,
                                                         const float* __restrict__ tok_scale,
                                                         const float* __restrict__ embed, int T, int d, int mask_id,
                                                         float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (t >= T) return;
  const int id = ids[t];
  const float s = tok_scale[t];
  const bool zero = id == mask_id || s == 0.0f;
  const f32x4* src = reinterpret_cast<const f32x4*>(embed + static_cast<size_t>(id) * d);
  f32x4* dst = reinterpret_cast<f32x4*>(out + static_cast<size_t>(t) * d);
  for (int c = lane; c < d / 4; c += 64) {
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    if (!zero) v = src[c] * s;
    __builtin_nontemporal_store(v, dst + c);
  }
}

__global__ void cast_kernel(const float* __restrict__ x, size_t n, uint16_t* __restrict__ out,
                            int to_bf16) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    out[i] = to_bf16 ? f32_to_bf16_bits(x[i]) : f32_to_f16_bits(x[i]);
}

inline dim3 grid_for(size_t n, int block = 256) {
  size_t g = (n + block - 1) / block;
  if (g > 65536) g = 65536;
  if (g == 0) g = 1;
  return dim3(static_cast<unsigned>(g));
}

inline dim3 rows_grid(int rows) { return dim3((rows + kRowsPerBlock - 1) / kRowsPerBlock); }

// Grid bound of the kernels that fold a per-tensor maximum with one atomic
// per block (four blocks per CU).
constexpr unsigned kReduceBlocks = 1024;

}  // namespace

hipError_t launch_layernorm(float* x, const float* resid, const float* gamma, const float* beta, float eps,
                            float* out, int rows, int d, float* tensor_absmax, hipStream_t s, int round16) {
  if (rows <= 0 || d <= 0) return hipSuccess;
  dim3 g = rows_grid(rows);
  const dim3 b(256);
  // With a per-tensor maximum the vectorised kernel walks the rows with a
  // bounded grid: one atomic per block.
  if (tensor_absmax && d % 4 == 0 && d <= 2560 && g.x > kReduceBlocks) g.x = kReduceBlocks;
  if (!out && !(tensor_absmax && d % 4 == 0 && d <= 2560)) return hipErrorInvalidValue;
  if (d % 4 == 0 && d <= 1280) {
    hipLaunchKernelGGL((layernorm_vec_kernel<5, false>), g, b, 0, s, x, resid, gamma, beta, eps, out, rows, d,
                       tensor_absmax, nullptr, 0, nullptr, round16);
  } else if (d % 4 == 0 && d <= 2560) {
    hipLaunchKernelGGL((layernorm_vec_kernel<10, false>), g, b, 0, s, x, resid, gamma, beta, eps, out, rows, d,
                       tensor_absmax, nullptr, 0, nullptr, round16);
  } else {
    hipLaunchKernelGGL(layernorm_any_kernel, g, b, 0, s, x, resid, gamma, beta, eps, out, rows, d, tensor_absmax,
                       round16);
  }
  return hipGetLastError();
}

hipError_t launch_layernorm_quant(float* x, const float* resid, const float* gamma, const float* beta, float eps,
                                  int rows, int d, int8_t* q, int ldq, float* scales, hipStream_t s, int round16) {
  if (rows <= 0 || d <= 0) return hipSuccess;
  if (d % 4 != 0 || d > 2560) return hipErrorInvalidValue;
  const dim3 g = rows_grid(rows), b(256);
  if (d <= 1280) {
    hipLaunchKernelGGL((layernorm_vec_kernel<5, true>), g, b, 0, s, x, resid, gamma, beta, eps, nullptr, rows, d,
                       nullptr, q, ldq, scales, round16);
  } else {
    hipLaunchKernelGGL((layernorm_vec_kernel<10, true>), g, b, 0, s, x, resid, gamma, beta, eps, nullptr, rows, d,
                       nullptr, q, ldq, scales, round16);
  }
  return hipGetLastError();
}

hipError_t launch_layernorm_quant_tensor(float* x, const float* gamma, const float* beta, float eps, int rows, int d,
                                         const float* absmax, int8_t* q, int ldq, float* scales, hipStream_t s,
                                         int round16) {
  if (rows <= 0 || d <= 0) return hipSuccess;
  if (d % 4 != 0 || d > 2560 || !absmax) return hipErrorInvalidValue;
  const dim3 g = rows_grid(rows), b(256);
  float* amax = const_cast<float*>(absmax);  // read only in the QUANT instantiation
  if (d <= 1280) {
    hipLaunchKernelGGL((layernorm_vec_kernel<5, true>), g, b, 0, s, x, nullptr, gamma, beta, eps, nullptr, rows, d,
                       amax, q, ldq, scales, round16);
  } else {
    hipLaunchKernelGGL((layernorm_vec_kernel<10, true>), g, b, 0, s, x, nullptr, gamma, beta, eps, nullptr, rows, d,
                       amax, q, ldq, scales, round16);
  }
  return hipGetLastError();
}

hipError_t launch_layernorm_quant_split(float* x, const SplitResid& r, const float* gamma, const float* beta,
                                        float eps, int rows, int d, int8_t* q, int ldq, float* scales,
                                        hipStream_t s, int round16) {
  if (rows <= 0 || d <= 0) return hipSuccess;
  if (d % 4 != 0 || d > 2560 || r.splits < 1 || !r.planes || !r.a_scale || !r.w_scale) return hipErrorInvalidValue;
  const dim3 g = rows_grid(rows), b(256);
  if (d <= 1280) {
    hipLaunchKernelGGL((layernorm_vec_kernel<5, true, true>), g, b, 0, s, x, nullptr, gamma, beta, eps, nullptr, rows,
                       d, nullptr, q, ldq, scales, round16, r);
  } else {
    hipLaunchKernelGGL((layernorm_vec_kernel<10, true, true>), g, b, 0, s, x, nullptr, gamma, beta, eps, nullptr,
                       rows, d, nullptr, q, ldq, scales, round16, r);
  }
  return hipGetLastError();
}

hipError_t launch_gelu_quant_rows(const float* x, int ldx, int rows, int cols, int8_t* q, int ldq, float* scales,
                                  hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (cols % 4 != 0 || ldx % 4 != 0 || cols > 10240) return hipErrorInvalidValue;
  const dim3 g = rows_grid(rows), b(256);
  if (cols == 5120) {  // ESM-2 650M's d_ff
    hipLaunchKernelGGL((gelu_quant_rows_kernel<20, true>), g, b, 0, s, x, ldx, rows, cols, q, ldq, scales);
  } else if (cols <= 1280) {
    hipLaunchKernelGGL((gelu_quant_rows_kernel<5, false>), g, b, 0, s, x, ldx, rows, cols, q, ldq, scales);
  } else if (cols <= 5120) {
    hipLaunchKernelGGL((gelu_quant_rows_kernel<20, false>), g, b, 0, s, x, ldx, rows, cols, q, ldq, scales);
  } else {
    // One block (four waves) per row, up to 2560 columns per wave.
    hipLaunchKernelGGL((gelu_quant_rows_split_kernel<10>), dim3(rows), b, 0, s, x, ldx, rows, cols, q, ldq, scales);
  }
  return hipGetLastError();
}

hipError_t launch_gelu_quant_rows_r24(const uint16_t* xh, const uint8_t* xl, int ldx, int rows, int cols, int8_t* q,
                                      int ldq, float* scales, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (cols % 64 != 0 || ldx % 8 != 0 || ldq % 4 != 0 || cols > 10240) return hipErrorInvalidValue;
  const dim3 b(256);
  // Below kSplitRows rows a one-wave-per-row grid leaves most SIMDs with one
  // or two waves, each waiting out its row's load latency alone: two waves
  // per row double the waves in flight (same bytes, same codes).
  constexpr int kSplitRows = 8192;
  if (cols <= 5120 && rows < kSplitRows)
    hipLaunchKernelGGL((gelu_quant_rows_r24_kernel<5, 2>), dim3((rows + 1) / 2), b, 0, s, xh, xl, ldx, rows, cols, q,
                       ldq, scales);
  else if (cols <= 5120)
    hipLaunchKernelGGL((gelu_quant_rows_r24_kernel<10, 1>), rows_grid(rows), b, 0, s, xh, xl, ldx, rows, cols, q, ldq,
                       scales);
  else
    hipLaunchKernelGGL((gelu_quant_rows_r24_kernel<5, 4>), dim3((rows + 15) & ~15), b, 0, s, xh, xl, ldx, rows, cols,
                       q, ldq, scales);
  return hipGetLastError();
}

hipError_t launch_quant_rows(const void* x, int src_kind, int ldx, int rows, int cols, int8_t* q,
                             int ldq, float* scales, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  const dim3 g = rows_grid(rows), b(256);
  if (src_kind == 0 && cols % 4 == 0 && ldx % 4 == 0 && cols <= 1280) {
    hipLaunchKernelGGL(quant_rows_vec_kernel<5>, g, b, 0, s, static_cast<const float*>(x), ldx, rows, cols, q,
                       ldq, scales);
  } else if (src_kind == 0 && cols % 4 == 0 && ldx % 4 == 0 && cols <= 5120) {
    hipLaunchKernelGGL(quant_rows_vec_kernel<20>, g, b, 0, s, static_cast<const float*>(x), ldx, rows, cols, q,
                       ldq, scales);
  } else if (src_kind == 0) {
    hipLaunchKernelGGL(quant_rows_kernel<0>, g, b, 0, s, x, ldx, rows, cols, q, ldq, scales);
  } else if (src_kind == 1) {
    hipLaunchKernelGGL(quant_rows_kernel<1>, g, b, 0, s, x, ldx, rows, cols, q, ldq, scales);
  } else {
    hipLaunchKernelGGL(quant_rows_kernel<2>, g, b, 0, s, x, ldx, rows, cols, q, ldq, scales);
  }
  return hipGetLastError();
}

hipError_t launch_quant_tensor(const float* x, int ldx, int rows, int cols, const float* absmax,
                               int8_t* q, int ldq, float* scales, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(quant_tensor_kernel, rows_grid(rows), dim3(256), 0, s, x, ldx, rows, cols, absmax, q,
                     ldq, scales);
  return hipGetLastError();
}

hipError_t launch_absmax(const float* x, size_t n, float* absmax, hipStream_t s) {
  if (n == 0) return hipSuccess;
  size_t g = (n / 4 + 255) / 256;
  if (g < 1) g = 1;
  if (g > 512) g = 512;  // two per CU: one atomic each
  hipLaunchKernelGGL(absmax_kernel, dim3(static_cast<unsigned>(g)), dim3(256), 0, s, x, n, absmax);
  return hipGetLastError();
}

hipError_t launch_max_of(const float* x, size_t n, float* out, hipStream_t s) {
  hipLaunchKernelGGL(max_of_kernel, dim3(1), dim3(1024), 0, s, x, n, out);
  return hipGetLastError();
}

hipError_t launch_observe_gather_r24(const uint16_t* xh, const uint8_t* xl, int cols, const uint32_t* pos, int count,
                                     float* out, hipStream_t s) {
  if (count <= 0) return hipSuccess;
  if (cols <= 0 || cols % 64 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(observe_gather_r24_kernel, dim3((count + 255) / 256), dim3(256), 0, s, xh, xl, cols, pos, count,
                     out);
  return hipGetLastError();
}

hipError_t launch_observe_gather(const float* x, const uint32_t* pos, int count, int gelu, float* out,
                                 hipStream_t s) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(observe_gather_kernel, dim3((count + 255) / 256), dim3(256), 0, s, x, pos, count, gelu, out);
  return hipGetLastError();
}

hipError_t launch_fill_f32(float* x, size_t n, float v, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_kernel, grid_for(n), dim3(256), 0, s, x, n, v);
  return hipGetLastError();
}

hipError_t launch_gelu(const float* x, float* out, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(gelu_kernel, grid_for(n), dim3(256), 0, s, x, out, n);
  return hipGetLastError();
}

hipError_t launch_residual_add(float* y, const float* x, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(residual_kernel, grid_for(n), dim3(256), 0, s, y, x, n);
  return hipGetLastError();
}

hipError_t launch_scale(float* x, size_t n, float scale, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(scale_kernel, grid_for(n), dim3(256), 0, s, x, n, scale);
  return hipGetLastError();
}

hipError_t launch_rope_f32(float* x, int ld, const int* pos, int T, int heads, int head_dim,
                           const float* cos_tab, const float* sin_tab, int tab_ld, float pre_scale,
                           hipStream_t s) {
  const size_t n = static_cast<size_t>(T) * heads * (head_dim / 2);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(rope_f32_kernel, grid_for(n), dim3(256), 0, s, x, ld, pos, T, heads, head_dim, cos_tab,
                     sin_tab, tab_ld, pre_scale);
  return hipGetLastError();
}

hipError_t launch_embed(const int* ids, const float* tok_scale, const float* embed, int T, int d,
                        int mask_token_id, float* out, hipStream_t s) {
  const size_t n = static_cast<size_t>(T) * d;
  if (n == 0) return hipSuccess;
  if (d % 4 == 0) {
    hipLaunchKernelGGL(embed_rows_kernel, rows_grid(T), dim3(256), 0, s, ids, tok_scale, embed, T, d, mask_token_id,
                       out);
  } else {
    hipLaunchKernelGGL(embed_kernel, grid_for(n), dim3(256), 0, s, ids, tok_scale, embed, T, d, mask_token_id,
                       out);
  }
  return hipGetLastError();
}

hipError_t launch_cast_f32(const float* x, size_t n, uint16_t* out, int to_bf16, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(cast_kernel, grid_for(n), dim3(256), 0, s, x, n, out, to_bf16);
  return hipGetLastError();
}

}  // namespace esm_gfx950
