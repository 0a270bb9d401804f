// C entry points over the bridge's facade arms, for callers without C++
// (the Python tests among them): each builds the reference's types from
// plain host arrays and calls the arm of gfx950_bridge.h. Every function
// returns 1 when the device path ran and 0 when the caller must take its CPU
// arm (esm_gfx950_bridge_last_error says why).
#include <cstdint>
#include <cstring>

#include "gfx950_bridge.h"

namespace g = esm::gfx950;

extern "C" {

const char* esm_gfx950_bridge_last_error(void) { return g::LastError(); }

int esm_gfx950_bridge_linear(const float* A, const float* W, const float* bias, float* C, int M, int N, int K) {
  return g::Linear(A, W, bias, C, M, N, K) ? 1 : 0;
}

// packed [N, K] int8 and scales [N]: the contents of an
// esm::quant::QuantizedTensor, as Quantize (pack.cpp:149-177) leaves them.
int esm_gfx950_bridge_linear_int8(const float* A, const std::int8_t* packed, const float* scales,
                                  const float* bias, float* C, int M, int N, int K) {
  esm::quant::QuantizedTensor W;
  W.N = N;
  W.K = K;
  W.packed.assign(packed, packed + static_cast<std::size_t>(N) * K);
  W.per_channel_scales.assign(scales, scales + N);
  const bool ran = g::LinearInt8(A, W, bias, C, M, N, K);
  g::ReleaseWeight(W);
  return ran ? 1 : 0;
}

int esm_gfx950_bridge_layernorm(const float* x, const float* gamma, const float* beta, float eps, float* out,
                                int num_rows, int d) {
  return g::LayerNorm(x, gamma, beta, eps, out, num_rows, d) ? 1 : 0;
}

int esm_gfx950_bridge_gelu(const float* x, float* out, size_t n) { return g::Gelu(x, out, n) ? 1 : 0; }

int esm_gfx950_bridge_residual_add(float* y, const float* x, size_t n) {
  return g::ResidualAddInplace(y, x, n) ? 1 : 0;
}

int esm_gfx950_bridge_scale(float* x, size_t n, float scale) { return g::ScaleInplace(x, n, scale) ? 1 : 0; }

int esm_gfx950_bridge_rope_apply_varlen(float* x, const float* cos, const float* sin, const int* cu_seqlens,
                                        int batch_size, int num_heads, int head_dim) {
  return g::RopeApplyVarlen(x, cos, sin, cu_seqlens, batch_size, num_heads, head_dim) ? 1 : 0;
}

int esm_gfx950_bridge_attention_varlen(const float* q, const float* k, const float* v, const int* cu_seqlens,
                                       int batch_size, int num_heads, int head_dim, float* out) {
  return g::AttentionVarlen(q, k, v, cu_seqlens, batch_size, num_heads, head_dim, out) ? 1 : 0;
}

}  // extern "C"
