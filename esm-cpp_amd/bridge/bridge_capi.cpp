// C entry points over the bridge's facade arms, for callers without C++
// (the Python tests among them): each builds the reference's types from
// plain host arrays and calls the arm of gfx950_bridge.h. Every function
// returns 1 when the device path ran and 0 when the caller must take its CPU
// arm (esm_gfx950_bridge_last_error says why).
#include <cstdint>
#include <cstring>
#include <span>
#include <stdexcept>
#include <string>
#include <vector>

#include "gfx950_bridge.h"

namespace g = esm::gfx950;

namespace {
// A failure raised in this layer (BatchView's validation), reported by
// esm_gfx950_bridge_last_error in place of the arm's message.
thread_local std::string g_capi_error;
}  // namespace

extern "C" {

const char* esm_gfx950_bridge_last_error(void) {
  return g_capi_error.empty() ? g::LastError() : g_capi_error.c_str();
}

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

// Model::ForwardPackedInto's device path through a BatchView built from
// the arrays (cu_len entries of cu, masks: NULL or [T]): logits of every
// sequence back to back in
// logits [T, vocab] (each the [L_b * vocab] buffer of the per-sequence
// split), hidden (NULL or [layers + 1, T, d]) the packed hidden states.
// Returns 1 when the device path ran, 0 when it failed, -1 when BatchView
// rejected the batch (std::invalid_argument; its message in last_error).
int esm_gfx950_bridge_forward_packed(esm_gfx950_model* model, const std::int32_t* ids, const std::int32_t* masks,
                                     const std::int32_t* cu, int cu_len, int batch_size, int total_tokens,
                                     float* logits, float* hidden) {
  g_capi_error.clear();
  const std::size_t T = total_tokens > 0 ? static_cast<std::size_t>(total_tokens) : 0;
  const std::size_t ncu = cu_len > 0 ? static_cast<std::size_t>(cu_len) : 0;
  std::vector<std::vector<float>> per_seq, states;
  try {
    const esm::BatchView view(std::span<const std::int32_t>(ids, T),
                              masks ? std::span<const std::int32_t>(masks, T) : std::span<const std::int32_t>(),
                              std::span<const std::int32_t>(cu, ncu), batch_size);
    if (!g::ForwardPacked(model, view, &per_seq, hidden ? &states : nullptr)) return 0;
  } catch (const std::invalid_argument& e) {
    g_capi_error = e.what();
    return -1;
  }
  std::size_t at = 0;
  for (const auto& v : per_seq) {
    std::memcpy(logits + at, v.data(), v.size() * sizeof(float));
    at += v.size();
  }
  std::size_t hat = 0;
  for (const auto& v : states) {
    std::memcpy(hidden + hat, v.data(), v.size() * sizeof(float));
    hat += v.size();
  }
  return 1;
}

// Model::ForwardScheduled's device path: n sequences back to back in ids
// (lengths[i] tokens each), masks NULL or laid out like ids; logits of
// sequence i at the same offset times vocab, in input order.
int esm_gfx950_bridge_forward_scheduled(esm_gfx950_model* model, const std::int32_t* ids,
                                        const std::int32_t* lengths, const std::int32_t* masks, int n,
                                        float imbalance_threshold, int max_batch_size, float* logits) {
  g_capi_error.clear();
  std::vector<std::vector<std::int32_t>> seqs(n > 0 ? n : 0), mks;
  std::size_t at = 0;
  for (int i = 0; i < n; ++i) {
    seqs[i].assign(ids + at, ids + at + lengths[i]);
    if (masks) mks.emplace_back(masks + at, masks + at + lengths[i]);
    at += static_cast<std::size_t>(lengths[i]);
  }
  esm::SchedulerConfig cfg;
  cfg.imbalance_threshold = imbalance_threshold;
  cfg.max_batch_size = max_batch_size;
  std::vector<std::vector<float>> out;
  if (!g::ForwardScheduled(model, seqs, mks, cfg, &out)) return 0;
  std::size_t o = 0;
  for (const auto& v : out) {
    std::memcpy(logits + o, v.data(), v.size() * sizeof(float));
    o += v.size();
  }
  return 1;
}

// A QuantizedTensor that lives across calls (the weight cache's key), for
// tests of the cache: create, read its packed storage, run LinearInt8 on it,
// free (which releases its device copy, as the integration's destructor does).
void* esm_gfx950_bridge_qt_create(const std::int8_t* packed, const float* scales, int N, int K) {
  auto* W = new esm::quant::QuantizedTensor();
  W->N = N;
  W->K = K;
  W->packed.assign(packed, packed + static_cast<std::size_t>(N) * K);
  W->per_channel_scales.assign(scales, scales + N);
  return W;
}

std::int8_t* esm_gfx950_bridge_qt_data(void* qt) {
  return static_cast<esm::quant::QuantizedTensor*>(qt)->packed.data();
}

int esm_gfx950_bridge_linear_int8_qt(const float* A, void* qt, const float* bias, float* C, int M) {
  g_capi_error.clear();
  const auto& W = *static_cast<esm::quant::QuantizedTensor*>(qt);
  return g::LinearInt8(A, W, bias, C, M, W.N, W.K) ? 1 : 0;
}

void esm_gfx950_bridge_qt_free(void* qt) {
  auto* W = static_cast<esm::quant::QuantizedTensor*>(qt);
  g::ReleaseWeight(*W);
  delete W;
}

}  // extern "C"
