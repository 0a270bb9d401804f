// Reference-side bridge to the gfx950 backend (see gfx950_bridge.h). Host
// code only: it includes the reference's headers and calls the C ABI of
// libesm_gfx950.so. Its one reference dependency is BatchView's
// constructor (src/batch.cpp), which the library it lives in already holds.
#include "gfx950_bridge.h"

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

namespace esm::gfx950 {
namespace {

std::mutex g_mu;                // one forward / op in flight (model.h:176-181)
std::string g_error;            // last failure, for LastError()

esm_gfx950_ctx* make_ctx() {
  esm_gfx950_ctx* c = nullptr;
  if (esm_gfx950_init(0, &c) != ESM_GFX950_OK) {
    g_error = "esm_gfx950_init failed (no gfx950 device)";
    return nullptr;
  }
  return c;
}

// Grow-only device buffers, one per argument slot of an arm (the analogue of
// the Workspace arena: no allocation once the largest call has been seen).
struct Slot {
  void* d = nullptr;
  std::size_t bytes = 0;
};
Slot g_slots[8];

void* slot(int i, std::size_t bytes) {
  Slot& s = g_slots[i];
  if (bytes > s.bytes) {
    if (s.d) esm_gfx950_free(Ctx(), s.d);
    s.d = nullptr;
    s.bytes = 0;
    if (esm_gfx950_malloc(Ctx(), bytes, &s.d) != ESM_GFX950_OK) return nullptr;
    s.bytes = bytes;
  }
  return s.d;
}

// Device copy of `bytes` host bytes in slot i (nullptr on failure).
void* upload(int i, const void* host, std::size_t bytes) {
  void* d = slot(i, std::max<std::size_t>(bytes, 4));
  if (d && bytes && esm_gfx950_memcpy_h2d(Ctx(), d, host, bytes) != ESM_GFX950_OK) return nullptr;
  return d;
}

bool fail() {
  esm_gfx950_ctx* c = Ctx();
  g_error = c ? esm_gfx950_last_error(c) : "no gfx950 context";
  return false;
}

bool ok(int rc) { return rc == ESM_GFX950_OK || fail(); }

bool download(void* host, const void* dev, std::size_t bytes) {
  return ok(esm_gfx950_memcpy_d2h(Ctx(), host, dev, bytes));
}

// Device weights by QuantizedTensor. The reference-side integration keeps
// the handle in a new QuantizedTensor member, freed by its destructor; this
// bridge, which cannot change that struct, keeps it in a side table keyed by
// the tensor's address and checked against its packed data pointer, shape and
// a checksum of its scales, so that a tensor rebuilt in reused storage is
// uploaded again.
struct DevWeight {
  esm_gfx950_weight* w = nullptr;
  const std::int8_t* data = nullptr;
  int N = 0, K = 0;
  std::uint64_t scale_sum = 0;
  std::uint64_t value_sum = 0;
};

// FNV-1a over the scales' bytes: N floats, cheap next to any call's staging.
std::uint64_t scale_checksum(const esm::quant::QuantizedTensor& W) {
  std::uint64_t h = 1469598103934665603ull;
  const auto* b = reinterpret_cast<const unsigned char*>(W.per_channel_scales.data());
  for (std::size_t i = 0; i < W.per_channel_scales.size() * sizeof(float); ++i) h = (h ^ b[i]) * 1099511628211ull;
  return h;
}
// FNV-1a over 4096 int8 values spread evenly over the tensor (all of them
// when it has fewer) and its size: a rewrite in place of more than a few
// values changes it.
std::uint64_t value_checksum(const esm::quant::QuantizedTensor& W) {
  constexpr std::size_t kSamples = 4096;
  const std::size_t n = W.packed.size();
  std::uint64_t h = 1469598103934665603ull ^ n;
  const std::size_t step = n > kSamples ? n / kSamples : 1;
  for (std::size_t i = 0; i < n; i += step)
    h = (h ^ static_cast<unsigned char>(W.packed[i])) * 1099511628211ull;
  return h;
}

std::unordered_map<const esm::quant::QuantizedTensor*, DevWeight> g_weights;

esm_gfx950_weight* device_weight(const esm::quant::QuantizedTensor& W) {
  DevWeight& e = g_weights[&W];
  const std::uint64_t sum = scale_checksum(W), vsum = value_checksum(W);
  if (e.w && e.data == W.packed.data() && e.N == W.N && e.K == W.K && e.scale_sum == sum && e.value_sum == vsum)
    return e.w;
  if (e.w) esm_gfx950_weight_free(Ctx(), e.w);
  e = DevWeight();
  if (static_cast<std::size_t>(W.N) * W.K != W.packed.size() ||
      W.per_channel_scales.size() != static_cast<std::size_t>(W.N)) {
    g_error = "LinearInt8: QuantizedTensor sizes do not match N x K";
    return nullptr;
  }
  if (esm_gfx950_weight_upload_i8(Ctx(), W.packed.data(), W.per_channel_scales.data(), W.N, W.K, &e.w) !=
      ESM_GFX950_OK) {
    fail();
    e = DevWeight();
    return nullptr;
  }
  e.data = W.packed.data();
  e.N = W.N;
  e.K = W.K;
  e.scale_sum = sum;
  e.value_sum = vsum;
  return e.w;
}

}  // namespace

esm_gfx950_ctx* Ctx() {
  static esm_gfx950_ctx* ctx = make_ctx();
  return ctx;
}

const char* LastError() {
  thread_local std::string copy;
  std::lock_guard<std::mutex> lk(g_mu);
  copy = g_error;
  return copy.c_str();
}

bool Linear(const float* A, const float* W, const float* bias, float* C, int M, int N, int K) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!Ctx()) return false;
  if (M <= 0 || N <= 0) return true;
  const std::size_t a = std::size_t(M) * std::max(K, 0) * 4, w = std::size_t(N) * std::max(K, 0) * 4;
  void* dA = upload(0, A, a);
  void* dW = upload(1, W, w);
  void* dB = bias ? upload(2, bias, std::size_t(N) * 4) : nullptr;
  void* dC = slot(3, std::size_t(M) * N * 4);
  if (!dA || !dW || (bias && !dB) || !dC) return fail();
  return ok(esm_gfx950_linear_f32(Ctx(), static_cast<const float*>(dA), static_cast<const float*>(dW),
                                  static_cast<const float*>(dB), static_cast<float*>(dC), M, N, K)) &&
         download(C, dC, std::size_t(M) * N * 4);
}

bool LinearInt8(const float* A, const esm::quant::QuantizedTensor& W, const float* bias, float* C, int M, int N,
                int K) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!Ctx()) return false;
  if (M <= 0 || N <= 0) return true;
  if (W.N != N || W.K != K) {
    g_error = "LinearInt8: QuantizedTensor is " + std::to_string(W.N) + " x " + std::to_string(W.K) +
              ", call is " + std::to_string(N) + " x " + std::to_string(K);
    return false;
  }
  esm_gfx950_weight* dW = device_weight(W);
  if (!dW) return false;
  void* dA = upload(0, A, std::size_t(M) * std::max(K, 0) * 4);
  void* dB = bias ? upload(2, bias, std::size_t(N) * 4) : nullptr;
  void* dC = slot(3, std::size_t(M) * N * 4);
  if (!dA || (bias && !dB) || !dC) return fail();
  return ok(esm_gfx950_linear_i8(Ctx(), static_cast<const float*>(dA), dW, static_cast<const float*>(dB),
                                 static_cast<float*>(dC), M, N, K, ESM_GFX950_ACT_PER_TENSOR)) &&
         download(C, dC, std::size_t(M) * N * 4);
}

void ReleaseWeight(const esm::quant::QuantizedTensor& W) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_weights.find(&W);
  if (it == g_weights.end()) return;
  if (it->second.w && Ctx()) esm_gfx950_weight_free(Ctx(), it->second.w);
  g_weights.erase(it);
}

bool LayerNorm(const float* x, const float* gamma, const float* beta, float eps, float* out, int num_rows, int d) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!Ctx()) return false;
  if (num_rows <= 0 || d <= 0) return true;
  const std::size_t n = std::size_t(num_rows) * d * 4;
  void* dx = upload(0, x, n);
  void* dg = upload(1, gamma, std::size_t(d) * 4);
  void* db = upload(2, beta, std::size_t(d) * 4);
  void* dy = slot(3, n);
  if (!dx || !dg || !db || !dy) return fail();
  return ok(esm_gfx950_layernorm(Ctx(), static_cast<const float*>(dx), static_cast<const float*>(dg),
                                 static_cast<const float*>(db), eps, static_cast<float*>(dy), num_rows, d)) &&
         download(out, dy, n);
}

bool Gelu(const float* x, float* out, std::size_t n) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!Ctx()) return false;
  if (n == 0) return true;
  void* dx = upload(0, x, n * 4);
  void* dy = slot(3, n * 4);
  if (!dx || !dy) return fail();
  return ok(esm_gfx950_gelu(Ctx(), static_cast<const float*>(dx), static_cast<float*>(dy), n)) &&
         download(out, dy, n * 4);
}

bool ResidualAddInplace(float* y, const float* x, std::size_t n) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!Ctx()) return false;
  if (n == 0) return true;
  void* dy = upload(3, y, n * 4);
  void* dx = upload(0, x, n * 4);
  if (!dx || !dy) return fail();
  return ok(esm_gfx950_residual_add(Ctx(), static_cast<float*>(dy), static_cast<const float*>(dx), n)) &&
         download(y, dy, n * 4);
}

bool ScaleInplace(float* x, std::size_t n, float scale) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!Ctx()) return false;
  if (n == 0) return true;
  void* dx = upload(3, x, n * 4);
  if (!dx) return fail();
  return ok(esm_gfx950_scale(Ctx(), static_cast<float*>(dx), n, scale)) && download(x, dx, n * 4);
}

bool RopeApplyVarlen(float* x, const float* cos, const float* sin, const int* cu_seqlens, int batch_size,
                     int num_heads, int head_dim) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!Ctx()) return false;
  if (batch_size <= 0) return true;
  int max_len = 0;
  for (int b = 0; b < batch_size; ++b) max_len = std::max(max_len, cu_seqlens[b + 1] - cu_seqlens[b]);
  const std::size_t T = static_cast<std::size_t>(std::max(cu_seqlens[batch_size], 0));
  const std::size_t nx = T * num_heads * head_dim * 4;
  void* dx = upload(3, x, nx);
  void* dc = upload(0, cos, std::size_t(max_len) * head_dim * 4);
  void* ds = upload(1, sin, std::size_t(max_len) * head_dim * 4);
  if (!dx || !dc || !ds) return fail();
  return ok(esm_gfx950_rope_apply_varlen(Ctx(), static_cast<float*>(dx), static_cast<const float*>(dc),
                                         static_cast<const float*>(ds), cu_seqlens, batch_size, num_heads,
                                         head_dim)) &&
         download(x, dx, nx);
}

bool AttentionVarlen(const float* q, const float* k, const float* v, const int* cu_seqlens, int batch_size,
                     int num_heads, int head_dim, float* out) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!Ctx()) return false;
  if (batch_size <= 0) return true;
  const std::size_t T = static_cast<std::size_t>(std::max(cu_seqlens[batch_size], 0));
  const std::size_t n = T * num_heads * head_dim * 4;
  if (n == 0) return true;
  void* dq = upload(0, q, n);
  void* dk = upload(1, k, n);
  void* dv = upload(2, v, n);
  void* dy = slot(3, n);
  if (!dq || !dk || !dv || !dy) return fail();
  const int precision = head_dim == 64 ? ESM_GFX950_ATTN_F16X3_MFMA : ESM_GFX950_ATTN_FP32;
  return ok(esm_gfx950_attention_varlen(Ctx(), static_cast<const float*>(dq), static_cast<const float*>(dk),
                                        static_cast<const float*>(dv), cu_seqlens, batch_size, num_heads, head_dim,
                                        static_cast<float*>(dy), precision)) &&
         download(out, dy, n);
}

namespace {

// The model's vocabulary and layer count, read back from the library.
bool model_dims(esm_gfx950_model* model, int* vocab, int* layers, int* hidden) {
  esm_gfx950_model_config c;
  if (esm_gfx950_model_get_config(model, &c) != ESM_GFX950_OK) {
    g_error = "model_get_config failed";
    return false;
  }
  *vocab = c.vocab_size;
  *layers = c.num_layers;
  *hidden = c.hidden_size;
  return true;
}

}  // namespace

bool ForwardPacked(esm_gfx950_model* model, const esm::BatchView& batch,
                   std::vector<std::vector<float>>* logits_per_seq_out,
                   std::vector<std::vector<float>>* hidden_packed_out) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!Ctx()) return false;
  if (!model) {
    g_error = "ForwardPacked: null model";
    return false;
  }
  const int T = static_cast<int>(batch.total_tokens());
  const int B = batch.batch_size;
  if (T == 0) {
    if (logits_per_seq_out) logits_per_seq_out->clear();
    if (hidden_packed_out) hidden_packed_out->clear();
    return true;
  }
  int V = 0, layers = 0, d = 0;
  if (!model_dims(model, &V, &layers, &d)) return false;
  const std::int32_t* masks = batch.packed_masks.empty() ? nullptr : batch.packed_masks.data();
  std::vector<float> packed(static_cast<std::size_t>(T) * V);
  if (hidden_packed_out) {
    std::vector<float> hidden(static_cast<std::size_t>(layers + 1) * T * d);
    if (!ok(esm_gfx950_forward_hidden_states(Ctx(), model, batch.packed_ids.data(), masks, batch.cu_seqlens.data(),
                                             B, T, packed.data(), hidden.data())))
      return false;
    const std::size_t Td = static_cast<std::size_t>(T) * d;
    hidden_packed_out->assign(static_cast<std::size_t>(layers + 1), {});
    for (int l = 0; l <= layers; ++l)
      (*hidden_packed_out)[l].assign(hidden.begin() + l * Td, hidden.begin() + (l + 1) * Td);
  } else if (!ok(esm_gfx950_forward_packed_masked(Ctx(), model, batch.packed_ids.data(), masks,
                                                  batch.cu_seqlens.data(), B, T, packed.data(), 0))) {
    return false;
  }
  if (logits_per_seq_out) {
    // The per-sequence split of model.cpp:1240-1252.
    logits_per_seq_out->resize(static_cast<std::size_t>(B));
    for (int b = 0; b < B; ++b) {
      const std::size_t start = static_cast<std::size_t>(batch.cu_seqlens[b]) * V;
      const std::size_t n = static_cast<std::size_t>(batch.sequence_length(b)) * V;
      (*logits_per_seq_out)[b].assign(packed.begin() + start, packed.begin() + start + n);
    }
  }
  return true;
}

bool ForwardScheduled(esm_gfx950_model* model, const std::vector<std::vector<std::int32_t>>& input_ids,
                      const std::vector<std::vector<std::int32_t>>& attention_masks,
                      const esm::SchedulerConfig& cfg, std::vector<std::vector<float>>* out) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!Ctx()) return false;
  out->clear();
  const std::size_t N = input_ids.size();
  if (N == 0) return true;
  if (!model) {
    g_error = "ForwardScheduled: null model";
    return false;
  }
  if (!attention_masks.empty() && attention_masks.size() != N) {
    g_error = "attention_masks/input_ids batch size mismatch";
    return false;
  }
  int V = 0, layers = 0, d = 0;
  if (!model_dims(model, &V, &layers, &d)) return false;
  out->resize(N);
  std::vector<std::int32_t> lens(N);
  for (std::size_t i = 0; i < N; ++i) {
    lens[i] = static_cast<std::int32_t>(input_ids[i].size());
    (*out)[i].resize(input_ids[i].size() * static_cast<std::size_t>(V));
  }
  if (attention_masks.empty()) {
    std::vector<const std::int32_t*> ids(N);
    std::vector<float*> outs(N);
    for (std::size_t i = 0; i < N; ++i) {
      ids[i] = input_ids[i].data();
      outs[i] = (*out)[i].data();
    }
    return ok(esm_gfx950_forward_scheduled(Ctx(), model, ids.data(), lens.data(), static_cast<int>(N),
                                           cfg.imbalance_threshold, cfg.max_batch_size, outs.data()));
  }
  // With masks: the plan of PlanBatches, each group one masked packed forward.
  for (std::size_t i = 0; i < N; ++i)
    if (attention_masks[i].size() != input_ids[i].size()) {
      g_error = "attention_masks[" + std::to_string(i) + "] does not match input_ids";
      return false;
    }
  std::vector<std::int32_t> order(N), sizes(N);
  int groups = 0;
  if (!ok(esm_gfx950_plan_batches(lens.data(), static_cast<int>(N), cfg.imbalance_threshold, cfg.max_batch_size,
                                  order.data(), sizes.data(), &groups)))
    return false;
  std::size_t at = 0;
  for (int g = 0; g < groups; ++g) {
    std::vector<std::int32_t> ids, masks, cu{0};
    const std::size_t first = at;
    for (int k = 0; k < sizes[g]; ++k, ++at) {
      const std::size_t i = static_cast<std::size_t>(order[at]);
      ids.insert(ids.end(), input_ids[i].begin(), input_ids[i].end());
      masks.insert(masks.end(), attention_masks[i].begin(), attention_masks[i].end());
      cu.push_back(static_cast<std::int32_t>(ids.size()));
    }
    if (sizes[g] == 0 || ids.empty()) continue;
    std::vector<float> packed(ids.size() * static_cast<std::size_t>(V));
    if (!ok(esm_gfx950_forward_packed_masked(Ctx(), model, ids.data(), masks.data(), cu.data(), sizes[g],
                                             static_cast<int>(ids.size()), packed.data(), 0)))
      return false;
    for (int k = 0; k < sizes[g]; ++k)
      std::copy(packed.begin() + static_cast<std::size_t>(cu[k]) * V,
                packed.begin() + static_cast<std::size_t>(cu[k + 1]) * V, (*out)[order[first + k]].begin());
  }
  return true;
}

}  // namespace esm::gfx950
