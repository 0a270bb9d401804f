// Reference-side bridge to the gfx950 backend (see gfx950_bridge.h). Host
// code only: it includes the reference's headers and calls the C ABI of
// libesm_gfx950.so; it links nothing of the reference.
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
};

// FNV-1a over the scales' bytes: N floats, cheap next to any call's staging.
std::uint64_t scale_checksum(const esm::quant::QuantizedTensor& W) {
  std::uint64_t h = 1469598103934665603ull;
  const auto* b = reinterpret_cast<const unsigned char*>(W.per_channel_scales.data());
  for (std::size_t i = 0; i < W.per_channel_scales.size() * sizeof(float); ++i) h = (h ^ b[i]) * 1099511628211ull;
  return h;
}
std::unordered_map<const esm::quant::QuantizedTensor*, DevWeight> g_weights;

esm_gfx950_weight* device_weight(const esm::quant::QuantizedTensor& W) {
  DevWeight& e = g_weights[&W];
  const std::uint64_t sum = scale_checksum(W);
  if (e.w && e.data == W.packed.data() && e.N == W.N && e.K == W.K && e.scale_sum == sum) return e.w;
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

}  // namespace esm::gfx950
