// ref_shim.cpp -- C-linkage wrappers around the reference's own kernel
// facade (esm::kernels::*, esm::quant::*), compiled from the unmodified
// reference sources under /root/reference by oracle/Makefile into
// oracle/_ref/libesmref.so.
//
// TEST INFRASTRUCTURE ONLY: used by tests/ to pin the oracle and by
// bench.py's cpu_baseline leg to time the reference CPU path; the product
// never loads it.
//
// The reference's Model::ForwardPackedInto lives in src/model.cpp, which
// includes a header that CMake generates at configure time
// (esm_cpp/artifact_trace_sha.h from cmake/artifact_trace_sha.h.in), so it
// is not buildable from its sources alone. esmref_forward_packed below
// restates its call sequence (src/model.cpp:932-1066 TransformerBlock,
// :1093-1255 ForwardPackedInto) over the reference's own kernel facade.
#include <immintrin.h>
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <unordered_map>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "esm_cpp/cpu_features.h"
#include "esm_cpp/io.h"
#include "esm_cpp/kernels.h"
#include "esm_cpp/observer.h"
#include "esm_cpp/quant.h"
#include "esm_cpp/scheduler.h"
#include "oracle.h"

namespace esm::kernels {
// Defined in the AVX-512 TU of gemm_int8.cpp (x86 builds).
void QuantizeActPrefixAvx512(const float* A, std::size_t MK, std::uint8_t* a_u8, float* act_scale_out);
void LinearVnni(const float* A, const esm::quant::QuantizedTensor& W, const float* bias, float* C, int M, int N,
                int K);
void AttentionVarlenAvx512(const float* q, const float* k, const float* v, const int* cu_seqlens, int batch_size,
                           int num_heads, int head_dim, float* out);
}  // namespace esm::kernels

namespace {

esm::quant::QuantizedTensor make_qt(const int8_t* packed, const float* scales, int N, int K) {
  esm::quant::QuantizedTensor qt;
  qt.N = N;
  qt.K = K;
  qt.packed.assign(packed, packed + static_cast<size_t>(N) * K);
  qt.per_channel_scales.assign(scales, scales + N);
  esm::quant::BuildKernelCache(&qt);
  return qt;
}

struct RefLayer {
  std::vector<float> ln1_w, ln1_b, ln2_w, ln2_b;
  esm::quant::QuantizedTensor w8[6];
  std::vector<float> w32[6];
  std::vector<float> bias[6];
  int N[6], K[6];
};

struct RefModel {
  or_model cfg{};
  std::vector<float> embed, final_ln_w, final_ln_b, lm_dense_w, lm_dense_b, lm_ln_w, lm_ln_b, dec_b;
  std::vector<RefLayer> layers;
};

std::vector<float> vec(const float* p, size_t n) { return std::vector<float>(p, p + n); }

// RoundToFp16Inplace (src/model.cpp:912-930) lives in model.cpp, which is
// not buildable here: the x86 F16C branch restated.
void or_round_fp16_shim(float* x, size_t n) {
  for (size_t i = 0; i < n; ++i)
    x[i] = _cvtsh_ss(_cvtss_sh(x[i], _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
}

}  // namespace

extern "C" {

const char* esmref_isa() {
  static std::string s;
  s = std::string(esm::IsaToString(esm::CurrentIsa()));
  return s.c_str();
}

const char* esmref_host_isa() {
  static std::string s;
  s = std::string(esm::IsaToString(esm::HostIsa()));
  return s.c_str();
}

void esmref_quantize(const float* W, int N, int K, int8_t* q, float* scales) {
  esm::quant::QuantizedTensor qt;
  esm::quant::Quantize(W, N, K, &qt);
  std::memcpy(q, qt.packed.data(), qt.packed.size());
  std::memcpy(scales, qt.per_channel_scales.data(), qt.per_channel_scales.size() * sizeof(float));
}

void esmref_linear_int8(const float* A, const int8_t* packed, const float* scales, const float* bias, float* C, int M,
                        int N, int K) {
  auto qt = make_qt(packed, scales, N, K);
  esm::kernels::LinearInt8(A, qt, bias, C, M, N, K);
}

void esmref_linear_int8_ref(const float* A, const int8_t* packed, const float* scales, const float* bias, float* C,
                            int M, int N, int K) {
  auto qt = make_qt(packed, scales, N, K);
  esm::kernels::LinearInt8Ref(A, qt, bias, C, M, N, K);
}

int esmref_has_avx512_prefix() {
#if defined(__x86_64__)
  return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") ? 1 : 0;
#else
  return 0;
#endif
}

// QuantizeActPrefixAvx512 (gemm_int8.cpp:391-508): u8 with zero-point 128.
void esmref_quant_act_prefix(const float* A, size_t MK, uint8_t* q, float* scale) {
  esm::kernels::QuantizeActPrefixAvx512(A, MK, q, scale);
}

void esmref_linear_vnni(const float* A, const int8_t* packed, const float* scales, const float* bias, float* C, int M,
                        int N, int K) {
  auto qt = make_qt(packed, scales, N, K);
  esm::kernels::LinearVnni(A, qt, bias, C, M, N, K);
}

void esmref_linear(const float* A, const float* W, const float* bias, float* C, int M, int N, int K) {
  esm::kernels::Linear(A, W, bias, C, M, N, K);
}
void esmref_linear_ref(const float* A, const float* W, const float* bias, float* C, int M, int N, int K) {
  esm::kernels::LinearRef(A, W, bias, C, M, N, K);
}
void esmref_layernorm_ref(const float* x, const float* g, const float* b, float eps, float* out, int rows, int d) {
  esm::kernels::LayerNormRef(x, g, b, eps, out, rows, d);
}
void esmref_layernorm(const float* x, const float* g, const float* b, float eps, float* out, int rows, int d) {
  esm::kernels::LayerNorm(x, g, b, eps, out, rows, d);
}
void esmref_gelu_ref(const float* x, float* out, size_t n) { esm::kernels::GeluRef(x, out, n); }
void esmref_gelu(const float* x, float* out, size_t n) { esm::kernels::Gelu(x, out, n); }
void esmref_rope_tables(int L, int dh, float* c, float* s) { esm::kernels::RopeBuildTables(L, dh, c, s); }
void esmref_rope_varlen_ref(float* x, const float* c, const float* s, const int* cu, int B, int H, int dh) {
  esm::kernels::RopeApplyVarlenRef(x, c, s, cu, B, H, dh);
}
void esmref_rope_varlen(float* x, const float* c, const float* s, const int* cu, int B, int H, int dh) {
  esm::kernels::RopeApplyVarlen(x, c, s, cu, B, H, dh);
}
void esmref_attention_varlen_ref(const float* q, const float* k, const float* v, const int* cu, int B, int H, int dh,
                                 float* out) {
  esm::kernels::AttentionVarlenRef(q, k, v, cu, B, H, dh, out);
}
void esmref_attention_varlen(const float* q, const float* k, const float* v, const int* cu, int B, int H, int dh,
                             float* out) {
  esm::kernels::AttentionVarlen(q, k, v, cu, B, H, dh, out);
}

// ---------------------------------------------------------------- model
void* esmref_model_create(const or_model* m) {
  auto* r = new RefModel();
  r->cfg = *m;
  const int d = m->hidden, f = m->ffn, V = m->vocab;
  r->embed = vec(m->embed, static_cast<size_t>(V) * d);
  r->layers.resize(m->num_layers);
  const int Ns[6] = {d, d, d, d, f, d};
  const int Ks[6] = {d, d, d, d, d, f};
  for (int l = 0; l < m->num_layers; ++l) {
    RefLayer& L = r->layers[l];
    L.ln1_w = vec(m->ln1_w[l], d);
    L.ln1_b = vec(m->ln1_b[l], d);
    L.ln2_w = vec(m->ln2_w[l], d);
    L.ln2_b = vec(m->ln2_b[l], d);
    for (int j = 0; j < 6; ++j) {
      const int idx = l * 6 + j;
      L.N[j] = Ns[j];
      L.K[j] = Ks[j];
      L.bias[j] = vec(m->bias[idx], Ns[j]);
      if (m->weights_int8) {
        L.w8[j] = make_qt(m->w_i8[idx], m->w_scale[idx], Ns[j], Ks[j]);
      } else {
        L.w32[j] = vec(m->w_f32[idx], static_cast<size_t>(Ns[j]) * Ks[j]);
      }
    }
  }
  r->final_ln_w = vec(m->final_ln_w, d);
  r->final_ln_b = vec(m->final_ln_b, d);
  r->lm_dense_w = vec(m->lm_dense_w, static_cast<size_t>(d) * d);
  r->lm_dense_b = vec(m->lm_dense_b, d);
  r->lm_ln_w = vec(m->lm_ln_w, d);
  r->lm_ln_b = vec(m->lm_ln_b, d);
  r->dec_b = vec(m->lm_decoder_bias, V);
  return r;
}

void esmref_model_free(void* h) { delete static_cast<RefModel*>(h); }

// Restated ForwardPackedInto over the reference facade, with the reference's
// own ActivationObserver (null: none) fed at TransformerBlock's four sites
// (src/model.cpp:952-955,996-999,1023-1026,1047-1050). Returns 0.
int esmref_forward_packed_observed(void* h, const int32_t* ids, const int32_t* cu, int B, int T, float* logits,
                                   void* observer) {
  auto* obs = static_cast<esm::ActivationObserver*>(observer);
  auto* r = static_cast<RefModel*>(h);
  const or_model& c = r->cfg;
  const int d = c.hidden, H = c.heads, dh = c.head_dim, f = c.ffn, V = c.vocab;
  const size_t Td = static_cast<size_t>(T) * d, Tf = static_cast<size_t>(T) * f;
  int maxL = 0;
  for (int b = 0; b < B; ++b) maxL = std::max(maxL, cu[b + 1] - cu[b]);
  std::vector<float> hidden(Td), ln(Td), qkv(3 * Td), cs(static_cast<size_t>(maxL) * dh),
      sn(static_cast<size_t>(maxL) * dh), attn(Td), proj(Td), inter(Tf), inter_g(Tf);
  // Embed (model.cpp:737-778).
  const float k_drop = 0.15f * 0.8f;
  for (int b = 0; b < B; ++b) {
    int src_len = 0, masks = 0;
    for (int t = cu[b]; t < cu[b + 1]; ++t) {
      ++src_len;
      if (ids[t] == c.mask_token_id) ++masks;
    }
    const float ratio = src_len > 0 ? static_cast<float>(masks) / static_cast<float>(src_len) : 0.0f;
    const float scale = (1.0f - k_drop) / std::max(1.0f - ratio, 1e-12f);
    for (int t = cu[b]; t < cu[b + 1]; ++t) {
      const float* row = r->embed.data() + static_cast<size_t>(ids[t]) * d;
      float* o = hidden.data() + static_cast<size_t>(t) * d;
      for (int i = 0; i < d; ++i) o[i] = ids[t] == c.mask_token_id ? 0.0f : row[i] * scale;
    }
  }
  auto linear = [&](const RefLayer& L, int j, const float* A, float* C, int M) {
    if (c.weights_int8) {
      esm::kernels::LinearInt8(A, L.w8[j], L.bias[j].data(), C, M, L.N[j], L.K[j]);
    } else {
      esm::kernels::Linear(A, L.w32[j].data(), L.bias[j].data(), C, M, L.N[j], L.K[j]);
    }
  };
  int li = 0;
  for (const RefLayer& L : r->layers) {
    const std::string site = "layer" + std::to_string(li++) + ".";
    float* q = qkv.data();
    float* k = qkv.data() + Td;
    float* v = qkv.data() + 2 * Td;
    esm::kernels::LayerNorm(hidden.data(), L.ln1_w.data(), L.ln1_b.data(), c.eps, ln.data(), T, d);
    if (obs) obs->Observe(site + "attn_ln_output", ln.data(), Td);
    linear(L, 0, ln.data(), q, T);
    linear(L, 1, ln.data(), k, T);
    linear(L, 2, ln.data(), v, T);
    const float q_scale = 1.0f / std::sqrt(static_cast<float>(dh));
    esm::kernels::ScaleInplace(q, Td, q_scale);
    esm::kernels::RopeBuildTables(maxL, dh, cs.data(), sn.data());
    esm::kernels::RopeApplyVarlen(q, cs.data(), sn.data(), cu, B, H, dh);
    esm::kernels::RopeApplyVarlen(k, cs.data(), sn.data(), cu, B, H, dh);
    esm::kernels::AttentionVarlen(q, k, v, cu, B, H, dh, attn.data());
    if (obs) obs->Observe(site + "attn_out", attn.data(), Td);
    linear(L, 3, attn.data(), proj.data(), T);
    esm::kernels::ResidualAddInplace(hidden.data(), proj.data(), Td);
    esm::kernels::LayerNorm(hidden.data(), L.ln2_w.data(), L.ln2_b.data(), c.eps, ln.data(), T, d);
    if (obs) obs->Observe(site + "ffn_ln_output", ln.data(), Td);
    if (c.fc1_fp16 && &L == &r->layers.front()) or_round_fp16_shim(ln.data(), ln.size());
    linear(L, 4, ln.data(), inter.data(), T);
    esm::kernels::Gelu(inter.data(), inter_g.data(), Tf);
    if (obs) obs->Observe(site + "inter_gelu", inter_g.data(), Tf);
    linear(L, 5, inter_g.data(), proj.data(), T);
    esm::kernels::ResidualAddInplace(hidden.data(), proj.data(), Td);
  }
  esm::kernels::LayerNorm(hidden.data(), r->final_ln_w.data(), r->final_ln_b.data(), c.eps, ln.data(), T, d);
  esm::kernels::Linear(ln.data(), r->lm_dense_w.data(), r->lm_dense_b.data(), proj.data(), T, d, d);
  esm::kernels::Gelu(proj.data(), attn.data(), Td);
  esm::kernels::LayerNorm(attn.data(), r->lm_ln_w.data(), r->lm_ln_b.data(), c.eps, ln.data(), T, d);
  esm::kernels::Linear(ln.data(), r->embed.data(), r->dec_b.data(), logits, T, V, d);
  return 0;
}

int esmref_forward_packed(void* h, const int32_t* ids, const int32_t* cu, int B, int T, float* logits) {
  return esmref_forward_packed_observed(h, ids, cu, B, T, logits, nullptr);
}

// The reference's ActivationObserver (src/quant/observer.cpp) behind C
// linkage.
void* esmref_observer_new() { return new esm::ActivationObserver(); }
void esmref_observer_free(void* h) { delete static_cast<esm::ActivationObserver*>(h); }
void esmref_observer_clear(void* h) { static_cast<esm::ActivationObserver*>(h)->Clear(); }
void esmref_observer_observe(void* h, const char* key, const float* values, size_t n) {
  static_cast<esm::ActivationObserver*>(h)->Observe(key, values, n);
}
// Percentile of one site: 1 and *out when the site exists, else 0.
int esmref_observer_percentile(void* h, const char* key, float pctile, float* out) {
  const auto all = static_cast<esm::ActivationObserver*>(h)->Percentile(pctile);
  auto it = all.find(key);
  if (it == all.end()) return 0;
  *out = it->second;
  return 1;
}
int esmref_observer_site_count(void* h) {
  return static_cast<int>(static_cast<esm::ActivationObserver*>(h)->Percentile(50.0f).size());
}

// Model::SaveToGguf (src/model.cpp:562-700) restated over a RefModel: the
// same metadata keys, tensor names, shapes and order, written by the
// reference's own GgufFile::Write (src/io/gguf.cpp:391-465). Returns 0, or -1
// with the exception message printed.
int esmref_gguf_save_model(void* h, const char* path) {
  auto* r = static_cast<RefModel*>(h);
  const or_model& c = r->cfg;
  using G = esm::io::GgufFile;
  const bool q = c.weights_int8 != 0;
  const uint64_t d = c.hidden, f = c.ffn, V = c.vocab;
  std::unordered_map<std::string, G::MetadataValue> meta;
  meta.emplace("general.architecture", std::string("esm"));
  meta.emplace("general.alignment", static_cast<std::int64_t>(32));
  meta.emplace("general.file_type", static_cast<std::int64_t>(q ? 2 : 1));
  meta.emplace("esm.block_count", static_cast<std::int64_t>(c.num_layers));
  meta.emplace("esm.embedding_length", static_cast<std::int64_t>(d));
  meta.emplace("esm.feed_forward_length", static_cast<std::int64_t>(f));
  meta.emplace("esm.attention.head_count", static_cast<std::int64_t>(c.heads));
  meta.emplace("esm.attention.head_count_kv", static_cast<std::int64_t>(c.heads));
  meta.emplace("esm.attention.layer_norm_epsilon", static_cast<double>(c.eps));
  meta.emplace("esm.rope.dimension_count", static_cast<std::int64_t>(c.head_dim));
  meta.emplace("esm.context_length", static_cast<std::int64_t>(1024));
  meta.emplace("esm.gguf_writer", std::string("esm-cpp 0.1.0"));
  meta.emplace("esm.weights_quantized", q);
  meta.emplace("esm.first_block_fc1_fp16", c.fc1_fp16 != 0);
  auto f32 = [](const std::vector<float>& w, std::vector<uint64_t> shape) {
    G::WriteTensor t;
    t.dtype = G::GgmlType::F32;
    t.shape = std::move(shape);
    t.data = w.data();
    t.size_bytes = w.size() * sizeof(float);
    return t;
  };
  std::vector<std::vector<std::byte>> blobs;
  blobs.reserve(static_cast<size_t>(c.num_layers) * 6);
  auto q8 = [&](const esm::quant::QuantizedTensor& qt, uint64_t K, uint64_t N) {
    std::vector<std::byte> b(qt.packed.size() + qt.per_channel_scales.size() * sizeof(float));
    std::memcpy(b.data(), qt.packed.data(), qt.packed.size());
    std::memcpy(b.data() + qt.packed.size(), qt.per_channel_scales.data(), qt.per_channel_scales.size() * 4);
    blobs.push_back(std::move(b));
    G::WriteTensor t;
    t.dtype = G::GgmlType::Q8_ESM;
    t.shape = {K, N};
    t.data = blobs.back().data();
    t.size_bytes = blobs.back().size();
    return t;
  };
  auto name = [](int i, const char* s) { return "blk." + std::to_string(i) + "." + s; };
  std::vector<std::pair<std::string, G::WriteTensor>> t;
  t.emplace_back("token_embd.weight", f32(r->embed, {d, V}));
  const char* wn[6] = {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight", "ffn_up.weight",
                       "ffn_down.weight"};
  const char* bn[6] = {"attn_q.bias", "attn_k.bias", "attn_v.bias", "attn_output.bias", "ffn_up.bias",
                       "ffn_down.bias"};
  for (int i = 0; i < c.num_layers; ++i) {
    const RefLayer& L = r->layers[i];
    t.emplace_back(name(i, "attn_norm.weight"), f32(L.ln1_w, {d}));
    t.emplace_back(name(i, "attn_norm.bias"), f32(L.ln1_b, {d}));
    for (int j = 0; j < 4; ++j)
      t.emplace_back(name(i, wn[j]), q ? q8(L.w8[j], d, d) : f32(L.w32[j], {d, d}));
    for (int j = 0; j < 4; ++j) t.emplace_back(name(i, bn[j]), f32(L.bias[j], {d}));
    t.emplace_back(name(i, "ffn_norm.weight"), f32(L.ln2_w, {d}));
    t.emplace_back(name(i, "ffn_norm.bias"), f32(L.ln2_b, {d}));
    t.emplace_back(name(i, wn[4]), q ? q8(L.w8[4], d, f) : f32(L.w32[4], {d, f}));
    t.emplace_back(name(i, wn[5]), q ? q8(L.w8[5], f, d) : f32(L.w32[5], {f, d}));
    t.emplace_back(name(i, bn[4]), f32(L.bias[4], {f}));
    t.emplace_back(name(i, bn[5]), f32(L.bias[5], {d}));
  }
  t.emplace_back("enc_norm.weight", f32(r->final_ln_w, {d}));
  t.emplace_back("enc_norm.bias", f32(r->final_ln_b, {d}));
  t.emplace_back("lm_head.weight", f32(r->lm_dense_w, {d, d}));
  t.emplace_back("lm_head.bias", f32(r->lm_dense_b, {d}));
  t.emplace_back("lm_head_norm.weight", f32(r->lm_ln_w, {d}));
  t.emplace_back("lm_head_norm.bias", f32(r->lm_ln_b, {d}));
  t.emplace_back("output.bias", f32(r->dec_b, {V}));
  try {
    G::Write(path, meta, t);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "esmref_gguf_save_model: %s\n", e.what());
    return -1;
  }
  return 0;
}

// One tensor of a GGUF file through the reference's reader
// (GgufFile::Open, src/io/gguf.cpp:251-340): type, dims, byte size, and up to
// `cap` bytes of data. Returns 0, 1 when the tensor is absent, -1 when the
// reader rejects the file.
int esmref_gguf_tensor(const char* path, const char* tname, void* data, size_t cap, uint32_t* type,
                       uint64_t* shape, uint32_t* ndim, size_t* bytes) {
  try {
    auto gf = esm::io::GgufFile::Open(path);
    auto info = gf->Get(tname);
    if (!info) return 1;
    *type = static_cast<uint32_t>(info->dtype);
    *ndim = static_cast<uint32_t>(info->shape.size());
    for (size_t i = 0; i < info->shape.size() && i < 8; ++i) shape[i] = info->shape[i];
    *bytes = info->size_bytes;
    if (cap) std::memcpy(data, info->data, std::min(cap, info->size_bytes));
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "esmref_gguf_tensor: %s\n", e.what());
    return -1;
  }
}

// Integer / bool / float metadata through the reference's reader: *kind 0
// absent, 1 int, 2 float, 3 bool, 4 string (length in *ival).
int esmref_gguf_meta(const char* path, const char* key, int* kind, int64_t* ival, double* fval) {
  try {
    auto gf = esm::io::GgufFile::Open(path);
    auto v = gf->Metadata(key);
    *kind = 0;
    if (!v) return 0;
    if (auto* i = std::get_if<std::int64_t>(&*v)) { *kind = 1; *ival = *i; }
    else if (auto* x = std::get_if<double>(&*v)) { *kind = 2; *fval = *x; }
    else if (auto* b = std::get_if<bool>(&*v)) { *kind = 3; *ival = *b ? 1 : 0; }
    else if (auto* s = std::get_if<std::string>(&*v)) { *kind = 4; *ival = static_cast<int64_t>(s->size()); }
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "esmref_gguf_meta: %s\n", e.what());
    return -1;
  }
}

// PlanBatches (src/sched/scheduler.cpp:54-75) flattened: the caller-index
// order of every group back to back in `order`, group sizes in `sizes`.
int esmref_plan_batches(const int32_t* lengths, int n, float imbalance_threshold, int max_batch_size,
                        int32_t* order, int32_t* sizes, int* num_groups) {
  std::vector<int> len(lengths, lengths + n);
  esm::SchedulerConfig cfg;
  cfg.imbalance_threshold = imbalance_threshold;
  cfg.max_batch_size = max_batch_size;
  const auto plan = esm::PlanBatches(len, cfg);
  int k = 0, g = 0;
  for (const auto& group : plan) {
    sizes[g++] = static_cast<int32_t>(group.size());
    for (int i : group) order[k++] = i;
  }
  *num_groups = g;
  return 0;
}

}  // extern "C"
