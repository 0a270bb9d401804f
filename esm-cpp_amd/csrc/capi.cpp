// C ABI of the gfx950 backend (declared in include/esm_gfx950.h): context
// and stream, device weight cache, op-level entry points mirroring
// esm::kernels::* and the device-resident packed forward that replaces
// Model::ForwardPackedInto (reference src/model.cpp:1093-1255).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <numeric>
#include <string>
#include <thread>
#include <vector>

#include "esm_gfx950.h"
#include "gguf.hpp"
#include "kernels.hpp"
#include "observer.hpp"

using namespace esm_gfx950;

namespace {

constexpr int kHeadDimMfma = 64;
// Power of two applied to Q before its split-fp16 split: keeps the lo parts
// of the pre-scaled (|q| ~ 0.1) values out of the fp16 subnormal range.
constexpr float kQPrescale = 8.0f;
// Most sequence groups the automatic group count uses.
constexpr int kAutoMaxParts = 3;

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
int pad16(int k) { return (k + 15) & ~15; }

}  // namespace

// Device scratch of esm_gfx950_linear_i8_noalloc (the allocation-free
// LinearInt8): the quantised activations, their scales and one absmax
// scalar. Every GPU the library runs on holds its own copy until the
// process ends. In host code `scratch` names a host-side stand-in, not device
// memory: its device address is taken at every esm_gfx950_init
// (hipGetSymbolAddress, that device current), kept in the context, and only
// that address is used. Taking it per context rather than once per process
// keeps it right after a hipDeviceReset, which may reload the code object.
constexpr size_t kNoAllocScratchBytes = size_t{64} << 20;
static __device__ __align__(256) int8_t scratch[kNoAllocScratchBytes];

namespace {
// The device address of `scratch` on the current device.
hipError_t scratch_address(void** out) {
  *out = nullptr;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (!p) return hipErrorInvalidSymbol;
  *out = p;
  return hipSuccess;
}
}  // namespace

struct esm_gfx950_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string err;
  std::string arch;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  // Device address of the static `scratch` array on this context's device.
  void* noalloc_scratch = nullptr;
  // Op-level scratch (grown on demand; the forward uses its own arena).
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  // Per-site kernel timing: each timed launch is bracketed by two events
  // recorded on the context stream; site_of[i] names the launch's site.
  bool timing = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> events;
  std::vector<std::string> site_of;
  size_t events_used = 0;

  int fail(int code, const std::string& msg) {
    err = msg;
    return code;
  }
  int hip_fail(const char* what, hipError_t e) {
    err = std::string(what) + ": " + hipGetErrorString(e);
    return ESM_GFX950_HIP_ERROR;
  }
  // Returns a device scratch region of at least `bytes` bytes.
  int get_scratch(size_t bytes, void** out) {
    if (bytes > scratch_bytes) {
      hipError_t e = hipStreamSynchronize(stream);
      if (e != hipSuccess) return hip_fail("hipStreamSynchronize", e);
      if (scratch) hipFree(scratch);
      scratch = nullptr;
      scratch_bytes = 0;
      const size_t n = align_up(bytes, 1 << 20);
      e = hipMalloc(&scratch, n);
      if (e != hipSuccess) return hip_fail("hipMalloc(scratch)", e);
      scratch_bytes = n;
    }
    *out = scratch;
    return ESM_GFX950_OK;
  }
  int time_begin(const char* site, int* slot) {
    *slot = -1;
    if (!timing) return ESM_GFX950_OK;
    if (events_used == events.size()) {
      hipEvent_t a, b;
      if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess)
        return fail(ESM_GFX950_HIP_ERROR, "hipEventCreate failed");
      events.emplace_back(a, b);
      site_of.emplace_back();
    }
    *slot = static_cast<int>(events_used++);
    site_of[*slot] = site;
    hipError_t e = hipEventRecord(events[*slot].first, stream);
    if (e != hipSuccess) return hip_fail("hipEventRecord", e);
    return ESM_GFX950_OK;
  }
  int time_end(int slot) {
    if (slot < 0) return ESM_GFX950_OK;
    hipError_t e = hipEventRecord(events[slot].second, stream);
    if (e != hipSuccess) return hip_fail("hipEventRecord", e);
    return ESM_GFX950_OK;
  }
};

struct esm_gfx950_weight {
  int N = 0, K = 0, ldk = 0;
  int8_t* data = nullptr;  // [N, ldk], zero past K
  float* scales = nullptr;  // [N]
};

// Activation observer (reference esm::ActivationObserver): per-site
// reservoirs on the host, plus device and pinned staging for the gathered
// values, grown on demand (kReservoirSize entries per site of one call).
struct esm_gfx950_observer {
  std::map<std::string, obs::Reservoir> sites;
  uint32_t* d_pos = nullptr;
  float* d_val = nullptr;
  uint32_t* h_pos = nullptr;
  float* h_val = nullptr;
  size_t cap_sites = 0;
};

#define ESM_HIP(ctx, expr)                                   \
  do {                                                       \
    hipError_t e_ = (expr);                                  \
    if (e_ != hipSuccess) return (ctx)->hip_fail(#expr, e_); \
  } while (0)

#define ESM_TRY(expr)                            \
  do {                                           \
    int rc_ = (expr);                            \
    if (rc_ != ESM_GFX950_OK) return rc_;        \
  } while (0)

#define ESM_REQUIRE(ctx, cond, msg)                                   \
  do {                                                                \
    if (!(cond)) return (ctx)->fail(ESM_GFX950_INVALID_ARGUMENT, msg); \
  } while (0)

namespace {

// BatchView validation (reference src/batch.cpp:8-46), same messages.
int validate_batch(esm_gfx950_ctx* ctx, const int32_t* cu, int batch_size, long total) {
  if (batch_size < 1) return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "BatchView: batch_size must be >= 1");
  if (!cu) return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "BatchView: cu_seqlens is null");
  if (cu[0] != 0) return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "BatchView: cu_seqlens[0] must be 0");
  for (int i = 1; i <= batch_size; ++i)
    if (cu[i] < cu[i - 1])
      return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "BatchView: cu_seqlens must be non-decreasing");
  if (total >= 0 && cu[batch_size] != total)
    return ctx->fail(ESM_GFX950_INVALID_ARGUMENT,
                     "BatchView: cu_seqlens.back() (" + std::to_string(cu[batch_size]) +
                         ") must equal packed_ids.size() (" + std::to_string(total) + ")");
  return ESM_GFX950_OK;
}

// Work list for the attention kernels: (sequence, head, query tile), longest
// sequences first so the long tiles start early and the short ones fill in.
//
// xcd_queues: workgroup i runs on XCD i % 8 (the dispatcher's round-robin),
// and each XCD has its own L2. The list is then laid out as 8 interleaved
// queues (item i belongs to queue i % 8); every (sequence, head) goes whole
// to the shortest queue, so its query tiles run on one XCD back to back and
// the later tiles re-read that head's K / V from that XCD's L2 instead of
// HBM. Queues are padded to equal length with items whose q0 lies past every
// sequence (the kernels return at once for those).
constexpr int kNumXcd = 8;
constexpr int kNoQueries = 1 << 30;

void build_work(const int32_t* cu, int B, int H, int qtile, std::vector<AttnWork>* out, bool xcd_queues = false) {
  std::vector<int> order(B);
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
    return (cu[a + 1] - cu[a]) > (cu[b + 1] - cu[b]);
  });
  out->clear();
  if (!xcd_queues) {
    for (int b : order) {
      const int L = cu[b + 1] - cu[b];
      for (int q0 = 0; q0 < L; q0 += qtile)
        for (int h = 0; h < H; ++h) out->push_back(AttnWork{b, h, q0, 0});
    }
    return;
  }
  std::vector<AttnWork> queue[kNumXcd];
  for (int b : order) {
    const int L = cu[b + 1] - cu[b];
    for (int h = 0; h < H; ++h) {
      int x = 0;
      for (int y = 1; y < kNumXcd; ++y)
        if (queue[y].size() < queue[x].size()) x = y;
      for (int q0 = 0; q0 < L; q0 += qtile) queue[x].push_back(AttnWork{b, h, q0, 0});
    }
  }
  size_t n = 0;
  for (const auto& qu : queue) n = std::max(n, qu.size());
  if (n == 0) return;
  for (auto& qu : queue) qu.resize(n, AttnWork{order[0], 0, kNoQueries, 0});
  out->reserve(n * kNumXcd);
  for (size_t i = 0; i < n; ++i)
    for (const auto& qu : queue) out->push_back(qu[i]);
}

// Upper bound of build_work's item count for B sequences of T tokens in
// all, the longest maxL tokens. Before padding there are at most
// H * (T / qtile + B) items (one per started query tile). Every (sequence,
// head) goes to the shortest queue, so no queue exceeds the mean by more
// than one (sequence, head)'s tiles, ceil(maxL / qtile); padding all
// kNumXcd queues to the longest adds at most kNumXcd times that.
size_t max_work_items(int B, int T, int maxL, int H, int qtile) {
  const size_t tiles_max = static_cast<size_t>(maxL) / qtile + 1;
  return static_cast<size_t>(H) * (static_cast<size_t>(B) + static_cast<size_t>(T) / qtile + 1) +
         kNumXcd * (tiles_max + 1);
}

// Position of every packed token inside its sequence.
void build_pos(const int32_t* cu, int B, int32_t* pos) {
  for (int b = 0; b < B; ++b)
    for (int t = cu[b]; t < cu[b + 1]; ++t) pos[t] = t - cu[b];
}

// RopeBuildTables (reference src/kernels/rope_tables.cpp:14-29): same float
// formula evaluated with the host C library.
void rope_tables(int seq_len, int head_dim, float* cos_t, float* sin_t) {
  const int half = head_dim / 2;
  for (int i = 0; i < half; ++i) {
    const float exponent = static_cast<float>(2 * i) / static_cast<float>(head_dim);
    const float inv_freq = std::pow(10000.0f, -exponent);
    for (int t = 0; t < seq_len; ++t) {
      const float angle = static_cast<float>(t) * inv_freq;
      const float c = std::cos(angle);
      const float s = std::sin(angle);
      cos_t[t * head_dim + i] = c;
      cos_t[t * head_dim + i + half] = c;
      sin_t[t * head_dim + i] = s;
      sin_t[t * head_dim + i + half] = s;
    }
  }
}

}  // namespace

// ------------------------------------------------------------------ context
extern "C" int esm_gfx950_init(int device, esm_gfx950_ctx** out) {
  if (!out) return ESM_GFX950_INVALID_ARGUMENT;
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= device || device < 0)
    return ESM_GFX950_HIP_ERROR;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return ESM_GFX950_HIP_ERROR;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return ESM_GFX950_HIP_ERROR;
  if (hipSetDevice(device) != hipSuccess) return ESM_GFX950_HIP_ERROR;
  void* noalloc = nullptr;
  if (scratch_address(&noalloc) != hipSuccess) return ESM_GFX950_HIP_ERROR;
  auto* ctx = new esm_gfx950_ctx();
  ctx->device = device;
  ctx->noalloc_scratch = noalloc;
  ctx->arch = prop.gcnArchName;
  if (hipStreamCreate(&ctx->stream) != hipSuccess || hipEventCreate(&ctx->t0) != hipSuccess ||
      hipEventCreate(&ctx->t1) != hipSuccess) {
    delete ctx;
    return ESM_GFX950_HIP_ERROR;
  }
  *out = ctx;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_destroy(esm_gfx950_ctx* ctx) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  if (ctx->scratch) hipFree(ctx->scratch);
  for (auto& e : ctx->events) {
    hipEventDestroy(e.first);
    hipEventDestroy(e.second);
  }
  hipEventDestroy(ctx->t0);
  hipEventDestroy(ctx->t1);
  hipStreamDestroy(ctx->stream);
  delete ctx;
  return ESM_GFX950_OK;
}

extern "C" const char* esm_gfx950_last_error(const esm_gfx950_ctx* ctx) {
  return ctx ? ctx->err.c_str() : "null context";
}

extern "C" const char* esm_gfx950_device_arch(const esm_gfx950_ctx* ctx) {
  return ctx ? ctx->arch.c_str() : "";
}

extern "C" int esm_gfx950_sync(esm_gfx950_ctx* ctx) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_malloc(esm_gfx950_ctx* ctx, size_t bytes, void** dptr) {
  if (!ctx || !dptr) return ESM_GFX950_INVALID_ARGUMENT;
  *dptr = nullptr;
  if (bytes == 0) bytes = 256;
  ESM_HIP(ctx, hipMalloc(dptr, bytes));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_free(esm_gfx950_ctx* ctx, void* dptr) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  if (!dptr) return ESM_GFX950_OK;
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  ESM_HIP(ctx, hipFree(dptr));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_memcpy_h2d(esm_gfx950_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  if (bytes == 0) return ESM_GFX950_OK;
  ESM_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_memcpy_d2h(esm_gfx950_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  if (bytes == 0) return ESM_GFX950_OK;
  ESM_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_memcpy_d2d(esm_gfx950_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  if (bytes == 0) return ESM_GFX950_OK;
  ESM_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_timer_start(esm_gfx950_ctx* ctx) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_HIP(ctx, hipEventRecord(ctx->t0, ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_timer_stop(esm_gfx950_ctx* ctx, float* elapsed_ms) {
  if (!ctx || !elapsed_ms) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_HIP(ctx, hipEventRecord(ctx->t1, ctx->stream));
  ESM_HIP(ctx, hipEventSynchronize(ctx->t1));
  ESM_HIP(ctx, hipEventElapsedTime(elapsed_ms, ctx->t0, ctx->t1));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_kernel_timing(esm_gfx950_ctx* ctx, int enable) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  ctx->timing = enable != 0;
  ctx->events_used = 0;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_kernel_timing_query(esm_gfx950_ctx* ctx, const char* site, int* launches,
                                              double* total_ms) {
  if (!ctx || !site || !launches || !total_ms) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  double sum = 0.0;
  int n = 0;
  for (size_t i = 0; i < ctx->events_used; ++i) {
    if (ctx->site_of[i] != site) continue;
    float ms = 0.f;
    ESM_HIP(ctx, hipEventElapsedTime(&ms, ctx->events[i].first, ctx->events[i].second));
    sum += ms;
    ++n;
  }
  *launches = n;
  *total_ms = sum;
  return ESM_GFX950_OK;
}

// ------------------------------------------------------------------ weights
extern "C" int esm_gfx950_weight_upload_i8(esm_gfx950_ctx* ctx, const int8_t* packed, const float* scales,
                                           int N, int K, esm_gfx950_weight** out) {
  if (!ctx || !out) return ESM_GFX950_INVALID_ARGUMENT;
  *out = nullptr;
  ESM_REQUIRE(ctx, packed && scales && N > 0 && K > 0, "weight_upload_i8: bad arguments");
  auto* w = new esm_gfx950_weight();
  w->N = N;
  w->K = K;
  w->ldk = pad16(K);
  std::vector<int8_t> host(static_cast<size_t>(N) * w->ldk, 0);
  for (int n = 0; n < N; ++n)
    std::memcpy(host.data() + static_cast<size_t>(n) * w->ldk, packed + static_cast<size_t>(n) * K, K);
  hipError_t e = hipMalloc(&w->data, host.size());
  if (e == hipSuccess) e = hipMalloc(&w->scales, static_cast<size_t>(N) * sizeof(float));
  if (e == hipSuccess)
    e = hipMemcpyAsync(w->data, host.data(), host.size(), hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(w->scales, scales, static_cast<size_t>(N) * sizeof(float), hipMemcpyHostToDevice,
                       ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    if (w->data) hipFree(w->data);
    if (w->scales) hipFree(w->scales);
    delete w;
    return ctx->hip_fail("weight_upload_i8", e);
  }
  *out = w;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_weight_free(esm_gfx950_ctx* ctx, esm_gfx950_weight* w) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  if (!w) return ESM_GFX950_OK;
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  hipFree(w->data);
  hipFree(w->scales);
  delete w;
  return ESM_GFX950_OK;
}

// ------------------------------------------------------------------ INT8 ops
extern "C" int esm_gfx950_gemm_i8_i32(esm_gfx950_ctx* ctx, const int8_t* A, int lda,
                                      const esm_gfx950_weight* W, int M, int32_t* C) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, A && W && C && M >= 0, "gemm_i8_i32: bad arguments");
  ESM_REQUIRE(ctx, lda >= W->K && lda % 16 == 0, "gemm_i8_i32: lda must be >= K and a multiple of 16");
  GemmI8Args p;
  p.A = A;
  p.lda = lda;
  p.W = W->data;
  p.ldw = W->ldk;
  p.M = M;
  p.N = W->N;
  p.K = W->ldk;
  p.C_i32 = C;
  p.ldc = W->N;
  ESM_HIP(ctx, launch_gemm_i8(p, kEpiI32, ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_set_gemm_split_k(int splits) {
  return set_gemm_split_k(splits) ? ESM_GFX950_OK : ESM_GFX950_INVALID_ARGUMENT;
}

extern "C" int esm_gfx950_set_gemm_tile_rows(int rows) {
  return set_gemm_tile_rows(rows) ? ESM_GFX950_OK : ESM_GFX950_INVALID_ARGUMENT;
}

extern "C" int esm_gfx950_linear_i8_q(esm_gfx950_ctx* ctx, const int8_t* A, int lda, const float* a_scale,
                                      const esm_gfx950_weight* W, const float* bias, float* C, int M,
                                      int gelu) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, A && a_scale && W && C && M >= 0, "linear_i8_q: bad arguments");
  ESM_REQUIRE(ctx, lda >= W->K && lda % 16 == 0, "linear_i8_q: lda must be >= K and a multiple of 16");
  GemmI8Args p;
  p.A = A;
  p.lda = lda;
  p.W = W->data;
  p.ldw = W->ldk;
  p.M = M;
  p.N = W->N;
  p.K = W->ldk;
  p.C_f32 = C;
  p.ldc = W->N;
  p.a_scale = a_scale;
  p.w_scale = W->scales;
  p.bias = bias;
  ESM_HIP(ctx, launch_gemm_i8(p, gelu ? kEpiF32Gelu : kEpiF32, ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_linear_i8_gelu_quant_r24(esm_gfx950_ctx* ctx, const int8_t* A, int lda,
                                                   const float* a_scale, const esm_gfx950_weight* W, const float* bias,
                                                   int M, uint16_t* inter_hi, uint8_t* inter_lo, int8_t* q, int ldq,
                                                   float* q_scale) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, A && a_scale && W && inter_hi && inter_lo && q && q_scale && M >= 0,
              "linear_i8_gelu_quant_r24: bad arguments");
  ESM_REQUIRE(ctx, W->N % 64 == 0 && W->N <= 10240, "linear_i8_gelu_quant_r24: N must be a multiple of 64, <= 10240");
  ESM_REQUIRE(ctx, ldq >= W->N && ldq % 4 == 0, "linear_i8_gelu_quant_r24: ldq must be >= N and a multiple of 4");
  GemmI8Args p;
  p.A = A;
  p.lda = lda;
  p.W = W->data;
  p.ldw = W->ldk;
  p.M = M;
  p.N = W->N;
  p.K = W->ldk;
  p.a_scale = a_scale;
  p.w_scale = W->scales;
  p.bias = bias;
  p.C_f16 = inter_hi;
  p.C_u8 = inter_lo;
  p.ldc = W->N;
  ESM_REQUIRE(ctx, gemm_i8_pipelined_ok(p),
              "linear_i8_gelu_quant_r24: needs K % 128 == 0, lda % 16 == 0 and 16-byte aligned operands");
  if (M == 0) return ESM_GFX950_OK;
  // The forward's sequence (layer_int8): the GEMM's 24-bit epilogue, then
  // the GELU + per-row quantisation pass over the two planes.
  ESM_HIP(ctx, launch_gemm_i8(p, kEpiF32R24, ctx->stream));
  ESM_HIP(ctx, launch_gelu_quant_rows_r24(inter_hi, inter_lo, W->N, M, W->N, q, ldq, q_scale, ctx->stream));
  return ESM_GFX950_OK;
}

namespace {
int quantize_into(esm_gfx950_ctx* ctx, const float* x, int M, int K, int mode, int8_t* q, int ldq,
                  float* scales, float* absmax_slot) {
  if (mode == ESM_GFX950_ACT_PER_TOKEN) {
    ESM_HIP(ctx, launch_quant_rows(x, 0, K, M, K, q, ldq, scales, ctx->stream));
  } else if (mode == ESM_GFX950_ACT_PER_TENSOR) {
    ESM_HIP(ctx, launch_fill_f32(absmax_slot, 1, 0.0f, ctx->stream));
    ESM_HIP(ctx, launch_absmax(x, static_cast<size_t>(M) * K, absmax_slot, ctx->stream));
    ESM_HIP(ctx, launch_quant_tensor(x, K, M, K, absmax_slot, q, ldq, scales, ctx->stream));
  } else {
    return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "unknown activation quantisation mode");
  }
  return ESM_GFX950_OK;
}
}  // namespace

extern "C" int esm_gfx950_quantize_act(esm_gfx950_ctx* ctx, const float* x, int M, int K, int mode,
                                       int8_t* q, int ldq, float* scales) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, x && q && scales && M >= 0 && K > 0 && ldq >= K, "quantize_act: bad arguments");
  void* s = nullptr;
  ESM_TRY(ctx->get_scratch(256, &s));
  return quantize_into(ctx, x, M, K, mode, q, ldq, scales, static_cast<float*>(s));
}

extern "C" int esm_gfx950_gelu_quantize_act(esm_gfx950_ctx* ctx, const float* x, int M, int K, int8_t* q, int ldq,
                                            float* scales) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, x && q && scales && M >= 0 && K > 0 && ldq >= K, "gelu_quantize_act: bad arguments");
  ESM_REQUIRE(ctx, K % 4 == 0 && K <= 10240, "gelu_quantize_act: K must be a multiple of 4 and at most 10240");
  ESM_HIP(ctx, launch_gelu_quant_rows(x, K, M, K, q, ldq, scales, ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_linear_i8(esm_gfx950_ctx* ctx, const float* A, const esm_gfx950_weight* W,
                                    const float* bias, float* C, int M, int N, int K, int act_mode) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  if (M <= 0 || N <= 0 || K <= 0) {
    if (M > 0 && N > 0 && C) ESM_HIP(ctx, launch_fill_f32(C, static_cast<size_t>(M) * N, 0.0f, ctx->stream));
    return ESM_GFX950_OK;
  }
  ESM_REQUIRE(ctx, A && W && C, "linear_i8: null pointer");
  if (W->N != N || W->K != K)
    return ctx->fail(ESM_GFX950_SHAPE_MISMATCH, "linear_i8: weight shape does not match N, K");
  const int ldq = W->ldk;
  const size_t qbytes = align_up(static_cast<size_t>(M) * ldq, 256);
  const size_t sbytes = align_up(static_cast<size_t>(M) * sizeof(float), 256);
  void* s = nullptr;
  ESM_TRY(ctx->get_scratch(qbytes + sbytes + 256, &s));
  auto* q = static_cast<int8_t*>(s);
  auto* scales = reinterpret_cast<float*>(static_cast<char*>(s) + qbytes);
  auto* amax = reinterpret_cast<float*>(static_cast<char*>(s) + qbytes + sbytes);
  ESM_TRY(quantize_into(ctx, A, M, K, act_mode, q, ldq, scales, amax));
  return esm_gfx950_linear_i8_q(ctx, q, ldq, scales, W, bias, C, M, 0);
}

extern "C" int esm_gfx950_linear_i8_noalloc(esm_gfx950_ctx* ctx, const float* A, const esm_gfx950_weight* W,
                                            const float* bias, float* C, int M, int N, int K, int act_mode) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  if (M <= 0 || N <= 0 || K <= 0) {
    if (M > 0 && N > 0 && C) ESM_HIP(ctx, launch_fill_f32(C, static_cast<size_t>(M) * N, 0.0f, ctx->stream));
    return ESM_GFX950_OK;
  }
  ESM_REQUIRE(ctx, A && W && C, "linear_i8_noalloc: null pointer");
  if (W->N != N || W->K != K)
    return ctx->fail(ESM_GFX950_SHAPE_MISMATCH, "linear_i8_noalloc: weight shape does not match N, K");
  if (!ctx->noalloc_scratch) return ctx->fail(ESM_GFX950_HIP_ERROR, "linear_i8_noalloc: no device scratch");
  // Layout in the static scratch: q [M, ldq] int8, scales [M] fp32, absmax.
  const int ldq = W->ldk;
  const size_t qbytes = align_up(static_cast<size_t>(M) * ldq, 256);
  const size_t sbytes = align_up(static_cast<size_t>(M) * sizeof(float), 256);
  if (qbytes + sbytes + 256 > kNoAllocScratchBytes)
    return ctx->fail(ESM_GFX950_OUT_OF_RANGE,
                     "linear_i8_noalloc: M * pad16(K) + 4 * M = " + std::to_string(qbytes + sbytes) +
                         " bytes of quantised activations exceed its " +
                         std::to_string(kNoAllocScratchBytes >> 20) + " MiB static scratch (use esm_gfx950_linear_i8)");
  char* base = static_cast<char*>(ctx->noalloc_scratch);
  auto* q = reinterpret_cast<int8_t*>(base);
  auto* scales = reinterpret_cast<float*>(base + qbytes);
  auto* amax = reinterpret_cast<float*>(base + qbytes + sbytes);  // zeroed by quantize_into (fill kernel)
  ESM_TRY(quantize_into(ctx, A, M, K, act_mode, q, ldq, scales, amax));
  return esm_gfx950_linear_i8_q(ctx, q, ldq, scales, W, bias, C, M, 0);
}

// ------------------------------------------------------------------ fp32 ops
extern "C" int esm_gfx950_linear_f32(esm_gfx950_ctx* ctx, const float* A, const float* W, const float* bias,
                                     float* C, int M, int N, int K) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  if (M <= 0 || N <= 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, A && W && C && K >= 0, "linear_f32: bad arguments");
  GemmF32Args p;
  p.A = A;
  p.lda = K;
  p.W = W;
  p.ldw = K;
  p.bias = bias;
  p.C = C;
  p.ldc = N;
  p.M = M;
  p.N = N;
  p.K = K;
  ESM_HIP(ctx, launch_gemm_f32(p, kF32Store, ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_layernorm(esm_gfx950_ctx* ctx, const float* x, const float* gamma,
                                    const float* beta, float eps, float* out, int num_rows, int d) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, (x && gamma && beta && out) || num_rows <= 0, "layernorm: null pointer");
  ESM_HIP(ctx, launch_layernorm(const_cast<float*>(x), nullptr, gamma, beta, eps, out, num_rows, d, nullptr,
                                ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_gelu(esm_gfx950_ctx* ctx, const float* x, float* out, size_t n) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_HIP(ctx, launch_gelu(x, out, n, ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_residual_add(esm_gfx950_ctx* ctx, float* y, const float* x, size_t n) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_HIP(ctx, launch_residual_add(y, x, n, ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_scale(esm_gfx950_ctx* ctx, float* x, size_t n, float scale) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_HIP(ctx, launch_scale(x, n, scale, ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_rope_build_tables(int seq_len, int head_dim, float* cos_out, float* sin_out) {
  if (seq_len < 0 || head_dim <= 0 || (seq_len > 0 && (!cos_out || !sin_out)))
    return ESM_GFX950_INVALID_ARGUMENT;
  rope_tables(seq_len, head_dim, cos_out, sin_out);
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_attention_work_items(const int32_t* cu_seqlens, int batch_size, int num_heads, int mfma,
                                               size_t* items, size_t* capacity) {
  if (!cu_seqlens || batch_size < 1 || num_heads < 1 || !items || !capacity) return ESM_GFX950_INVALID_ARGUMENT;
  int maxL = 0;
  for (int b = 0; b < batch_size; ++b) {
    if (cu_seqlens[b + 1] < cu_seqlens[b]) return ESM_GFX950_INVALID_ARGUMENT;
    maxL = std::max(maxL, cu_seqlens[b + 1] - cu_seqlens[b]);
  }
  const int T = cu_seqlens[batch_size] - cu_seqlens[0];
  std::vector<AttnWork> work;
  try {
    build_work(cu_seqlens, batch_size, num_heads, mfma ? kAttnMfmaQTile : kAttnF32QTile, &work, mfma != 0);
  } catch (const std::exception&) {
    return ESM_GFX950_INTERNAL;
  }
  *items = work.size();
  *capacity = std::max(max_work_items(batch_size, T, maxL, num_heads, kAttnMfmaQTile),
                       max_work_items(batch_size, T, maxL, num_heads, kAttnF32QTile));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_rope_apply_varlen(esm_gfx950_ctx* ctx, float* x, const float* cos, const float* sin,
                                            const int* cu_seqlens, int batch_size, int num_heads,
                                            int head_dim) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_TRY(validate_batch(ctx, cu_seqlens, batch_size, -1));
  ESM_REQUIRE(ctx, head_dim > 0 && head_dim % 2 == 0 && num_heads > 0, "rope: bad head shape");
  const int T = cu_seqlens[batch_size];
  if (T == 0) return ESM_GFX950_OK;
  std::vector<int32_t> pos(T);
  build_pos(cu_seqlens, batch_size, pos.data());
  void* s = nullptr;
  ESM_TRY(ctx->get_scratch(static_cast<size_t>(T) * 4, &s));
  ESM_HIP(ctx, hipMemcpyAsync(s, pos.data(), static_cast<size_t>(T) * 4, hipMemcpyHostToDevice, ctx->stream));
  ESM_HIP(ctx, launch_rope_f32(x, num_heads * head_dim, static_cast<int*>(s), T, num_heads, head_dim, cos, sin,
                               head_dim, 1.0f, ctx->stream));
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ESM_GFX950_OK;
}

namespace {
// Uploads cu_seqlens and the work list into op scratch (after `reserve`
// bytes used by the caller) and returns device pointers.
int stage_attention_meta(esm_gfx950_ctx* ctx, const int* cu, int B, int H, int qtile, size_t reserve,
                         int** d_cu, AttnWork** d_work, int* nwork, bool xcd_queues) {
  std::vector<AttnWork> work;
  build_work(cu, B, H, qtile, &work, xcd_queues);
  const size_t cu_bytes = align_up(static_cast<size_t>(B + 1) * 4, 256);
  const size_t wbytes = work.size() * sizeof(AttnWork);
  void* s = nullptr;
  ESM_TRY(ctx->get_scratch(reserve + cu_bytes + wbytes + 256, &s));
  char* base = static_cast<char*>(s) + reserve;
  *d_cu = reinterpret_cast<int*>(base);
  *d_work = reinterpret_cast<AttnWork*>(base + cu_bytes);
  ESM_HIP(ctx, hipMemcpyAsync(*d_cu, cu, static_cast<size_t>(B + 1) * 4, hipMemcpyHostToDevice, ctx->stream));
  if (wbytes)
    ESM_HIP(ctx, hipMemcpyAsync(*d_work, work.data(), wbytes, hipMemcpyHostToDevice, ctx->stream));
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  *nwork = static_cast<int>(work.size());
  return ESM_GFX950_OK;
}
}  // namespace

extern "C" int esm_gfx950_attention_varlen(esm_gfx950_ctx* ctx, const float* q, const float* k, const float* v,
                                           const int* cu_seqlens, int batch_size, int num_heads, int head_dim,
                                           float* out, int precision) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_TRY(validate_batch(ctx, cu_seqlens, batch_size, -1));
  ESM_REQUIRE(ctx, num_heads > 0 && head_dim > 0, "attention_varlen: bad head shape");
  const int T = cu_seqlens[batch_size];
  if (T == 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, q && k && v && out, "attention_varlen: null pointer");
  const int ld = num_heads * head_dim;
  if (precision == ESM_GFX950_ATTN_FP32) {
    ESM_REQUIRE(ctx, head_dim <= 128, "attention_varlen: fp32 path supports head_dim <= 128");
    int* d_cu;
    AttnWork* d_work;
    int nwork;
    ESM_TRY(stage_attention_meta(ctx, cu_seqlens, batch_size, num_heads, kAttnF32QTile, 0, &d_cu, &d_work, &nwork,
                                 false));
    ESM_HIP(ctx, launch_attention_f32(q, k, v, ld, head_dim, d_cu, d_work, nwork, out, ld, ctx->stream));
    ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return ESM_GFX950_OK;
  }
  if (precision != ESM_GFX950_ATTN_BF16_MFMA && precision != ESM_GFX950_ATTN_F16X3_MFMA)
    return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "attention_varlen: unknown precision");
  ESM_REQUIRE(ctx, head_dim == kHeadDimMfma, "attention_varlen: the MFMA path needs head_dim == 64");
  if (precision == ESM_GFX950_ATTN_F16X3_MFMA) {
    // Pack the fp32 operands into split-fp16 words (Q times kQPrescale), then
    // run the split-fp16 kernel.
    const size_t n = static_cast<size_t>(T) * ld;
    const size_t wbytes = align_up(n * 4, 256);
    int* d_cu;
    AttnWork* d_work;
    int nwork;
    ESM_TRY(stage_attention_meta(ctx, cu_seqlens, batch_size, num_heads, kAttnMfmaQTile, 3 * wbytes, &d_cu, &d_work,
                                 &nwork, true));
    char* base = static_cast<char*>(ctx->scratch);
    auto* qw = reinterpret_cast<uint32_t*>(base);
    auto* kp = reinterpret_cast<uint16_t*>(base + wbytes);      // [T, 2 ld]: hi | lo
    auto* vp = reinterpret_cast<uint16_t*>(base + 2 * wbytes);
    ESM_HIP(ctx, launch_pack_x3(q, ld, T, ld, kQPrescale, qw, nullptr, ld, ctx->stream));
    ESM_HIP(ctx, launch_pack_x3(k, ld, T, ld, 1.0f, nullptr, kp, 2 * ld, ctx->stream));
    ESM_HIP(ctx, launch_pack_x3(v, ld, T, ld, 1.0f, nullptr, vp, 2 * ld, ctx->stream));
    int max_len = 0;
    for (int b = 0; b < batch_size; ++b) max_len = std::max(max_len, cu_seqlens[b + 1] - cu_seqlens[b]);
    int slot;
    ESM_TRY(ctx->time_begin("attention", &slot));
    ESM_HIP(ctx, launch_attention_x3(qw, ld, kp, kp + ld, vp, vp + ld, 2 * ld, kQPrescale, d_cu, d_work, nwork, out,
                                     ld, max_len, ctx->stream));
    ESM_TRY(ctx->time_end(slot));
    ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return ESM_GFX950_OK;
  }
  const size_t n = static_cast<size_t>(T) * ld;
  const size_t cbytes = align_up(n * 2, 256);
  int* d_cu;
  AttnWork* d_work;
  int nwork;
  ESM_TRY(stage_attention_meta(ctx, cu_seqlens, batch_size, num_heads, kAttnMfmaQTile, 3 * cbytes, &d_cu, &d_work,
                               &nwork, true));
  char* base = static_cast<char*>(ctx->scratch);
  auto* qb = reinterpret_cast<uint16_t*>(base);
  auto* kb = reinterpret_cast<uint16_t*>(base + cbytes);
  auto* vb = reinterpret_cast<uint16_t*>(base + 2 * cbytes);
  ESM_HIP(ctx, launch_cast_f32(q, n, qb, 1, ctx->stream));
  ESM_HIP(ctx, launch_cast_f32(k, n, kb, 1, ctx->stream));
  ESM_HIP(ctx, launch_cast_f32(v, n, vb, 0, ctx->stream));
  ESM_HIP(ctx, launch_attention_mfma(qb, kb, vb, 0, 0, ld, d_cu, d_work, nwork, out, ld, nullptr, ctx->stream));
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_attention_varlen_bf16(esm_gfx950_ctx* ctx, const uint16_t* q, const uint16_t* k,
                                                const uint16_t* v, int v_is_fp16, const int* cu_seqlens,
                                                int batch_size, int num_heads, float* out) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_TRY(validate_batch(ctx, cu_seqlens, batch_size, -1));
  ESM_REQUIRE(ctx, num_heads > 0, "attention_varlen_bf16: bad head count");
  const int T = cu_seqlens[batch_size];
  if (T == 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, q && k && v && out, "attention_varlen_bf16: null pointer");
  int* d_cu;
  AttnWork* d_work;
  int nwork;
  ESM_TRY(
      stage_attention_meta(ctx, cu_seqlens, batch_size, num_heads, kAttnMfmaQTile, 0, &d_cu, &d_work, &nwork, true));
  const int ld = num_heads * kHeadDimMfma;
  int slot;
  ESM_TRY(ctx->time_begin("attention", &slot));
  ESM_HIP(ctx, launch_attention_mfma(q, k, v, 0, v_is_fp16 ? 0 : 1, ld, d_cu, d_work, nwork, out, ld, nullptr,
                                     ctx->stream));
  ESM_TRY(ctx->time_end(slot));
  return ESM_GFX950_OK;
}

// ------------------------------------------------- the reference's x86 kernels
extern "C" int esm_gfx950_layernorm_avx512(esm_gfx950_ctx* ctx, const float* x, const float* gamma, const float* beta,
                                           float eps, float* out, int num_rows, int d) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  if (num_rows <= 0 || d <= 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, x && gamma && beta && out, "layernorm_avx512: null pointer");
  ESM_REQUIRE(ctx, d <= 2560, "layernorm_avx512: d must be <= 2560");
  ESM_HIP(ctx, launch_layernorm_x86(const_cast<float*>(x), nullptr, gamma, beta, eps, out, num_rows, d, nullptr, 0,
                                    ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_gelu_avx512(esm_gfx950_ctx* ctx, const float* x, float* out, size_t n) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, n == 0 || (x && out), "gelu_avx512: null pointer");
  ESM_HIP(ctx, launch_gelu_x86(x, out, n, nullptr, ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_expf_glibc(esm_gfx950_ctx* ctx, const float* x, float* out, size_t n) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, n == 0 || (x && out), "expf_glibc: null pointer");
  ESM_HIP(ctx, launch_expf_glibc(x, out, n, ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_linear_f32_avx512(esm_gfx950_ctx* ctx, const float* A, const float* W, const float* bias,
                                            float* C, int M, int N, int K) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  if (M <= 0 || N <= 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, A && W && C && K >= 0, "linear_f32_avx512: bad arguments");
  ESM_HIP(ctx, launch_linear_x86(A, K, W, K, bias, C, N, M, N, K, kF32Store, ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_rope_apply_varlen_avx512(esm_gfx950_ctx* ctx, float* x, const float* cos, const float* sin,
                                                   const int* cu_seqlens, int batch_size, int num_heads,
                                                   int head_dim) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_TRY(validate_batch(ctx, cu_seqlens, batch_size, -1));
  ESM_REQUIRE(ctx, head_dim > 0 && head_dim % 2 == 0 && num_heads > 0, "rope_avx512: bad head shape");
  const int T = cu_seqlens[batch_size];
  if (T == 0) return ESM_GFX950_OK;
  std::vector<int32_t> pos(T);
  build_pos(cu_seqlens, batch_size, pos.data());
  void* sp = nullptr;
  ESM_TRY(ctx->get_scratch(static_cast<size_t>(T) * 4, &sp));
  ESM_HIP(ctx, hipMemcpyAsync(sp, pos.data(), static_cast<size_t>(T) * 4, hipMemcpyHostToDevice, ctx->stream));
  ESM_HIP(ctx, launch_rope_x86(x, num_heads * head_dim, static_cast<int*>(sp), T, num_heads, head_dim, cos, sin,
                               head_dim, 1.0f, ctx->stream));
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_attention_varlen_avx512(esm_gfx950_ctx* ctx, const float* q, const float* k, const float* v,
                                                  const int* cu_seqlens, int batch_size, int num_heads, int head_dim,
                                                  float* out) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_TRY(validate_batch(ctx, cu_seqlens, batch_size, -1));
  ESM_REQUIRE(ctx, num_heads > 0 && attention_x86_supported(head_dim),
              "attention_varlen_avx512: head_dim must be 16, 32 or 64");
  const int T = cu_seqlens[batch_size];
  if (T == 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, q && k && v && out, "attention_varlen_avx512: null pointer");
  // The forward's form of the kernel: a work list of 64-query items,
  // longest sequences first, and the score cache (when its per-head offsets
  // fit 32 bits). Scratch: cu, the work list, the scores.
  int maxL = 0;
  for (int b = 0; b < batch_size; ++b) maxL = std::max(maxL, cu_seqlens[b + 1] - cu_seqlens[b]);
  std::vector<AttnWork> work;
  build_work(cu_seqlens, batch_size, num_heads, kAttnF32QTile, &work);
  const size_t cu_bytes = (static_cast<size_t>(batch_size + 1) * 4 + 15) & ~static_cast<size_t>(15);
  const size_t work_bytes = (work.size() * sizeof(AttnWork) + 255) & ~static_cast<size_t>(255);
  const size_t n_scores = attention_x86_score_floats(cu_seqlens, batch_size, num_heads);
  const bool cache = n_scores / static_cast<size_t>(num_heads) < (static_cast<size_t>(1) << 32);
  void* sp = nullptr;
  ESM_TRY(ctx->get_scratch(cu_bytes + work_bytes + (cache ? n_scores * 4 : 0), &sp));
  char* base = static_cast<char*>(sp);
  ESM_HIP(ctx, hipMemcpyAsync(base, cu_seqlens, static_cast<size_t>(batch_size + 1) * 4, hipMemcpyHostToDevice,
                              ctx->stream));
  ESM_HIP(ctx, hipMemcpyAsync(base + cu_bytes, work.data(), work.size() * sizeof(AttnWork), hipMemcpyHostToDevice,
                              ctx->stream));
  const int ld = num_heads * head_dim;
  ESM_HIP(ctx, launch_attention_x86(q, k, v, ld, head_dim, reinterpret_cast<int*>(base), batch_size, num_heads, maxL,
                                    out, ld, ctx->stream,
                                    cache ? reinterpret_cast<float*>(base + cu_bytes + work_bytes) : nullptr,
                                    reinterpret_cast<AttnWork*>(base + cu_bytes), static_cast<int>(work.size())));
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ESM_GFX950_OK;
}

// -------------------------------------------------------------------- model
namespace {

struct DevLinear {
  // int8 weights
  int8_t* w8 = nullptr;
  float* ws = nullptr;
  // fp32 weights
  float* w32 = nullptr;
  float* bias = nullptr;
  int N = 0, K = 0, ldk = 0;
};

struct DevLayer {
  float *ln1_w = nullptr, *ln1_b = nullptr, *ln2_w = nullptr, *ln2_b = nullptr;
  DevLinear qkv, out, fc1, fc2;
};

}  // namespace

struct esm_gfx950_model {
  esm_gfx950_model_config cfg{};
  std::vector<void*> allocations;  // every weight allocation
  float* embed = nullptr;
  std::vector<DevLayer> layers;
  float *final_ln_w = nullptr, *final_ln_b = nullptr;
  float *lm_dense_w = nullptr, *lm_dense_b = nullptr;
  // lm head dense weight as split-fp16 planes of W * 2^shift (null when
  // d % 32 != 0) and whether the forward uses them (split-fp16 GEMM) or the
  // fp32 weight (fp32 MFMA).
  uint16_t *lm_w_hi = nullptr, *lm_w_lo = nullptr;
  float lm_w_unscale = 1.0f;
  bool lm_dense_split = false;
  float *lm_ln_w = nullptr, *lm_ln_b = nullptr;
  float* dec_bias = nullptr;
  // W8A8 models: Q's 1/sqrt(head_dim) multiplied into the Q weight scales and
  // bias at upload (exact when it is a power of two).
  bool q_scale_folded = false;
  // Layer 0's fc1 input rounded to fp16 (reference Config::first_block_fc1_fp16,
  // include/esm_cpp/model.h:36-41; applied at src/model.cpp:1028-1033).
  bool first_block_fc1_fp16 = false;
  // ESM_GFX950_NUMERICS_X86_AVX512: the forward reproduces the reference's
  // x86 AVX-512 kernels bit for bit (per-tensor activation scales);
  // ESM_GFX950_NUMERICS_X86_AMX: the same with LinearAmx's row split.
  int numerics = ESM_GFX950_NUMERICS_DEFAULT;
  // A staged batch is split into `parts` contiguous sequence groups; each
  // part has its own arena and metadata. Part 0 runs on the context stream,
  // every other part on a HIP stream of its own, so the parts' kernels can
  // occupy different CUs at the same time. Part p's tokens are rows
  // [t0, t0 + T) of the packed batch.
  struct Part {
    void* arena = nullptr;  // grown when the part exceeds every earlier batch
    size_t arena_bytes = 0;
    int cap_T = 0, cap_B = 0, cap_L = 0;
    void* meta_host = nullptr;  // pinned staging of the per-batch metadata
    void* meta_dev = nullptr;
    size_t meta_bytes = 0;
    hipEvent_t meta_done = nullptr;  // the part's metadata copy has consumed meta_host
    hipEvent_t done = nullptr;       // the part's forward has finished (join)
    hipStream_t stream = nullptr;    // null: the context stream
    int rope_len = 0;                // rows currently in the device rope tables
    int T = 0, B = 0, nwork = 0, t0 = 0;
    int maxL = 0;                    // longest sequence of the staged part
    size_t x86_score_floats = 0;     // attention_x86_score_floats of the staged part
  };
  std::vector<Part> parts = std::vector<Part>(1);
  // Automatic group count (esm_gfx950_model_set_parts(0), the default): each
  // staged batch takes as many of the parts as its size warrants.
  bool auto_parts = true;
  // Per-token W8A8: fc1's output goes to the GELU + quant pass as 24-bit
  // values (esm_gfx950_model_set_ffn_intermediate_bits(24), the default) or
  // as fp32 (32).
  bool ffn_r24 = true;
  int staged_T = 0;  // tokens of the staged batch (all parts)
  // esm_gfx950_forward_scheduled: device and pinned host logits, two of each
  // so one group's copy-out overlaps the next group's forward.
  float* sched_dev[2] = {nullptr, nullptr};
  float* sched_host[2] = {nullptr, nullptr};
  hipEvent_t sched_copied[2] = {nullptr, nullptr};
  size_t sched_cap = 0;  // floats per buffer
};

namespace {

int upload(esm_gfx950_ctx* ctx, esm_gfx950_model* m, const void* src, size_t bytes, void** dst) {
  *dst = nullptr;
  if (!src) return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "model_create: null weight pointer");
  ESM_HIP(ctx, hipMalloc(dst, bytes));
  m->allocations.push_back(*dst);
  ESM_HIP(ctx, hipMemcpyAsync(*dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ESM_GFX950_OK;
}

template <typename T>
int upload_f(esm_gfx950_ctx* ctx, esm_gfx950_model* m, const T* src, size_t n, T** dst) {
  void* p = nullptr;
  int rc = upload(ctx, m, src, n * sizeof(T), &p);
  *dst = static_cast<T*>(p);
  return rc;
}

// Concatenates the given linears along N into one device weight.
// part0_scale multiplies part 0's per-channel scales and bias (int8 only).
// W [N, K] fp32 as the two fp16 planes of the split-fp16 GEMM: hi = fp16(x),
// lo = fp16(x - hi) of x = W * 2^shift, with the shift putting max|W| in
// [2^13, 2^14) so that the lo parts of small weights stay normal fp16.
int upload_split(esm_gfx950_ctx* ctx, esm_gfx950_model* m, const float* w, int N, int K) {
  const size_t n = static_cast<size_t>(N) * K;
  float amax = 0.0f;
  for (size_t i = 0; i < n; ++i) amax = std::max(amax, std::fabs(w[i]));
  int shift = 0;
  if (amax > 0.0f && std::isfinite(amax)) {
    int e = 0;
    std::frexp(amax, &e);  // amax in [2^(e-1), 2^e)
    shift = std::min(100, std::max(-100, 14 - e));
  }
  std::vector<uint16_t> hi(n), lo(n);
  for (size_t i = 0; i < n; ++i) {
    const float x = std::ldexp(w[i], shift);
    const _Float16 h = static_cast<_Float16>(x);
    const _Float16 l = static_cast<_Float16>(x - static_cast<float>(h));
    hi[i] = __builtin_bit_cast(uint16_t, h);
    lo[i] = __builtin_bit_cast(uint16_t, l);
  }
  ESM_TRY(upload_f(ctx, m, hi.data(), n, &m->lm_w_hi));
  ESM_TRY(upload_f(ctx, m, lo.data(), n, &m->lm_w_lo));
  m->lm_w_unscale = std::ldexp(1.0f, -shift);
  return ESM_GFX950_OK;
}

int upload_linear(esm_gfx950_ctx* ctx, esm_gfx950_model* m, const esm_gfx950_linear_desc* const* parts,
                  int nparts, int N_each, int K, bool int8, DevLinear* out, float part0_scale = 1.0f) {
  const int N = N_each * nparts;
  out->N = N;
  out->K = K;
  out->ldk = int8 ? pad16(K) : K;
  std::vector<float> bias(static_cast<size_t>(N));
  for (int p = 0; p < nparts; ++p) {
    if (!parts[p]->bias) return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "model_create: null bias");
    std::memcpy(bias.data() + static_cast<size_t>(p) * N_each, parts[p]->bias, N_each * sizeof(float));
  }
  if (int8 && part0_scale != 1.0f)
    for (int n = 0; n < N_each; ++n) bias[n] *= part0_scale;
  ESM_TRY(upload_f(ctx, m, bias.data(), bias.size(), &out->bias));
  if (int8) {
    std::vector<int8_t> w(static_cast<size_t>(N) * out->ldk, 0);
    std::vector<float> s(static_cast<size_t>(N));
    for (int p = 0; p < nparts; ++p) {
      if (!parts[p]->w_i8 || !parts[p]->w_scale)
        return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "model_create: null int8 weight");
      for (int n = 0; n < N_each; ++n)
        std::memcpy(w.data() + static_cast<size_t>(p * N_each + n) * out->ldk,
                    parts[p]->w_i8 + static_cast<size_t>(n) * K, K);
      std::memcpy(s.data() + static_cast<size_t>(p) * N_each, parts[p]->w_scale, N_each * sizeof(float));
    }
    if (part0_scale != 1.0f)
      for (int n = 0; n < N_each; ++n) s[n] *= part0_scale;
    ESM_TRY(upload_f(ctx, m, w.data(), w.size(), &out->w8));
    ESM_TRY(upload_f(ctx, m, s.data(), s.size(), &out->ws));
  } else {
    std::vector<float> w(static_cast<size_t>(N) * K);
    for (int p = 0; p < nparts; ++p) {
      if (!parts[p]->w_f32) return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "model_create: null fp32 weight");
      std::memcpy(w.data() + static_cast<size_t>(p) * N_each * K, parts[p]->w_f32,
                  static_cast<size_t>(N_each) * K * sizeof(float));
    }
    ESM_TRY(upload_f(ctx, m, w.data(), w.size(), &out->w32));
  }
  return ESM_GFX950_OK;
}

void free_part(esm_gfx950_model::Part& p) {
  if (p.arena) hipFree(p.arena);
  if (p.meta_dev) hipFree(p.meta_dev);
  if (p.meta_host) hipHostFree(p.meta_host);
  if (p.meta_done) hipEventDestroy(p.meta_done);
  if (p.done) hipEventDestroy(p.done);
  if (p.stream) hipStreamDestroy(p.stream);
  p = esm_gfx950_model::Part();
}

void free_model(esm_gfx950_model* m) {
  for (void* p : m->allocations) hipFree(p);
  for (auto& p : m->parts) free_part(p);
  for (int i = 0; i < 2; ++i) {
    if (m->sched_dev[i]) hipFree(m->sched_dev[i]);
    if (m->sched_host[i]) hipHostFree(m->sched_host[i]);
    if (m->sched_copied[i]) hipEventDestroy(m->sched_copied[i]);
  }
  delete m;
}

// Events (and, for multi-part models, a stream) of one part.
int init_part(esm_gfx950_ctx* ctx, esm_gfx950_model::Part& p, bool own_stream) {
  ESM_HIP(ctx, hipEventCreateWithFlags(&p.meta_done, hipEventDisableTiming));
  ESM_HIP(ctx, hipEventCreateWithFlags(&p.done, hipEventDisableTiming));
  if (own_stream) ESM_HIP(ctx, hipStreamCreate(&p.stream));
  return ESM_GFX950_OK;
}

}  // namespace

extern "C" int esm_gfx950_model_create(esm_gfx950_ctx* ctx, const esm_gfx950_model_desc* desc,
                                       esm_gfx950_model** out) {
  if (!ctx || !desc || !out) return ESM_GFX950_INVALID_ARGUMENT;
  *out = nullptr;
  const auto& c = desc->cfg;
  ESM_REQUIRE(ctx, c.num_layers >= 0 && c.hidden_size > 0 && c.num_heads > 0 && c.head_dim > 0 &&
                       c.num_heads * c.head_dim == c.hidden_size && c.intermediate_size > 0 && c.vocab_size > 0,
              "model_create: inconsistent config");
  ESM_REQUIRE(ctx, c.head_dim % 2 == 0 && c.head_dim <= 128, "model_create: head_dim must be even and <= 128");
  ESM_REQUIRE(ctx, c.act_quant_mode == ESM_GFX950_ACT_PER_TENSOR || c.act_quant_mode == ESM_GFX950_ACT_PER_TOKEN,
              "model_create: unknown act_quant_mode");
  ESM_REQUIRE(ctx, c.attention_mode >= ESM_GFX950_ATTN_MODE_FP16 && c.attention_mode <= ESM_GFX950_ATTN_MODE_F16X3,
              "model_create: unknown attention_mode");
  if (c.weights_int8) {
    ESM_REQUIRE(ctx, c.hidden_size % 16 == 0 && c.intermediate_size % 16 == 0,
                "model_create: W8A8 needs hidden and intermediate sizes divisible by 16");
    ESM_REQUIRE(ctx, (c.attention_mode == ESM_GFX950_ATTN_MODE_FP32) || c.head_dim == kHeadDimMfma,
                "model_create: MFMA attention needs head_dim 64 (use ESM_GFX950_ATTN_MODE_FP32)");
    ESM_REQUIRE(ctx, c.hidden_size % 4 == 0 && c.hidden_size <= 2560,
                "model_create: fused LayerNorm+quant supports hidden_size % 4 == 0 and <= 2560");
    // The split-fp16 QKV epilogue exists only in the pipelined GEMM, which
    // needs K = hidden_size to be a multiple of 128.
    ESM_REQUIRE(ctx, c.attention_mode != ESM_GFX950_ATTN_MODE_F16X3 || c.hidden_size % 128 == 0,
                "model_create: ESM_GFX950_ATTN_MODE_F16X3 needs hidden_size % 128 == 0 (use another attention_mode)");
    ESM_REQUIRE(ctx, c.act_quant_mode != ESM_GFX950_ACT_PER_TOKEN || c.intermediate_size <= 10240,
                "model_create: per-token activation scales support intermediate_size <= 10240");
  }
  ESM_REQUIRE(ctx, desc->layers || c.num_layers == 0, "model_create: null layers");
  auto* m = new esm_gfx950_model();
  m->cfg = c;
  const int d = c.hidden_size, f = c.intermediate_size, V = c.vocab_size;
  const bool i8 = c.weights_int8 != 0;
  // ScaleInplace(q, 1/sqrt(dh)) after the Q projection (reference
  // src/model.cpp:975-979) commutes exactly with the dequant fma when the
  // factor is a power of two: fma(acc, a*(w*f), b*f) == fma(acc, a*w, b)*f.
  const float q_scale = 1.0f / std::sqrt(static_cast<float>(c.head_dim));
  int q_exp = 0;
  const bool pow2 = std::frexp(q_scale, &q_exp) == 0.5f;
  const float q_fold = (i8 && pow2) ? q_scale : 1.0f;
  m->q_scale_folded = i8 && pow2;
  int rc = ESM_GFX950_OK;
  auto step = [&](int r) {
    if (rc == ESM_GFX950_OK) rc = r;
    return rc == ESM_GFX950_OK;
  };
  step(upload_f(ctx, m, desc->embed, static_cast<size_t>(V) * d, &m->embed));
  m->layers.resize(c.num_layers);
  for (int i = 0; i < c.num_layers && rc == ESM_GFX950_OK; ++i) {
    const auto& L = desc->layers[i];
    DevLayer& D = m->layers[i];
    step(upload_f(ctx, m, L.attn_ln_w, d, &D.ln1_w));
    step(upload_f(ctx, m, L.attn_ln_b, d, &D.ln1_b));
    step(upload_f(ctx, m, L.ffn_ln_w, d, &D.ln2_w));
    step(upload_f(ctx, m, L.ffn_ln_b, d, &D.ln2_b));
    const esm_gfx950_linear_desc* qkv[3] = {&L.q, &L.k, &L.v};
    const esm_gfx950_linear_desc* o1[1] = {&L.out};
    const esm_gfx950_linear_desc* f1[1] = {&L.fc1};
    const esm_gfx950_linear_desc* f2[1] = {&L.fc2};
    if (rc == ESM_GFX950_OK) step(upload_linear(ctx, m, qkv, 3, d, d, i8, &D.qkv, q_fold));
    if (rc == ESM_GFX950_OK) step(upload_linear(ctx, m, o1, 1, d, d, i8, &D.out));
    if (rc == ESM_GFX950_OK) step(upload_linear(ctx, m, f1, 1, f, d, i8, &D.fc1));
    if (rc == ESM_GFX950_OK) step(upload_linear(ctx, m, f2, 1, d, f, i8, &D.fc2));
  }
  step(upload_f(ctx, m, desc->final_ln_w, d, &m->final_ln_w));
  step(upload_f(ctx, m, desc->final_ln_b, d, &m->final_ln_b));
  step(upload_f(ctx, m, desc->lm_dense_w, static_cast<size_t>(d) * d, &m->lm_dense_w));
  step(upload_f(ctx, m, desc->lm_dense_b, d, &m->lm_dense_b));
  if (rc == ESM_GFX950_OK && d % 32 == 0) {
    step(upload_split(ctx, m, desc->lm_dense_w, d, d));
    // W8A8 models run the dense on the split-fp16 GEMM; all-fp32 models keep
    // the fp32 MFMA kernel (esm_gfx950_model_set_lm_dense_split switches).
    m->lm_dense_split = i8;
  }
  step(upload_f(ctx, m, desc->lm_ln_w, d, &m->lm_ln_w));
  step(upload_f(ctx, m, desc->lm_ln_b, d, &m->lm_ln_b));
  step(upload_f(ctx, m, desc->lm_decoder_bias, V, &m->dec_bias));
  if (rc == ESM_GFX950_OK) {
    // The automatic group count (the default) can use up to kAutoMaxParts.
    m->parts.assign(kAutoMaxParts, esm_gfx950_model::Part());
    for (int i = 0; i < kAutoMaxParts; ++i) step(init_part(ctx, m->parts[i], i > 0));
  }
  if (rc != ESM_GFX950_OK) {
    hipStreamSynchronize(ctx->stream);
    free_model(m);
    return rc;
  }
  *out = m;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_model_free(esm_gfx950_ctx* ctx, esm_gfx950_model* model) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  if (!model) return ESM_GFX950_OK;
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  free_model(model);
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_model_set_act_mode(esm_gfx950_ctx* ctx, esm_gfx950_model* model, int act_mode) {
  if (!ctx || !model) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, act_mode == ESM_GFX950_ACT_PER_TENSOR || act_mode == ESM_GFX950_ACT_PER_TOKEN,
              "model_set_act_mode: unknown mode");
  ESM_REQUIRE(ctx, act_mode != ESM_GFX950_ACT_PER_TOKEN || !model->cfg.weights_int8 ||
                       model->cfg.intermediate_size <= 10240,
              "model_set_act_mode: per-token activation scales support intermediate_size <= 10240");
  model->cfg.act_quant_mode = act_mode;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_model_set_first_block_fc1_fp16(esm_gfx950_ctx* ctx, esm_gfx950_model* model, int enabled) {
  if (!ctx || !model) return ESM_GFX950_INVALID_ARGUMENT;
  model->first_block_fc1_fp16 = enabled != 0;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_model_set_ffn_intermediate_bits(esm_gfx950_ctx* ctx, esm_gfx950_model* model, int bits) {
  if (!ctx || !model) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, bits == 24 || bits == 32, "model_set_ffn_intermediate_bits: bits must be 24 or 32");
  model->ffn_r24 = bits == 24;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_model_set_numerics(esm_gfx950_ctx* ctx, esm_gfx950_model* model, int numerics) {
  if (!ctx || !model) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx,
              numerics == ESM_GFX950_NUMERICS_DEFAULT || numerics == ESM_GFX950_NUMERICS_X86_AVX512 ||
                  numerics == ESM_GFX950_NUMERICS_X86_AMX,
              "model_set_numerics: unknown numerics");
  const auto& c = model->cfg;
  if (numerics != ESM_GFX950_NUMERICS_DEFAULT) {
    ESM_REQUIRE(ctx, attention_x86_supported(c.head_dim),
                "model_set_numerics: the x86 attention supports head_dim 16, 32 and 64");
    ESM_REQUIRE(ctx, c.hidden_size <= 2560, "model_set_numerics: the x86 LayerNorm supports hidden_size <= 2560");
  }
  if (model->numerics == numerics) return ESM_GFX950_OK;
  // The arena layout depends on the numerics (fp32 Q|K|V rows): drop the
  // staged batch and its buffers; the next upload sizes them again.
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  for (auto& p : model->parts) {
    if (p.stream) ESM_HIP(ctx, hipStreamSynchronize(p.stream));
    if (p.arena) hipFree(p.arena);
    p.arena = nullptr;
    p.arena_bytes = 0;
    p.cap_T = 0;
    p.T = 0;
  }
  model->staged_T = 0;
  model->numerics = numerics;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_model_set_lm_dense_split(esm_gfx950_ctx* ctx, esm_gfx950_model* model, int enabled) {
  if (!ctx || !model) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, !enabled || model->lm_w_hi, "model_set_lm_dense_split: hidden size is not a multiple of 32");
  model->lm_dense_split = enabled != 0;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_model_arena_bytes(const esm_gfx950_model* model, size_t* bytes) {
  if (!model || !bytes) return ESM_GFX950_INVALID_ARGUMENT;
  size_t b = 0;
  for (const auto& p : model->parts) b += p.arena_bytes + p.meta_bytes;
  *bytes = b;
  return ESM_GFX950_OK;
}

namespace {

// Arena layout for T tokens (every region 256-byte aligned).
struct Arena {
  float* hidden;     // [T, d]
  float* ln;         // [T, d]   fp32 LN output / final LN
  int8_t* xq;        // [T, max(d, ffn) padded]
  float* xs;         // [T] activation scales
  uint16_t* qb;      // [T, d] bf16 Q
  uint16_t* kb;      // [T, d] bf16 K
  uint16_t* vb;      // [T, d] fp16 V
  float* qkv;        // [T, 3d] fp32 (fp32 paths)
  float* attn;       // [T, d]
  float* ybuf;       // [T, d] out-proj / fc2 output awaiting its residual add
  float* inter;      // [T, ffn]
  float* lm_a;       // [T, d]
  float* logits;     // [T, V]
  float* absmax;     // scratch scalars
  size_t bytes;
};

// Attention modes whose Q/K/V live in the fp32 [T, 3d] buffer.
bool qkv_is_f32(const esm_gfx950_model_config& c) {
  return c.attention_mode == ESM_GFX950_ATTN_MODE_FP32 || c.attention_mode == ESM_GFX950_ATTN_MODE_F16X3;
}

Arena layout(const esm_gfx950_model_config& c, int T, char* base, bool x86 = false) {
  const size_t d = c.hidden_size, f = c.intermediate_size, V = c.vocab_size;
  const size_t Ts = static_cast<size_t>(T);
  const size_t wq = std::max<size_t>(pad16(c.hidden_size), pad16(c.intermediate_size));
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align_up(bytes, 256);
    return p;
  };
  Arena a;
  a.hidden = reinterpret_cast<float*>(take(Ts * d * 4));
  a.ln = reinterpret_cast<float*>(take(Ts * d * 4));
  a.xq = reinterpret_cast<int8_t*>(take(Ts * wq));
  a.xs = reinterpret_cast<float*>(take(Ts * 4));
  a.qb = reinterpret_cast<uint16_t*>(take(Ts * d * 2));
  a.kb = reinterpret_cast<uint16_t*>(take(Ts * d * 2));
  a.vb = reinterpret_cast<uint16_t*>(take(Ts * d * 2));
  const bool need_qkv_f32 = !c.weights_int8 || qkv_is_f32(c) || x86;
  a.qkv = reinterpret_cast<float*>(take(need_qkv_f32 ? Ts * 3 * d * 4 : 0));
  a.attn = reinterpret_cast<float*>(take(Ts * d * 4));
  a.ybuf = reinterpret_cast<float*>(take(c.weights_int8 ? Ts * d * 4 : 0));
  a.inter = reinterpret_cast<float*>(take(Ts * f * 4));
  a.lm_a = reinterpret_cast<float*>(take(Ts * d * 4));
  a.logits = reinterpret_cast<float*>(take(Ts * V * 4));
  a.absmax = reinterpret_cast<float*>(take(256));
  a.bytes = off;
  return a;
}

struct Meta {
  int32_t* ids;
  float* tok_scale;
  int32_t* pos;
  int32_t* cu;
  AttnWork* work;
  size_t work_cap;  // work items the region holds
  float* cos_t;
  float* sin_t;
  size_t bytes;
};

Meta meta_layout(int T, int B, int maxL, int H, int dh, char* base) {
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align_up(bytes, 256);
    return p;
  };
  Meta m;
  m.ids = reinterpret_cast<int32_t*>(take(static_cast<size_t>(T) * 4));
  m.tok_scale = reinterpret_cast<float*>(take(static_cast<size_t>(T) * 4));
  m.pos = reinterpret_cast<int32_t*>(take(static_cast<size_t>(T) * 4));
  m.cu = reinterpret_cast<int32_t*>(take(static_cast<size_t>(B + 1) * 4));
  m.work_cap = std::max(max_work_items(B, T, maxL, H, kAttnMfmaQTile), max_work_items(B, T, maxL, H, kAttnF32QTile));
  m.work = reinterpret_cast<AttnWork*>(take(m.work_cap * sizeof(AttnWork)));
  m.cos_t = reinterpret_cast<float*>(take(static_cast<size_t>(maxL) * dh * 4));
  m.sin_t = reinterpret_cast<float*>(take(static_cast<size_t>(maxL) * dh * 4));
  m.bytes = off;
  return m;
}

// The arena of one staged part (its layout depends on the model's numerics).
Arena part_arena(const esm_gfx950_model* m, const esm_gfx950_model::Part& P) {
  return layout(m->cfg, P.cap_T, static_cast<char*>(P.arena), m->numerics != ESM_GFX950_NUMERICS_DEFAULT);
}

template <typename P>
P shift(P p, const char* from, const char* to) {
  return reinterpret_cast<P>(const_cast<char*>(to) + (reinterpret_cast<const char*>(p) - from));
}

// Capture state of one esm_gfx950_forward_with_observer call. The sites are
// known before the forward starts (four per layer, reference
// src/model.cpp:952-955,996-999,1023-1026,1047-1050), and Algorithm R's
// decisions need only each site's value count, so host threads plan every
// site's reservoir slots while the device runs; capture() waits for its
// site's plan, then copies the positions to the device and gathers the
// values behind the kernel that produced them. finish() copies the gathered
// values back and stores them in the reservoirs.
struct ObsSite {
  obs::Reservoir* r = nullptr;
  size_t n = 0;
  std::vector<uint32_t> slots;
  size_t count = 0;
};

class ObsRun {
 public:
  ObsRun(esm_gfx950_observer* o, std::vector<ObsSite> sites) : obs_(o), sites_(std::move(sites)) {
    done_.assign(sites_.size(), 0);
    // Test hook for the failure path: ESM_GFX950_TEST_OBSERVER_FAIL_SITE=k
    // makes the capture of site k (0-based, forward order) fail on the host
    // after the kernels before it have been enqueued.
    if (const char* e = std::getenv("ESM_GFX950_TEST_OBSERVER_FAIL_SITE")) fail_site_ = std::strtol(e, nullptr, 10);
    size_t workers = std::thread::hardware_concurrency();
    if (const char* e = std::getenv("ESM_NUM_THREADS")) workers = std::strtoul(e, nullptr, 10);
    workers = std::max<size_t>(1, std::min<size_t>({workers, 16, sites_.size()}));
    // Workers take sites in forward order from a shared counter.
    for (size_t w = 0; w < workers; ++w) {
      try {
        threads_.emplace_back([this] { work(); });
      } catch (...) {
        break;
      }
    }
    if (threads_.empty()) work();
  }
  ~ObsRun() { join(); }
  void join() {
    for (auto& t : threads_)
      if (t.joinable()) t.join();
  }
  void work() {
    for (;;) {
      size_t k;
      {
        std::lock_guard<std::mutex> lk(mu_);
        if (taken_ == sites_.size()) return;
        k = taken_++;
      }
      ObsSite& st = sites_[k];
      int ok = 1;
      try {
        st.slots.resize(obs::kReservoirSize);
        st.count = obs::plan(*st.r, st.n, st.slots.data(), obs_->h_pos + k * obs::kReservoirSize);
      } catch (...) {
        ok = -1;
      }
      {
        std::lock_guard<std::mutex> lk(mu_);
        done_[k] = ok;
      }
      cv_.notify_all();
    }
  }

  // The next site's values: x [n] fp32 on the device (gelu: GELU applied on
  // the fly, for the per-token path whose fc1 output is stored pre-GELU).
  // r24_lo != null: x is kEpiF32R24's high plane (uint16) and r24_lo its low
  // plane, rows of r24_cols values, GELU applied.
  int capture(esm_gfx950_ctx* ctx, const void* x, size_t n, int gelu, const uint8_t* r24_lo = nullptr,
              int r24_cols = 0) {
    if (next_ >= sites_.size() || sites_[next_].n != n)
      return ctx->fail(ESM_GFX950_INTERNAL, "forward_with_observer: site sequence mismatch");
    if (fail_site_ >= 0 && static_cast<size_t>(fail_site_) == next_)
      return ctx->fail(ESM_GFX950_INTERNAL, "forward_with_observer: failure injected at site " +
                                                std::to_string(fail_site_) + " (test hook)");
    const size_t k = next_++;
    {
      std::unique_lock<std::mutex> lk(mu_);
      cv_.wait(lk, [&] { return done_[k] != 0; });
    }
    if (done_[k] < 0) return ctx->fail(ESM_GFX950_INTERNAL, "forward_with_observer: out of host memory");
    const ObsSite& st = sites_[k];
    const size_t off = k * obs::kReservoirSize;
    if (st.count == 0) return ESM_GFX950_OK;
    ESM_HIP(ctx, hipMemcpyAsync(obs_->d_pos + off, obs_->h_pos + off, st.count * 4, hipMemcpyHostToDevice,
                                ctx->stream));
    if (r24_lo)
      ESM_HIP(ctx, launch_observe_gather_r24(static_cast<const uint16_t*>(x), r24_lo, r24_cols, obs_->d_pos + off,
                                             static_cast<int>(st.count), obs_->d_val + off, ctx->stream));
    else
      ESM_HIP(ctx, launch_observe_gather(static_cast<const float*>(x), obs_->d_pos + off, static_cast<int>(st.count),
                                         gelu, obs_->d_val + off, ctx->stream));
    return ESM_GFX950_OK;
  }

  // After the forward: gathered values into the reservoirs (synchronises).
  int finish(esm_gfx950_ctx* ctx) {
    join();
    if (next_ != sites_.size()) return ctx->fail(ESM_GFX950_INTERNAL, "forward_with_observer: sites not captured");
    ESM_HIP(ctx, hipMemcpyAsync(obs_->h_val, obs_->d_val, sites_.size() * obs::kReservoirSize * 4,
                                hipMemcpyDeviceToHost, ctx->stream));
    ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (size_t k = 0; k < sites_.size(); ++k) {
      const ObsSite& st = sites_[k];
      const float* v = obs_->h_val + k * obs::kReservoirSize;
      for (size_t w = 0; w < st.count; ++w) st.r->samples[st.slots[w]] = v[w];
    }
    return ESM_GFX950_OK;
  }

 private:
  esm_gfx950_observer* obs_;
  std::vector<ObsSite> sites_;
  std::vector<int> done_;  // 0 pending, 1 planned, -1 failed
  std::mutex mu_;
  std::condition_variable cv_;
  std::vector<std::thread> threads_;
  size_t taken_ = 0;
  size_t next_ = 0;
  long fail_site_ = -1;
};

// One pre-LN encoder layer on the device (reference TransformerBlock,
// src/model.cpp:932-1066): LN -> QKV -> Q-scale -> RoPE -> attention ->
// out-proj -> residual -> LN -> fc1 -> GELU -> fc2 -> residual.
// The out-proj and fc2 GEMMs add their outputs into hidden in their
// epilogues (the residual adds, hidden + out), so the LayerNorm kernels that
// follow read hidden alone. `resid_in`, when not null, is a pending [T, d]
// residual for this layer's first LayerNorm to add; when split_in->splits >
// 0, the previous layer's fc2 output is instead still split-K int32 partial
// sums in the FFN intermediate buffer, which that LayerNorm kernel sums,
// dequantises and adds. With split_out set (per-token mode, not the last
// layer), this layer's fc2 may leave its output that way too: split_out
// says whether it did.
// Whether the per-tensor LayerNorm + quantisation can take the two-pass form
// (launch_layernorm's maximum alone, then launch_layernorm_quant_tensor).
bool ln_tensor_quant_ok(int d) { return d % 4 == 0 && d <= 2560; }

int layer_int8(esm_gfx950_ctx* ctx, const esm_gfx950_model* m, const DevLayer& L, int round16, const Arena& a,
               const Meta& md, int T, int nwork, int max_len, const float* resid_in, ObsRun* ob, int cus,
               const SplitResid* split_in = nullptr, SplitResid* split_out = nullptr) {
  const auto& c = m->cfg;
  const int d = c.hidden_size, f = c.intermediate_size, H = c.num_heads, dh = c.head_dim;
  const int ldq_d = pad16(d), ldq_f = pad16(f);
  const bool tok = c.act_quant_mode == ESM_GFX950_ACT_PER_TOKEN;
  hipStream_t s = ctx->stream;
  const float q_scale = 1.0f / std::sqrt(static_cast<float>(dh));
  int slot;

  const size_t Td = static_cast<size_t>(T) * d, Tf = static_cast<size_t>(T) * f;

  // (residual) + attn LN + activation quant
  if (tok) {
    const bool split = split_in && split_in->splits > 0;
    ESM_TRY(ctx->time_begin(resid_in || split ? "ln_quant" : "ln_quant_first", &slot));
    if (split)
      ESM_HIP(ctx, launch_layernorm_quant_split(a.hidden, *split_in, L.ln1_w, L.ln1_b, c.layer_norm_eps, T, d, a.xq,
                                                ldq_d, a.xs, s));
    else
      ESM_HIP(ctx, launch_layernorm_quant(a.hidden, resid_in, L.ln1_w, L.ln1_b, c.layer_norm_eps, T, d, a.xq,
                                          ldq_d, a.xs, s));
    ESM_TRY(ctx->time_end(slot));
    if (ob) {
      // The fused kernel keeps the LN output in registers: recompute it
      // (hidden already holds the residual sum) for the observer.
      ESM_HIP(ctx, launch_layernorm(a.hidden, nullptr, L.ln1_w, L.ln1_b, c.layer_norm_eps, a.lm_a, T, d, nullptr, s));
      ESM_TRY(ob->capture(ctx, a.lm_a, Td, 0));
    }
  } else {
    // The layer's four per-tensor maxima (attention LN, attention output,
    // FFN LN, FFN intermediate) start at zero.
    ESM_HIP(ctx, launch_fill_f32(a.absmax, 4, 0.0f, s));
    if (!ob && ln_tensor_quant_ok(d)) {
      // The LN's maximum first (no fp32 output), then the LN again,
      // quantised with the tensor scale: the same codes as LN + quant_tensor.
      ESM_HIP(ctx, launch_layernorm(a.hidden, resid_in, L.ln1_w, L.ln1_b, c.layer_norm_eps, nullptr, T, d, a.absmax,
                                    s));
      ESM_HIP(ctx, launch_layernorm_quant_tensor(a.hidden, L.ln1_w, L.ln1_b, c.layer_norm_eps, T, d, a.absmax, a.xq,
                                                 ldq_d, a.xs, s));
    } else {
      ESM_HIP(ctx, launch_layernorm(a.hidden, resid_in, L.ln1_w, L.ln1_b, c.layer_norm_eps, a.ln, T, d, a.absmax, s));
      if (ob) ESM_TRY(ob->capture(ctx, a.ln, Td, 0));
      ESM_HIP(ctx, launch_quant_tensor(a.ln, d, T, d, a.absmax, a.xq, ldq_d, a.xs, s));
    }
  }

  // QKV projection (one GEMM over the concatenated [3d, d] weight)
  GemmI8Args g;
  g.A = a.xq;
  g.lda = ldq_d;
  g.W = L.qkv.w8;
  g.ldw = L.qkv.ldk;
  g.M = T;
  g.cus = cus;
  g.N = 3 * d;
  g.K = L.qkv.ldk;
  g.a_scale = a.xs;
  g.w_scale = L.qkv.ws;
  g.bias = L.qkv.bias;
  g.d_model = d;
  g.pos = md.pos;
  g.rope_cos = md.cos_t;
  g.rope_sin = md.sin_t;
  // Q's 1/sqrt(dh) is already in the Q weight scales and bias when it is a
  // power of two (see model_create); otherwise the epilogues apply it.
  g.q_scale = m->q_scale_folded ? 1.0f : q_scale;
  const bool f32qkv = qkv_is_f32(c);
  ESM_TRY(ctx->time_begin("qkv", &slot));
  if (c.attention_mode == ESM_GFX950_ATTN_MODE_F16X3) {
    // Dequant + bias, Q scale, RoPE, then every value stored as a split-fp16
    // word (Q times kQPrescale) for the split-fp16 attention kernel.
    g.C_f32 = a.qkv;
    g.ldc = 3 * d;
    g.q_prescale = kQPrescale;
    if (!gemm_i8_pipelined_ok(g))
      return ctx->fail(ESM_GFX950_OUT_OF_RANGE,
                       "forward: the split-fp16 QKV epilogue needs T * hidden_size <= 2^32 bytes; use a smaller "
                       "batch or another attention_mode");
    ESM_HIP(ctx, launch_gemm_i8(g, kEpiQkvSplit, s));
  } else if (f32qkv && dh == kHeadDimMfma) {
    // Dequant + bias, Q scale and RoPE fused; fp32 Q|K|V rows.
    g.C_f32 = a.qkv;
    g.ldc = 3 * d;
    ESM_HIP(ctx, launch_gemm_i8(g, kEpiQkvRopeF32, s));
  } else if (f32qkv) {
    g.C_f32 = a.qkv;
    g.ldc = 3 * d;
    ESM_HIP(ctx, launch_gemm_i8(g, kEpiF32, s));
    ESM_HIP(ctx, launch_rope_f32(a.qkv, 3 * d, md.pos, T, H, dh, md.cos_t, md.sin_t, dh, g.q_scale, s));
    ESM_HIP(ctx, launch_rope_f32(a.qkv + d, 3 * d, md.pos, T, H, dh, md.cos_t, md.sin_t, dh, 1.0f, s));
  } else {
    g.q_out = a.qb;
    g.k_out = a.kb;
    g.v_out = a.vb;
    g.qk_fp16 = c.attention_mode == ESM_GFX950_ATTN_MODE_FP16 ? 1 : 0;
    ESM_HIP(ctx, launch_gemm_i8(g, kEpiQkvRope, s));
  }
  ESM_TRY(ctx->time_end(slot));

  // attention
  float* amax_attn = tok ? nullptr : a.absmax + 1;
  ESM_TRY(ctx->time_begin("attention", &slot));
  if (f32qkv) {
    if (c.attention_mode == ESM_GFX950_ATTN_MODE_F16X3) {
      // The QKV epilogue's layout: per [3 d]-word row, Q words, then K's
      // and V's hi and lo fp16 planes (d elements each).
      const auto* w = reinterpret_cast<const uint32_t*>(a.qkv);
      const auto* h16 = reinterpret_cast<const uint16_t*>(a.qkv);
      // Per tensor, the attention kernel leaves its waves' maxima (in the
      // FFN buffer, dead here) and one workgroup reduces them.
      float* part = !tok && static_cast<size_t>(nwork) * 4 <= Tf ? a.inter : nullptr;
      ESM_HIP(ctx, launch_attention_x3(w, 3 * d, h16 + 2 * d, h16 + 3 * d, h16 + 4 * d, h16 + 5 * d, 6 * d, kQPrescale,
                                       md.cu, md.work, nwork, a.attn, d, max_len, s, part));
      if (part)
        ESM_HIP(ctx, launch_max_of(part, static_cast<size_t>(nwork) * 4, amax_attn, s));
      else if (!tok)
        ESM_HIP(ctx, launch_absmax(a.attn, static_cast<size_t>(T) * d, amax_attn, s));
    } else {
      ESM_HIP(ctx, launch_attention_f32(a.qkv, a.qkv + d, a.qkv + 2 * d, 3 * d, dh, md.cu, md.work, nwork, a.attn,
                                        d, s));
      if (!tok) ESM_HIP(ctx, launch_absmax(a.attn, static_cast<size_t>(T) * d, amax_attn, s));
    }
  } else {
    const int qk16 = c.attention_mode == ESM_GFX950_ATTN_MODE_FP16 ? 1 : 0;
    ESM_HIP(ctx, launch_attention_mfma(a.qb, a.kb, a.vb, qk16, 0, d, md.cu, md.work, nwork, a.attn, d, amax_attn, s));
  }
  ESM_TRY(ctx->time_end(slot));
  if (ob) ESM_TRY(ob->capture(ctx, a.attn, Td, 0));
  if (tok) {
    ESM_TRY(ctx->time_begin("attn_quant", &slot));
    ESM_HIP(ctx, launch_quant_rows(a.attn, 0, d, T, d, a.xq, ldq_d, a.xs, s));
    ESM_TRY(ctx->time_end(slot));
  } else {
    ESM_HIP(ctx, launch_quant_tensor(a.attn, d, T, d, amax_attn, a.xq, ldq_d, a.xs, s));
  }

  // out-proj, added into hidden (the residual add)
  g = GemmI8Args();
  g.A = a.xq;
  g.lda = ldq_d;
  g.W = L.out.w8;
  g.ldw = L.out.ldk;
  g.M = T;
  g.cus = cus;
  g.N = d;
  g.K = L.out.ldk;
  g.a_scale = a.xs;
  g.w_scale = L.out.ws;
  g.bias = L.out.bias;
  g.C_f32 = a.hidden;
  g.ldc = d;
  // The FFN intermediate is dead here (its last reader was the previous
  // layer's GELU pass): small grids may split K into it.
  g.splitk_ws = reinterpret_cast<int32_t*>(a.inter);
  g.splitk_ws_elems = Tf;
  ESM_TRY(ctx->time_begin("out", &slot));
  ESM_HIP(ctx, launch_gemm_i8(g, kEpiF32Resid, s));
  ESM_TRY(ctx->time_end(slot));

  // ffn LN + quant. The observer sees the LN output before the first-block
  // fp16 rounding (reference src/model.cpp:1023-1033).
  if (tok) {
    ESM_TRY(ctx->time_begin("ln_quant", &slot));
    ESM_HIP(ctx, launch_layernorm_quant(a.hidden, nullptr, L.ln2_w, L.ln2_b, c.layer_norm_eps, T, d, a.xq, ldq_d,
                                        a.xs, s, round16));
    ESM_TRY(ctx->time_end(slot));
    if (ob) {
      ESM_HIP(ctx, launch_layernorm(a.hidden, nullptr, L.ln2_w, L.ln2_b, c.layer_norm_eps, a.lm_a, T, d, nullptr, s));
      ESM_TRY(ob->capture(ctx, a.lm_a, Td, 0));
    }
  } else if (!ob && ln_tensor_quant_ok(d)) {
    ESM_HIP(ctx, launch_layernorm(a.hidden, nullptr, L.ln2_w, L.ln2_b, c.layer_norm_eps, nullptr, T, d, a.absmax + 2,
                                  s, round16));
    ESM_HIP(ctx, launch_layernorm_quant_tensor(a.hidden, L.ln2_w, L.ln2_b, c.layer_norm_eps, T, d, a.absmax + 2, a.xq,
                                               ldq_d, a.xs, s, round16));
  } else {
    ESM_HIP(ctx, launch_layernorm(a.hidden, nullptr, L.ln2_w, L.ln2_b, c.layer_norm_eps, a.ln, T, d, a.absmax + 2,
                                  s, round16));
    if (ob && round16) {
      ESM_HIP(ctx, launch_layernorm(a.hidden, nullptr, L.ln2_w, L.ln2_b, c.layer_norm_eps, a.lm_a, T, d, nullptr, s));
      ESM_TRY(ob->capture(ctx, a.lm_a, Td, 0));
    } else if (ob) {
      ESM_TRY(ob->capture(ctx, a.ln, Td, 0));
    }
    ESM_HIP(ctx, launch_quant_tensor(a.ln, d, T, d, a.absmax + 2, a.xq, ldq_d, a.xs, s));
  }

  // fc1 + GELU
  g = GemmI8Args();
  g.A = a.xq;
  g.lda = ldq_d;
  g.W = L.fc1.w8;
  g.ldw = L.fc1.ldk;
  g.M = T;
  g.cus = cus;
  g.N = f;
  g.K = L.fc1.ldk;
  g.a_scale = a.xs;
  g.w_scale = L.fc1.ws;
  g.bias = L.fc1.bias;
  g.C_f32 = a.inter;
  g.ldc = f;
  if (tok && m->ffn_r24 && f % 64 == 0 && f <= 10240 && gemm_i8_pipelined_ok(g)) {
    // Dequant + bias rounded to 24 bits (a high 16-bit plane, then a low
    // byte plane, in the FFN buffer): 3 bytes per value instead of 4 for the
    // GEMM to write and the GELU + quant pass to read.
    g.C_f32 = nullptr;
    g.C_f16 = reinterpret_cast<uint16_t*>(a.inter);
    g.C_u8 = reinterpret_cast<uint8_t*>(a.inter) + Tf * 2;
    ESM_TRY(ctx->time_begin("fc1", &slot));
    ESM_HIP(ctx, launch_gemm_i8(g, kEpiF32R24, s));
    ESM_TRY(ctx->time_end(slot));
    // The observer sees GELU of the 24-bit values fc2's quantisation reads.
    if (ob) ESM_TRY(ob->capture(ctx, g.C_f16, Tf, 1, g.C_u8, f));
    ESM_TRY(ctx->time_begin("gelu_quant", &slot));
    ESM_HIP(ctx, launch_gelu_quant_rows_r24(g.C_f16, g.C_u8, f, T, f, a.xq, ldq_f, a.xs, s));
    ESM_TRY(ctx->time_end(slot));
  } else if (tok) {
    // Dequant + bias only; GELU runs in the per-token quantisation pass that
    // reads these rows anyway.
    ESM_TRY(ctx->time_begin("fc1", &slot));
    ESM_HIP(ctx, launch_gemm_i8(g, kEpiF32, s));
    ESM_TRY(ctx->time_end(slot));
    if (ob) ESM_TRY(ob->capture(ctx, a.inter, Tf, 1));
    ESM_TRY(ctx->time_begin("gelu_quant", &slot));
    ESM_HIP(ctx, launch_gelu_quant_rows(a.inter, f, T, f, a.xq, ldq_f, a.xs, s));
    ESM_TRY(ctx->time_end(slot));
  } else {
    // GELU with the erf of the fused GELU + quantisation passes (Abramowitz
    // & Stegun 7.1.26, as the reference's AVX-512 Gelu) in the epilogue,
    // with the tensor's maximum.
    g.tensor_absmax = a.absmax + 3;
    ESM_TRY(ctx->time_begin("fc1", &slot));
    ESM_HIP(ctx, launch_gemm_i8(g, kEpiF32GeluAs, s));
    ESM_TRY(ctx->time_end(slot));
    if (ob) ESM_TRY(ob->capture(ctx, a.inter, Tf, 0));
    ESM_HIP(ctx, launch_quant_tensor(a.inter, f, T, f, a.absmax + 3, a.xq, ldq_f, a.xs, s));
  }

  // fc2, added into hidden (the residual add) or left as split-K partial sums
  // for the next layer's first LayerNorm
  g = GemmI8Args();
  g.A = a.xq;
  g.lda = ldq_f;
  g.W = L.fc2.w8;
  g.ldw = L.fc2.ldk;
  g.M = T;
  g.cus = cus;
  g.N = d;
  g.K = L.fc2.ldk;
  g.a_scale = a.xs;
  g.w_scale = L.fc2.ws;
  g.bias = L.fc2.bias;
  g.C_f32 = a.hidden;
  g.ldc = d;
  // fc2's input is already quantised from the FFN intermediate, which is
  // therefore free to hold split-K partial sums.
  g.splitk_ws = reinterpret_cast<int32_t*>(a.inter);
  g.splitk_ws_elems = Tf;
  ESM_TRY(ctx->time_begin("fc2", &slot));
  if (split_out) split_out->splits = 0;
  int rows = 0;
  const int S = split_out && tok && !ob && gemm_i8_pipelined_ok(g) ? gemm_i8_split_k(T, d, g.K, cus, true, &rows) : 1;
  if (S > 1 && static_cast<size_t>(S) * Td <= Tf) {
    // The next layer's first LayerNorm sums the partial planes.
    g.C_i32 = g.splitk_ws;
    g.ldc = d;
    ESM_HIP(ctx, launch_gemm_i8_partials(g, S, rows, s));
    *split_out = SplitResid{g.splitk_ws, S, a.xs, L.fc2.ws, L.fc2.bias};
  } else {
    ESM_HIP(ctx, launch_gemm_i8(g, kEpiF32Resid, s));
  }
  ESM_TRY(ctx->time_end(slot));
  return ESM_GFX950_OK;
}

int f32_linear(esm_gfx950_ctx* ctx, const float* A, const DevLinear& W, float* C, int M, int epi) {
  GemmF32Args p;
  p.A = A;
  p.lda = W.K;
  p.W = W.w32;
  p.ldw = W.K;
  p.bias = W.bias;
  p.C = C;
  p.ldc = W.N;
  p.M = M;
  p.N = W.N;
  p.K = W.K;
  ESM_HIP(ctx, launch_gemm_f32(p, epi, ctx->stream));
  return ESM_GFX950_OK;
}

int layer_f32(esm_gfx950_ctx* ctx, const esm_gfx950_model* m, const DevLayer& L, int round16, const Arena& a,
              const Meta& md, int T, int nwork, ObsRun* ob) {
  const auto& c = m->cfg;
  const int d = c.hidden_size, H = c.num_heads, dh = c.head_dim;
  hipStream_t s = ctx->stream;
  const float q_scale = 1.0f / std::sqrt(static_cast<float>(dh));
  const size_t Td = static_cast<size_t>(T) * d, Tf = static_cast<size_t>(T) * c.intermediate_size;
  ESM_HIP(ctx, launch_layernorm(a.hidden, nullptr, L.ln1_w, L.ln1_b, c.layer_norm_eps, a.ln, T, d, nullptr, s));
  if (ob) ESM_TRY(ob->capture(ctx, a.ln, Td, 0));
  ESM_TRY(f32_linear(ctx, a.ln, L.qkv, a.qkv, T, kF32Store));
  ESM_HIP(ctx, launch_rope_f32(a.qkv, 3 * d, md.pos, T, H, dh, md.cos_t, md.sin_t, dh, q_scale, s));
  ESM_HIP(ctx, launch_rope_f32(a.qkv + d, 3 * d, md.pos, T, H, dh, md.cos_t, md.sin_t, dh, 1.0f, s));
  ESM_HIP(ctx, launch_attention_f32(a.qkv, a.qkv + d, a.qkv + 2 * d, 3 * d, dh, md.cu, md.work, nwork, a.attn, d, s));
  if (ob) ESM_TRY(ob->capture(ctx, a.attn, Td, 0));
  ESM_TRY(f32_linear(ctx, a.attn, L.out, a.hidden, T, kF32Resid));
  ESM_HIP(ctx, launch_layernorm(a.hidden, nullptr, L.ln2_w, L.ln2_b, c.layer_norm_eps, a.ln, T, d, nullptr, s,
                                round16));
  if (ob && round16) {
    ESM_HIP(ctx, launch_layernorm(a.hidden, nullptr, L.ln2_w, L.ln2_b, c.layer_norm_eps, a.lm_a, T, d, nullptr, s));
    ESM_TRY(ob->capture(ctx, a.lm_a, Td, 0));
  } else if (ob) {
    ESM_TRY(ob->capture(ctx, a.ln, Td, 0));
  }
  ESM_TRY(f32_linear(ctx, a.ln, L.fc1, a.inter, T, kF32Gelu));
  if (ob) ESM_TRY(ob->capture(ctx, a.inter, Tf, 0));
  ESM_TRY(f32_linear(ctx, a.inter, L.fc2, a.hidden, T, kF32Resid));
  return ESM_GFX950_OK;
}

// The x86-exact attention's score scratch: the FFN buffer (dead while the
// attention runs) when the part's scores fit there and in 32-bit offsets.
float* x86_score_scratch(const esm_gfx950_model::Part& P, const Arena& a, size_t Tf, int heads) {
  const size_t per_head = P.x86_score_floats / static_cast<size_t>(heads);
  return P.x86_score_floats <= Tf && per_head < (static_cast<size_t>(1) << 32) ? a.inter : nullptr;
}

// TransformerBlock (reference src/model.cpp:932-1066) on the reference's x86
// AVX-512 VNNI kernels, bit for bit: LayerNormAvx512, LinearVnni (per-tensor
// activation scale, QuantizeActPrefixAvx512; the INT8 GEMM's dequant
// epilogue is FinalizeStore16's expression) or LinearAmx (numerics X86_AMX:
// the same, with its last T % 32 rows quantised on their own, reference
// src/kernels/gemm_amx.cpp:218-309), ScaleInplace (folded into the Q
// weight scales when exact) and RopeApplyVarlenAvx512, AttentionVarlenAvx512,
// GeluAvx512, ResidualAddInplace. Q, K and V come from one GEMM over the
// concatenated weight: the reference's three LinearInt8 calls quantise the
// same LayerNorm output to the same bytes and scale. `resid_in` as in
// layer_int8.
int layer_int8_x86(esm_gfx950_ctx* ctx, const esm_gfx950_model* m, const DevLayer& L, int round16, const Arena& a,
                   const Meta& md, const esm_gfx950_model::Part& P, const float* resid_in, ObsRun* ob) {
  const auto& c = m->cfg;
  const int d = c.hidden_size, f = c.intermediate_size, H = c.num_heads, dh = c.head_dim, T = P.T;
  const int ldq_d = pad16(d), ldq_f = pad16(f);
  const size_t Td = static_cast<size_t>(T) * d, Tf = static_cast<size_t>(T) * f;
  hipStream_t s = ctx->stream;
  int slot;
  auto linear = [&](const DevLinear& W, int lda, float* C, const char* site, int epi = kEpiF32,
                    float* tensor_absmax = nullptr) -> int {
    GemmI8Args g;
    g.A = a.xq;
    g.lda = lda;
    g.W = W.w8;
    g.ldw = W.ldk;
    g.M = T;
    g.N = W.N;
    g.K = W.ldk;
    g.a_scale = a.xs;
    g.w_scale = W.ws;
    g.bias = W.bias;
    g.C_f32 = C;
    g.ldc = W.N;
    g.tensor_absmax = tensor_absmax;
    ESM_TRY(ctx->time_begin(site, &slot));
    ESM_HIP(ctx, launch_gemm_i8(g, epi, s));
    return ctx->time_end(slot);
  };

  // QuantizeActPrefixAvx512 of x [T, cols] with the whole tensor's absmax
  // (amax, already reduced); for LinearAmx (numerics X86_AMX) with its
  // shape gate met by the consuming linear (N % 32, K % 64, T >= 32), the
  // last T % 32 rows again with their own absmax (slot: a scratch scalar).
  const bool amx = m->numerics == ESM_GFX950_NUMERICS_X86_AMX;
  const int t_main = T & ~31;
  auto quant = [&](const float* x, int cols, int ldq, float* amax, int n_out, float* slot) -> int {
    ESM_HIP(ctx, launch_quant_tensor(x, cols, T, cols, amax, a.xq, ldq, a.xs, s));
    if (amx && T >= 32 && n_out % 32 == 0 && cols % 64 == 0 && t_main < T) {
      const float* xt = x + static_cast<size_t>(t_main) * cols;
      ESM_HIP(ctx, launch_fill_f32(slot, 1, 0.0f, s));
      ESM_HIP(ctx, launch_absmax(xt, static_cast<size_t>(T - t_main) * cols, slot, s));
      ESM_HIP(ctx, launch_quant_tensor(xt, cols, T - t_main, cols, slot, a.xq + static_cast<size_t>(t_main) * ldq, ldq,
                                       a.xs + t_main, s));
    }
    return ESM_GFX950_OK;
  };
  // Without an observer (which samples the fp32 LayerNorm output), a
  // LayerNorm and its quantisation run as two passes over hidden: the
  // maxima (and the residual add), then the LayerNorm again, quantised; the
  // same codes and scales as the LayerNorm output's launch_quant_tensor.
  const bool ln_two_pass = !ob && layernorm_x86_rows_ok(d);
  auto ln_quant = [&](const float* resid, const float* gamma, const float* beta, int r16, float* amax, int n_out,
                      float* slot) -> int {
    const bool tail = amx && T >= 32 && n_out % 32 == 0 && d % 64 == 0 && t_main < T;
    ESM_HIP(ctx, launch_layernorm_x86(a.hidden, resid, gamma, beta, c.layer_norm_eps, nullptr, T, d, amax, r16, s,
                                      tail ? slot : nullptr, tail ? t_main : T));
    ESM_HIP(ctx, launch_layernorm_x86_quant(a.hidden, gamma, beta, c.layer_norm_eps, T, d, amax, tail ? slot : nullptr,
                                            tail ? t_main : T, a.xq, ldq_d, a.xs, r16, s));
    return ESM_GFX950_OK;
  };

  ESM_HIP(ctx, launch_fill_f32(a.absmax, 8, 0.0f, s));
  // Q, K and V are three linears of N = d each in the reference.
  if (ln_two_pass) {
    ESM_TRY(ln_quant(resid_in, L.ln1_w, L.ln1_b, 0, a.absmax, d, a.absmax + 4));
  } else {
    ESM_HIP(ctx, launch_layernorm_x86(a.hidden, resid_in, L.ln1_w, L.ln1_b, c.layer_norm_eps, a.ln, T, d, a.absmax, 0,
                                      s));
    if (ob) ESM_TRY(ob->capture(ctx, a.ln, Td, 0));
    ESM_TRY(quant(a.ln, d, ldq_d, a.absmax, d, a.absmax + 4));
  }
  const float q_scale = m->q_scale_folded ? 1.0f : 1.0f / std::sqrt(static_cast<float>(dh));
  {
    // ScaleInplace and RopeApplyVarlenAvx512 in the QKV GEMM's epilogue
    // (64-wide heads, pipelined kernel), else as passes of their own.
    GemmI8Args g;
    g.A = a.xq;
    g.lda = ldq_d;
    g.W = L.qkv.w8;
    g.ldw = L.qkv.ldk;
    g.M = T;
    g.N = L.qkv.N;
    g.K = L.qkv.ldk;
    g.a_scale = a.xs;
    g.w_scale = L.qkv.ws;
    g.bias = L.qkv.bias;
    g.C_f32 = a.qkv;
    g.ldc = L.qkv.N;
    g.d_model = d;
    g.pos = md.pos;
    g.rope_cos = md.cos_t;
    g.rope_sin = md.sin_t;
    g.q_scale = q_scale;
    g.rope_x86 = 1;
    if (dh == kHeadDimMfma && gemm_i8_pipelined_ok(g)) {
      ESM_TRY(ctx->time_begin("qkv", &slot));
      ESM_HIP(ctx, launch_gemm_i8(g, kEpiQkvRopeF32, s));
      ESM_TRY(ctx->time_end(slot));
    } else {
      ESM_TRY(linear(L.qkv, ldq_d, a.qkv, "qkv"));
      ESM_HIP(ctx, launch_rope_x86(a.qkv, 3 * d, md.pos, T, H, dh, md.cos_t, md.sin_t, dh, q_scale, s));
      ESM_HIP(ctx, launch_rope_x86(a.qkv + d, 3 * d, md.pos, T, H, dh, md.cos_t, md.sin_t, dh, 1.0f, s));
    }
  }
  ESM_TRY(ctx->time_begin("attention", &slot));
  // Each work item's largest |output| goes to the LayerNorm buffer (dead
  // here) and one workgroup reduces them: the output's maximum.
  float* part = static_cast<size_t>(P.nwork) <= Td ? a.ln : nullptr;
  ESM_HIP(ctx, launch_attention_x86(a.qkv, a.qkv + d, a.qkv + 2 * d, 3 * d, dh, md.cu, P.B, H, P.maxL, a.attn, d, s,
                                    x86_score_scratch(P, a, Tf, H), md.work, P.nwork, part));
  ESM_TRY(ctx->time_end(slot));
  if (ob) ESM_TRY(ob->capture(ctx, a.attn, Td, 0));
  if (part)
    ESM_HIP(ctx, launch_max_of(part, static_cast<size_t>(P.nwork), a.absmax + 1, s));
  else
    ESM_HIP(ctx, launch_absmax(a.attn, Td, a.absmax + 1, s));
  ESM_TRY(quant(a.attn, d, ldq_d, a.absmax + 1, d, a.absmax + 5));
  ESM_TRY(linear(L.out, ldq_d, a.ybuf, "out"));
  if (ln_two_pass) {
    ESM_TRY(ln_quant(a.ybuf, L.ln2_w, L.ln2_b, round16, a.absmax + 2, f, a.absmax + 6));
  } else {
    ESM_HIP(ctx, launch_layernorm_x86(a.hidden, a.ybuf, L.ln2_w, L.ln2_b, c.layer_norm_eps, a.ln, T, d, a.absmax + 2,
                                      round16, s));
    if (ob && round16) {
      // The observer sees the LayerNorm output before the fp16 rounding.
      ESM_HIP(ctx, launch_layernorm_x86(a.hidden, nullptr, L.ln2_w, L.ln2_b, c.layer_norm_eps, a.lm_a, T, d, nullptr,
                                        0, s));
      ESM_TRY(ob->capture(ctx, a.lm_a, Td, 0));
    } else if (ob) {
      ESM_TRY(ob->capture(ctx, a.ln, Td, 0));
    }
    ESM_TRY(quant(a.ln, d, ldq_d, a.absmax + 2, f, a.absmax + 6));
  }
  // fc1 + GeluAvx512 (and the GELU output's maximum) in the GEMM's epilogue.
  ESM_TRY(linear(L.fc1, ldq_d, a.inter, "fc1", kEpiF32GeluX86, a.absmax + 3));
  if (ob) ESM_TRY(ob->capture(ctx, a.inter, Tf, 0));
  ESM_TRY(quant(a.inter, f, ldq_f, a.absmax + 3, d, a.absmax + 7));
  return linear(L.fc2, ldq_f, a.ybuf, "fc2");
}

// TransformerBlock of an all-fp32 model on the reference's x86 kernels:
// LinearAvx512 for every projection (Q|K|V as one concatenated weight: each
// output is its own dot product), then as layer_int8_x86.
int layer_f32_x86(esm_gfx950_ctx* ctx, const esm_gfx950_model* m, const DevLayer& L, int round16, const Arena& a,
                  const Meta& md, const esm_gfx950_model::Part& P, ObsRun* ob) {
  const auto& c = m->cfg;
  const int d = c.hidden_size, H = c.num_heads, dh = c.head_dim, T = P.T;
  const size_t Td = static_cast<size_t>(T) * d, Tf = static_cast<size_t>(T) * c.intermediate_size;
  hipStream_t s = ctx->stream;
  auto linear = [&](const float* A, const DevLinear& W, float* C, int epi) -> int {
    ESM_HIP(ctx, launch_linear_x86(A, W.K, W.w32, W.K, W.bias, C, W.N, T, W.N, W.K, epi, s));
    return ESM_GFX950_OK;
  };
  ESM_HIP(ctx, launch_layernorm_x86(a.hidden, nullptr, L.ln1_w, L.ln1_b, c.layer_norm_eps, a.ln, T, d, nullptr, 0, s));
  if (ob) ESM_TRY(ob->capture(ctx, a.ln, Td, 0));
  ESM_TRY(linear(a.ln, L.qkv, a.qkv, kF32Store));
  const float q_scale = 1.0f / std::sqrt(static_cast<float>(dh));
  ESM_HIP(ctx, launch_rope_x86(a.qkv, 3 * d, md.pos, T, H, dh, md.cos_t, md.sin_t, dh, q_scale, s));
  ESM_HIP(ctx, launch_rope_x86(a.qkv + d, 3 * d, md.pos, T, H, dh, md.cos_t, md.sin_t, dh, 1.0f, s));
  ESM_HIP(ctx, launch_attention_x86(a.qkv, a.qkv + d, a.qkv + 2 * d, 3 * d, dh, md.cu, P.B, H, P.maxL, a.attn, d, s,
                                    x86_score_scratch(P, a, Tf, H), md.work, P.nwork));
  if (ob) ESM_TRY(ob->capture(ctx, a.attn, Td, 0));
  ESM_TRY(linear(a.attn, L.out, a.hidden, kF32Resid));
  ESM_HIP(ctx, launch_layernorm_x86(a.hidden, nullptr, L.ln2_w, L.ln2_b, c.layer_norm_eps, a.ln, T, d, nullptr,
                                    round16, s));
  if (ob && round16) {
    ESM_HIP(ctx, launch_layernorm_x86(a.hidden, nullptr, L.ln2_w, L.ln2_b, c.layer_norm_eps, a.lm_a, T, d, nullptr, 0,
                                      s));
    ESM_TRY(ob->capture(ctx, a.lm_a, Td, 0));
  } else if (ob) {
    ESM_TRY(ob->capture(ctx, a.ln, Td, 0));
  }
  ESM_TRY(linear(a.ln, L.fc1, a.inter, kF32Gelu));
  if (ob) ESM_TRY(ob->capture(ctx, a.inter, Tf, 0));
  return linear(a.inter, L.fc2, a.hidden, kF32Resid);
}

constexpr float kTokenDropoutMaskRatioTrain = 0.15f * 0.8f;

}  // namespace

namespace {

// Makes ctx->stream refer to a part's stream for the launches of that part.
struct StreamScope {
  esm_gfx950_ctx* ctx;
  hipStream_t saved;
  StreamScope(esm_gfx950_ctx* c, hipStream_t s) : ctx(c), saved(c->stream) {
    if (s) ctx->stream = s;
  }
  ~StreamScope() { ctx->stream = saved; }
};

// Stages one part: sequences [b0, b0 + B) of the packed batch, tokens
// [cu[b0], cu[b0 + B]). masks (nullable, packed like ids): 0 marks a pad.
int stage_part(esm_gfx950_ctx* ctx, esm_gfx950_model* m, esm_gfx950_model::Part& P, const int32_t* ids,
               const int32_t* masks, const int32_t* cu, int b0, int B) {
  const auto& c = m->cfg;
  const int H = c.num_heads, dh = c.head_dim;
  const int t0 = cu[b0];
  const int T = cu[b0 + B] - t0;
  int maxL = 0;
  for (int b = b0; b < b0 + B; ++b) maxL = std::max(maxL, cu[b + 1] - cu[b]);
  StreamScope scope(ctx, P.stream);

  // Grow the arena and metadata buffers only when this part exceeds them.
  if (T > P.cap_T || B > P.cap_B || maxL > P.cap_L) {
    ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    const int nT = std::max(T, P.cap_T), nB = std::max(B, P.cap_B), nL = std::max(maxL, P.cap_L);
    if (P.arena) hipFree(P.arena);
    if (P.meta_dev) hipFree(P.meta_dev);
    if (P.meta_host) hipHostFree(P.meta_host);
    P.arena = P.meta_dev = P.meta_host = nullptr;
    P.arena_bytes = P.meta_bytes = 0;
    P.cap_T = P.cap_B = P.cap_L = 0;
    const Arena probe = layout(c, nT, nullptr, m->numerics != ESM_GFX950_NUMERICS_DEFAULT);
    const Meta mprobe = meta_layout(nT, nB, nL, H, dh, nullptr);
    ESM_HIP(ctx, hipMalloc(&P.arena, probe.bytes));
    P.arena_bytes = probe.bytes;
    ESM_HIP(ctx, hipMalloc(&P.meta_dev, mprobe.bytes));
    ESM_HIP(ctx, hipHostMalloc(&P.meta_host, mprobe.bytes, hipHostMallocDefault));
    P.meta_bytes = mprobe.bytes;
    P.cap_T = nT;
    P.cap_B = nB;
    P.cap_L = nL;
    P.rope_len = 0;
  }
  const Meta mh = meta_layout(P.cap_T, P.cap_B, P.cap_L, H, dh, static_cast<char*>(P.meta_host));

  // Host metadata: ids, per-token embedding scale (Embed, model.cpp:737-778:
  // real tokens counted by the mask, mask tokens counted over every token;
  // a pad's scale is 0, which the embedding kernel turns into a zero row),
  // positions, cu_seqlens (rebased to the part), attention work list, rope
  // tables.
  ESM_HIP(ctx, hipEventSynchronize(P.meta_done));
  std::memcpy(mh.ids, ids + t0, static_cast<size_t>(T) * 4);
  for (int b = 0; b <= B; ++b) mh.cu[b] = cu[b0 + b] - t0;
  const int32_t* mk = masks ? masks + t0 : nullptr;
  for (int b = 0; b < B; ++b) {
    int src_len = 0, mask_tokens = 0;
    for (int t = mh.cu[b]; t < mh.cu[b + 1]; ++t) {
      if (!mk || mk[t] != 0) ++src_len;
      if (mh.ids[t] == c.mask_token_id) ++mask_tokens;
    }
    const float ratio = src_len > 0 ? static_cast<float>(mask_tokens) / static_cast<float>(src_len) : 0.0f;
    const float scale = (1.0f - kTokenDropoutMaskRatioTrain) / std::max(1.0f - ratio, 1e-12f);
    for (int t = mh.cu[b]; t < mh.cu[b + 1]; ++t) mh.tok_scale[t] = (mk && mk[t] == 0) ? 0.0f : scale;
  }
  build_pos(mh.cu, B, mh.pos);
  // The x86-exact attention takes 64-query tiles, longest sequences first.
  const bool mfma_attn = c.weights_int8 && c.attention_mode != ESM_GFX950_ATTN_MODE_FP32 &&
                         m->numerics == ESM_GFX950_NUMERICS_DEFAULT;
  std::vector<AttnWork> work;
  build_work(mh.cu, B, H, mfma_attn ? kAttnMfmaQTile : kAttnF32QTile, &work, mfma_attn);
  if (work.size() > mh.work_cap)
    return ctx->fail(ESM_GFX950_INTERNAL, "batch_upload: attention work list (" + std::to_string(work.size()) +
                                              " items) exceeds its metadata region (" +
                                              std::to_string(mh.work_cap) + ")");
  std::memcpy(mh.work, work.data(), work.size() * sizeof(AttnWork));
  const bool new_tables = P.rope_len < maxL;
  if (new_tables) rope_tables(P.cap_L, dh, mh.cos_t, mh.sin_t);
  const size_t upto = reinterpret_cast<const char*>(mh.cos_t) - static_cast<const char*>(P.meta_host);
  ESM_HIP(ctx, hipMemcpyAsync(P.meta_dev, P.meta_host, new_tables ? P.meta_bytes : upto, hipMemcpyHostToDevice,
                              ctx->stream));
  ESM_HIP(ctx, hipEventRecord(P.meta_done, ctx->stream));
  if (new_tables) P.rope_len = P.cap_L;
  P.T = T;
  P.B = B;
  P.t0 = t0;
  P.maxL = maxL;
  P.nwork = static_cast<int>(work.size());
  P.x86_score_floats = attention_x86_score_floats(mh.cu, B, m->cfg.num_heads);
  return ESM_GFX950_OK;
}

// The whole forward of one part on ctx->stream; logits rows [0, T).
// Hidden-state capture for esm_gfx950_forward_hidden_states: base points at
// this part's first row of state 0 in a device buffer [layers + 1, T, d],
// stride is T * d floats between states.
struct HiddenCapture {
  float* base = nullptr;
  size_t stride = 0;
};

int forward_part(esm_gfx950_ctx* ctx, const esm_gfx950_model* m, const esm_gfx950_model::Part& P, float* logits,
                 ObsRun* ob = nullptr, const HiddenCapture* cap = nullptr) {
  const auto& c = m->cfg;
  const int T = P.T;
  const int d = c.hidden_size, V = c.vocab_size, H = c.num_heads, dh = c.head_dim;
  const bool x86 = m->numerics != ESM_GFX950_NUMERICS_DEFAULT;
  const Arena a = part_arena(m, P);
  const Meta md = meta_layout(P.cap_T, P.cap_B, P.cap_L, H, dh, static_cast<char*>(P.meta_dev));
  const int nwork = P.nwork;

  hipStream_t s = ctx->stream;
  // Parts staged together run concurrently on their own streams: each
  // part's GEMMs pick their tile heights for its share of the CUs.
  int active = 0;
  for (const auto& q : m->parts) active += q.T > 0 ? 1 : 0;
  const int cus = active > 1 ? std::max(1, device_cus() / active) : 0;
  ESM_HIP(ctx, launch_embed(md.ids, md.tok_scale, m->embed, T, d, c.mask_token_id, a.hidden, s));
  const size_t Td = static_cast<size_t>(T) * d;
  auto capture = [&](size_t state, const float* src) -> int {
    ESM_HIP(ctx, hipMemcpyAsync(cap->base + state * cap->stride, src, Td * 4, hipMemcpyDeviceToDevice, s));
    return ESM_GFX950_OK;
  };
  if (cap) ESM_TRY(capture(0, a.hidden));
  // x86 numerics: fc2 output awaiting its residual add (in the next
  // LayerNorm); default numerics: fc2's split-K partial sums awaiting theirs.
  const float* pending = nullptr;
  SplitResid pending_split;
  for (size_t li = 0; li < m->layers.size(); ++li) {
    const DevLayer& L = m->layers[li];
    const int round16 = (li == 0 && m->first_block_fc1_fp16) ? 1 : 0;
    if (x86 && c.weights_int8) {
      ESM_TRY(layer_int8_x86(ctx, m, L, round16, a, md, P, pending, ob));
      pending = a.ybuf;
    } else if (x86) {
      ESM_TRY(layer_f32_x86(ctx, m, L, round16, a, md, P, ob));
    } else if (c.weights_int8) {
      SplitResid split_out;
      const bool last = li + 1 == m->layers.size();
      // A captured forward keeps every layer's hidden state whole: no split-K
      // partial sums left for the next layer (int32 sums, same bits).
      ESM_TRY(layer_int8(ctx, m, L, round16, a, md, T, nwork, P.maxL, pending, ob, cus, &pending_split,
                         last || cap ? nullptr : &split_out));
      pending = nullptr;  // fc2 added its output into hidden (or left split partials)
      pending_split = split_out;
    } else {
      ESM_TRY(layer_f32(ctx, m, L, round16, a, md, T, nwork, ob));
    }
    if (cap && li + 1 < m->layers.size()) {
      if (pending) {
        // The residual add the next LayerNorm would fuse (the same fp32 add).
        ESM_HIP(ctx, launch_residual_add(a.hidden, pending, Td, s));
        pending = nullptr;
      }
      ESM_TRY(capture(li + 1, a.hidden));
    }
  }
  if (x86) {
    // Final LN, then the lm head on the reference's x86 kernels: Linear
    // (LinearAvx512) -> Gelu -> LayerNorm -> tied decoder Linear
    // (reference src/model.cpp:1181-1239).
    ESM_HIP(ctx, launch_layernorm_x86(a.hidden, pending, m->final_ln_w, m->final_ln_b, c.layer_norm_eps, a.ln, T, d,
                                      nullptr, 0, s));
    if (cap) ESM_TRY(capture(m->layers.size(), a.ln));
    int slot;
    ESM_TRY(ctx->time_begin("lm_dense", &slot));
    ESM_HIP(ctx, launch_linear_x86(a.ln, d, m->lm_dense_w, d, m->lm_dense_b, a.lm_a, d, T, d, d, kF32Gelu, s));
    ESM_TRY(ctx->time_end(slot));
    ESM_HIP(ctx, launch_layernorm_x86(a.lm_a, nullptr, m->lm_ln_w, m->lm_ln_b, c.layer_norm_eps, a.attn, T, d, nullptr,
                                      0, s));
    ESM_HIP(ctx, launch_linear_x86(a.attn, d, m->embed, d, m->dec_bias, logits, V, T, V, d, kF32Store, s));
    return ESM_GFX950_OK;
  }
  // (Last residual +) final LN and lm head: dense -> GELU -> LN -> tied
  // decoder + bias (reference src/model.cpp:1181-1239).
  ESM_HIP(ctx, launch_layernorm(a.hidden, pending, m->final_ln_w, m->final_ln_b, c.layer_norm_eps, a.ln, T, d,
                                nullptr, s));
  if (cap) ESM_TRY(capture(m->layers.size(), a.ln));
  DevLinear dense;
  dense.w32 = m->lm_dense_w;
  dense.bias = m->lm_dense_b;
  dense.N = d;
  dense.K = d;
  int slot;
  ESM_TRY(ctx->time_begin("lm_dense", &slot));
  if (m->lm_dense_split) {
    GemmX3Args x;
    x.A = a.ln;
    x.lda = d;
    x.w_hi = m->lm_w_hi;
    x.w_lo = m->lm_w_lo;
    x.ldw = d;
    x.w_unscale = m->lm_w_unscale;
    x.bias = m->lm_dense_b;
    x.C = a.lm_a;
    x.ldc = d;
    x.M = T;
    x.N = d;
    x.K = d;
    ESM_HIP(ctx, launch_gemm_x3(x, kF32Gelu, s));
  } else {
    ESM_TRY(f32_linear(ctx, a.ln, dense, a.lm_a, T, kF32Gelu));
  }
  ESM_TRY(ctx->time_end(slot));
  ESM_HIP(ctx, launch_layernorm(a.lm_a, nullptr, m->lm_ln_w, m->lm_ln_b, c.layer_norm_eps, a.attn, T, d, nullptr, s));
  if (V <= 48 && d % 16 == 0) {
    // Tied decoder (vocabulary 33): the narrow fp32 MFMA kernel.
    GemmF32Args g;
    g.A = a.attn;
    g.lda = d;
    g.W = m->embed;
    g.ldw = d;
    g.bias = m->dec_bias;
    g.C = logits;
    g.ldc = V;
    g.M = T;
    g.N = V;
    g.K = d;
    ESM_HIP(ctx, launch_gemm_narrow(g, s));
  } else {
    DevLinear dec;
    dec.w32 = m->embed;
    dec.bias = m->dec_bias;
    dec.N = V;
    dec.K = d;
    ESM_TRY(f32_linear(ctx, a.attn, dec, logits, T, kF32Store));
  }
  return ESM_GFX950_OK;
}

}  // namespace

extern "C" int esm_gfx950_model_get_config(const esm_gfx950_model* m, esm_gfx950_model_config* out) {
  if (!m || !out) return ESM_GFX950_INVALID_ARGUMENT;
  *out = m->cfg;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_model_staged_parts(const esm_gfx950_model* m, int* parts) {
  if (!m || !parts) return ESM_GFX950_INVALID_ARGUMENT;
  int n = 0;
  for (const auto& P : m->parts) n += P.T > 0 ? 1 : 0;
  *parts = n;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_model_set_parts(esm_gfx950_ctx* ctx, esm_gfx950_model* m, int parts) {
  if (!ctx || !m) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, parts >= 0 && parts <= 4, "model_set_parts: parts must be 0 (automatic) or 1..4");
  const bool automatic = parts == 0;
  if (automatic) parts = kAutoMaxParts;
  m->auto_parts = automatic;
  if (static_cast<int>(m->parts.size()) == parts) return ESM_GFX950_OK;
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  for (auto& p : m->parts) {
    if (p.stream) ESM_HIP(ctx, hipStreamSynchronize(p.stream));
    free_part(p);
  }
  m->parts.assign(parts, esm_gfx950_model::Part());
  for (int i = 0; i < parts; ++i) ESM_TRY(init_part(ctx, m->parts[i], i > 0));
  m->staged_T = 0;
  return ESM_GFX950_OK;
}

namespace {

// Sequence groups for a batch of T tokens under the automatic count: one per
// 6e11 int8 operations of a layer's four linears (24 T d^2), at least one and
// at most kAutoMaxParts. Measured one-box forwards (ms, 1 / 2 / 3 groups):
// 650M uniform 8 x 256 (T = 2,048) 5.15 / 5.51 / 5.68; 650M config-4 varlen
// (T = 31,107) 41.7 / 40.9 / 41.6; 3B config 5 (T = 20,321) 92.9 / 90.2 /
// 89.4. Fewer tokens per group shrink every GEMM's grid; more groups let one
// group's GEMMs run beside another's attention and row kernels.
int auto_part_count(const esm_gfx950_model_config& c, int T) {
  const double work = 24.0 * static_cast<double>(T) * c.hidden_size * c.hidden_size;
  const int n = static_cast<int>(work / 6e11);
  return std::max(1, std::min(n, kAutoMaxParts));
}

// Validates and stages a packed batch in at most max_parts sequence groups.
int stage_batch(esm_gfx950_ctx* ctx, esm_gfx950_model* m, const int32_t* ids, const int32_t* cu, int B, int T,
                int max_parts, const int32_t* masks = nullptr) {
  ESM_TRY(validate_batch(ctx, cu, B, T));
  m->staged_T = 0;
  for (auto& p : m->parts) p.T = p.B = 0;
  if (T == 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, ids, "batch_upload: null ids");
  const int V = m->cfg.vocab_size;
  for (int t = 0; t < T; ++t)
    if (ids[t] < 0 || ids[t] >= V)
      return ctx->fail(ESM_GFX950_OUT_OF_RANGE, "forward_packed: token id out of range at " + std::to_string(t));
  // Contiguous sequence groups of about T / parts tokens each (never empty).
  // A per-tensor activation scale spans the whole batch, so that mode keeps
  // the batch in one part.
  const bool whole = m->cfg.weights_int8 && (m->cfg.act_quant_mode == ESM_GFX950_ACT_PER_TENSOR ||
                                            m->numerics != ESM_GFX950_NUMERICS_DEFAULT);
  int np = whole ? 1 : std::min({static_cast<int>(m->parts.size()), B, max_parts});
  if (m->auto_parts) np = std::min(np, auto_part_count(m->cfg, T));
  int b0 = 0;
  for (int p = 0; p < np; ++p) {
    int b1 = b0 + 1;
    const long target = static_cast<long>(T) * (p + 1) / np;
    while (b1 < B - (np - 1 - p) && cu[b1] < target) ++b1;
    if (p == np - 1) b1 = B;
    ESM_TRY(stage_part(ctx, m, m->parts[p], ids, masks, cu, b0, b1 - b0));
    b0 = b1;
  }
  m->staged_T = T;
  return ESM_GFX950_OK;
}

// Part 0 runs on the context stream itself (no own stream); parts 1.. with
// work wait for what is queued there so far ...
int fork_parts(esm_gfx950_ctx* ctx, esm_gfx950_model* m) {
  esm_gfx950_model::Part& P0 = m->parts[0];
  ESM_HIP(ctx, hipEventRecord(P0.done, ctx->stream));
  for (size_t i = 1; i < m->parts.size(); ++i)
    if (m->parts[i].T > 0) ESM_HIP(ctx, hipStreamWaitEvent(m->parts[i].stream, P0.done, 0));
  return ESM_GFX950_OK;
}

// ... and the context stream waits for their last work.
int join_parts(esm_gfx950_ctx* ctx, esm_gfx950_model* m) {
  for (size_t i = 1; i < m->parts.size(); ++i) {
    esm_gfx950_model::Part& P = m->parts[i];
    if (P.T == 0) continue;
    ESM_HIP(ctx, hipEventRecord(P.done, P.stream));
    ESM_HIP(ctx, hipStreamWaitEvent(ctx->stream, P.done, 0));
  }
  return ESM_GFX950_OK;
}

}  // namespace

extern "C" int esm_gfx950_batch_upload(esm_gfx950_ctx* ctx, esm_gfx950_model* m, const int32_t* ids,
                                       const int32_t* cu, int B, int T) {
  if (!ctx || !m) return ESM_GFX950_INVALID_ARGUMENT;
  return stage_batch(ctx, m, ids, cu, B, T, static_cast<int>(m->parts.size()));
}

extern "C" int esm_gfx950_batch_upload_masked(esm_gfx950_ctx* ctx, esm_gfx950_model* m, const int32_t* ids,
                                              const int32_t* masks, const int32_t* cu, int B, int T) {
  if (!ctx || !m) return ESM_GFX950_INVALID_ARGUMENT;
  return stage_batch(ctx, m, ids, cu, B, T, static_cast<int>(m->parts.size()), masks);
}

extern "C" int esm_gfx950_forward_device(esm_gfx950_ctx* ctx, esm_gfx950_model* m, float* logits) {
  if (!ctx || !m) return ESM_GFX950_INVALID_ARGUMENT;
  if (m->staged_T == 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, logits, "forward_device: null logits");
  const int V = m->cfg.vocab_size;
  if (m->parts.size() == 1 || m->parts[1].T == 0) return forward_part(ctx, m, m->parts[0], logits);
  ESM_REQUIRE(ctx,
              !(m->cfg.weights_int8 && (m->cfg.act_quant_mode == ESM_GFX950_ACT_PER_TENSOR ||
                                        m->numerics != ESM_GFX950_NUMERICS_DEFAULT)) ||
                  m->parts[1].T == 0,
              "forward_device: batch staged in several parts before the switch to per-tensor scales; upload it again");
  // Fork: part 0 runs on the context stream; every other part's stream
  // waits for the work queued so far there, runs its forward, and the
  // context stream joins them.
  ESM_TRY(fork_parts(ctx, m));
  for (auto& P : m->parts) {
    if (P.T == 0) continue;
    StreamScope scope(ctx, P.stream);
    ESM_TRY(forward_part(ctx, m, P, logits + static_cast<size_t>(P.t0) * V));
  }
  return join_parts(ctx, m);
}

extern "C" int esm_gfx950_forward_packed(esm_gfx950_ctx* ctx, esm_gfx950_model* m, const int32_t* ids,
                                         const int32_t* cu, int B, int T, float* logits, int logits_on_device) {
  return esm_gfx950_forward_packed_masked(ctx, m, ids, nullptr, cu, B, T, logits, logits_on_device);
}

extern "C" int esm_gfx950_forward_packed_masked(esm_gfx950_ctx* ctx, esm_gfx950_model* m, const int32_t* ids,
                                                const int32_t* masks, const int32_t* cu, int B, int T,
                                                float* logits, int logits_on_device) {
  if (!ctx || !m) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_TRY(esm_gfx950_batch_upload_masked(ctx, m, ids, masks, cu, B, T));
  if (T == 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, logits, "forward_packed: null logits");
  if (logits_on_device) return esm_gfx950_forward_device(ctx, m, logits);
  // Host logits: each part writes its rows into its own arena, then one
  // device-to-host copy per part after the join.
  const int V = m->cfg.vocab_size;
  if (m->parts.size() == 1 || m->parts[1].T == 0) {
    const esm_gfx950_model::Part& P = m->parts[0];
    const Arena a = part_arena(m, P);
    ESM_TRY(forward_part(ctx, m, P, a.logits));
    ESM_HIP(ctx, hipMemcpyAsync(logits, a.logits, static_cast<size_t>(T) * V * 4, hipMemcpyDeviceToHost, ctx->stream));
  } else {
    ESM_TRY(fork_parts(ctx, m));
    for (auto& P : m->parts) {
      if (P.T == 0) continue;
      StreamScope scope(ctx, P.stream);
      const Arena a = part_arena(m, P);
      ESM_TRY(forward_part(ctx, m, P, a.logits));
      ESM_HIP(ctx, hipMemcpyAsync(logits + static_cast<size_t>(P.t0) * V, a.logits, static_cast<size_t>(P.T) * V * 4,
                                  hipMemcpyDeviceToHost, ctx->stream));
    }
    ESM_TRY(join_parts(ctx, m));
  }
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_forward_hidden_states(esm_gfx950_ctx* ctx, esm_gfx950_model* m, const int32_t* ids,
                                                const int32_t* masks, const int32_t* cu, int B, int T, float* logits,
                                                float* hidden) {
  if (!ctx || !m) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_TRY(esm_gfx950_batch_upload_masked(ctx, m, ids, masks, cu, B, T));
  if (T == 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, logits && hidden, "forward_hidden_states: null logits or hidden");
  const int V = m->cfg.vocab_size, d = m->cfg.hidden_size;
  const size_t states = m->layers.size() + 1, Td = static_cast<size_t>(T) * d;
  float* dev_hidden = nullptr;
  ESM_HIP(ctx, hipMalloc(&dev_hidden, states * Td * 4));
  auto run = [&]() -> int {
    const bool several = m->parts.size() > 1 && m->parts[1].T > 0;
    if (several) ESM_TRY(fork_parts(ctx, m));
    for (auto& P : m->parts) {
      if (P.T == 0) continue;
      StreamScope scope(ctx, several ? P.stream : ctx->stream);
      const Arena a = part_arena(m, P);
      HiddenCapture cap{dev_hidden + static_cast<size_t>(P.t0) * d, Td};
      ESM_TRY(forward_part(ctx, m, P, a.logits, nullptr, &cap));
      ESM_HIP(ctx, hipMemcpyAsync(logits + static_cast<size_t>(P.t0) * V, a.logits, static_cast<size_t>(P.T) * V * 4,
                                  hipMemcpyDeviceToHost, ctx->stream));
    }
    if (several) ESM_TRY(join_parts(ctx, m));
    ESM_HIP(ctx, hipMemcpyAsync(hidden, dev_hidden, states * Td * 4, hipMemcpyDeviceToHost, ctx->stream));
    ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return ESM_GFX950_OK;
  };
  const int rc = run();
  if (rc != ESM_GFX950_OK) hipStreamSynchronize(ctx->stream);
  hipFree(dev_hidden);
  return rc;
}

// ---------------------------------------------------------------- observer
namespace {

// Device and pinned staging for `nsites` sites' reservoir slots.
int reserve_observer(esm_gfx950_ctx* ctx, esm_gfx950_observer* o, size_t nsites) {
  if (nsites <= o->cap_sites) return ESM_GFX950_OK;
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  if (o->d_pos) hipFree(o->d_pos);
  if (o->d_val) hipFree(o->d_val);
  if (o->h_pos) hipHostFree(o->h_pos);
  if (o->h_val) hipHostFree(o->h_val);
  o->d_pos = o->h_pos = nullptr;
  o->d_val = o->h_val = nullptr;
  o->cap_sites = 0;
  const size_t n = nsites * obs::kReservoirSize;
  ESM_HIP(ctx, hipMalloc(&o->d_pos, n * 4));
  ESM_HIP(ctx, hipMalloc(&o->d_val, n * 4));
  ESM_HIP(ctx, hipHostMalloc(&o->h_pos, n * 4, hipHostMallocDefault));
  ESM_HIP(ctx, hipHostMalloc(&o->h_val, n * 4, hipHostMallocDefault));
  o->cap_sites = nsites;
  return ESM_GFX950_OK;
}

void free_observer_buffers(esm_gfx950_observer* o) {
  if (o->d_pos) hipFree(o->d_pos);
  if (o->d_val) hipFree(o->d_val);
  if (o->h_pos) hipHostFree(o->h_pos);
  if (o->h_val) hipHostFree(o->h_val);
  o->d_pos = o->h_pos = nullptr;
  o->d_val = o->h_val = nullptr;
  o->cap_sites = 0;
}

// Site keys in the order TransformerBlock observes them.
constexpr const char* kObsSites[4] = {"attn_ln_output", "attn_out", "ffn_ln_output", "inter_gelu"};

}  // namespace

extern "C" int esm_gfx950_observer_create(esm_gfx950_ctx* ctx, esm_gfx950_observer** out) {
  if (!ctx || !out) return ESM_GFX950_INVALID_ARGUMENT;
  *out = new (std::nothrow) esm_gfx950_observer();
  return *out ? ESM_GFX950_OK : ctx->fail(ESM_GFX950_INTERNAL, "observer_create: out of memory");
}

extern "C" int esm_gfx950_observer_free(esm_gfx950_ctx* ctx, esm_gfx950_observer* obs) {
  if (!ctx) return ESM_GFX950_INVALID_ARGUMENT;
  if (!obs) return ESM_GFX950_OK;
  ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
  free_observer_buffers(obs);
  delete obs;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_observer_clear(esm_gfx950_observer* obs) {
  if (!obs) return ESM_GFX950_INVALID_ARGUMENT;
  obs->sites.clear();
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_observer_site_count(const esm_gfx950_observer* obs, size_t* count) {
  if (!obs || !count) return ESM_GFX950_INVALID_ARGUMENT;
  *count = obs->sites.size();
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_observer_site_name(const esm_gfx950_observer* obs, size_t i, const char** name) {
  if (!obs || !name) return ESM_GFX950_INVALID_ARGUMENT;
  if (i >= obs->sites.size()) return ESM_GFX950_OUT_OF_RANGE;
  auto it = obs->sites.begin();
  std::advance(it, static_cast<std::ptrdiff_t>(i));
  *name = it->first.c_str();
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_observer_percentile(const esm_gfx950_observer* obs, const char* site, float pctile,
                                              float* out) {
  if (!obs || !site || !out || std::isnan(pctile)) return ESM_GFX950_INVALID_ARGUMENT;
  auto it = obs->sites.find(site);
  if (it == obs->sites.end()) return ESM_GFX950_NOT_FOUND;
  try {
    *out = obs::percentile(it->second, pctile);
  } catch (const std::exception&) {
    return ESM_GFX950_INTERNAL;
  }
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_observer_observe(esm_gfx950_ctx* ctx, esm_gfx950_observer* obs, const char* site,
                                           const float* values, size_t n) {
  if (!ctx || !obs) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, site, "observer_observe: null site key");
  if (n == 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, values, "observer_observe: null values");
  if (n >= UINT32_MAX) return ctx->fail(ESM_GFX950_OUT_OF_RANGE, "observer_observe: more than 2^32 - 2 values");
  ESM_TRY(reserve_observer(ctx, obs, 1));
  // Planned on a copy of the site's reservoir; the copy replaces the site
  // only once the gathered values are in, so a failed call changes nothing.
  size_t count = 0;
  std::vector<uint32_t> slots;
  obs::Reservoir r;
  try {
    auto it = obs->sites.find(site);
    if (it != obs->sites.end()) r = it->second;
    slots.resize(obs::kReservoirSize);
    count = obs::plan(r, n, slots.data(), obs->h_pos);
  } catch (const std::exception& e) {
    return ctx->fail(ESM_GFX950_INTERNAL, std::string("observer_observe: ") + e.what());
  }
  if (count > 0) {
    ESM_HIP(ctx, hipMemcpyAsync(obs->d_pos, obs->h_pos, count * 4, hipMemcpyHostToDevice, ctx->stream));
    ESM_HIP(ctx, launch_observe_gather(values, obs->d_pos, static_cast<int>(count), 0, obs->d_val, ctx->stream));
    ESM_HIP(ctx, hipMemcpyAsync(obs->h_val, obs->d_val, count * 4, hipMemcpyDeviceToHost, ctx->stream));
    ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (size_t w = 0; w < count; ++w) r.samples[slots[w]] = obs->h_val[w];
  }
  try {
    obs->sites[site] = std::move(r);
  } catch (const std::exception& e) {
    return ctx->fail(ESM_GFX950_INTERNAL, std::string("observer_observe: ") + e.what());
  }
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_forward_with_observer(esm_gfx950_ctx* ctx, esm_gfx950_model* m, const int32_t* ids,
                                                const int32_t* cu, int B, int T, float* logits,
                                                esm_gfx950_observer* obs) {
  if (!ctx || !m) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, obs, "forward_with_observer: null observer");
  // The observer sees each site's values in packed row order, so the batch
  // is staged as one sequence group.
  ESM_TRY(stage_batch(ctx, m, ids, cu, B, T, 1));
  if (T == 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, logits, "forward_with_observer: null logits");
  const auto& c = m->cfg;
  const size_t Td = static_cast<size_t>(T) * c.hidden_size, Tf = static_cast<size_t>(T) * c.intermediate_size;
  if (Tf >= UINT32_MAX) return ctx->fail(ESM_GFX950_OUT_OF_RANGE, "forward_with_observer: batch too large");
  const size_t nsites = 4 * m->layers.size();
  ESM_TRY(reserve_observer(ctx, obs, nsites));
  // The reservoirs advance while the forward runs (the host plans each
  // site ahead of the device); a call that fails part-way puts back the
  // state it started from, so later percentiles are unaffected.
  struct Restore {
    esm_gfx950_observer* o;
    std::map<std::string, obs::Reservoir> before;
    bool done = false;
    ~Restore() {
      if (!done) o->sites.swap(before);
    }
  };
  std::unique_ptr<Restore> restore;
  try {
    restore.reset(new Restore{obs, obs->sites});
  } catch (const std::exception& e) {
    return ctx->fail(ESM_GFX950_INTERNAL, std::string("forward_with_observer: ") + e.what());
  }
  std::vector<ObsSite> sites(nsites);
  try {
    for (size_t l = 0; l < m->layers.size(); ++l)
      for (int k = 0; k < 4; ++k) {
        ObsSite& st = sites[4 * l + k];
        st.r = &obs->sites["layer" + std::to_string(l) + "." + kObsSites[k]];
        st.n = k == 3 ? Tf : Td;
      }
  } catch (const std::exception& e) {
    return ctx->fail(ESM_GFX950_INTERNAL, std::string("forward_with_observer: ") + e.what());
  }
  esm_gfx950_model::Part& P = m->parts[0];
  if (P.stream) {
    ESM_HIP(ctx, hipEventRecord(P.done, ctx->stream));
    ESM_HIP(ctx, hipStreamWaitEvent(P.stream, P.done, 0));
  }
  StreamScope scope(ctx, P.stream);
  ObsRun run(obs, std::move(sites));
  const Arena a = part_arena(m, P);
  const int rc = forward_part(ctx, m, P, a.logits, &run);
  if (rc != ESM_GFX950_OK) {
    // Whatever was enqueued completes before the reservoirs are restored.
    hipStreamSynchronize(ctx->stream);
    return rc;
  }
  ESM_HIP(ctx, hipMemcpyAsync(logits, a.logits, static_cast<size_t>(T) * c.vocab_size * 4, hipMemcpyDeviceToHost,
                              ctx->stream));
  ESM_TRY(run.finish(ctx));
  restore->done = true;
  return ESM_GFX950_OK;
}

// ---------------------------------------------------------------- scheduler
namespace {

// PlanChunk (reference src/sched/scheduler.cpp:13-50): a group whose longest
// sequence exceeds `threshold` times its mean length is sorted by length
// (std::sort, ascending) and split at size/2, and both halves are planned
// again; otherwise it is emitted as one group. Groups of one are emitted.
void plan_group(std::vector<int>& idx, const int32_t* lengths, float threshold, std::vector<std::vector<int>>* out) {
  if (idx.empty()) return;
  if (idx.size() > 1) {
    int longest = 0;
    long sum = 0;
    for (int i : idx) {
      longest = std::max(longest, static_cast<int>(lengths[i]));
      sum += lengths[i];
    }
    const float mean = static_cast<float>(sum) / static_cast<float>(idx.size());
    if (mean > 0.0f && static_cast<float>(longest) / mean > threshold) {
      std::sort(idx.begin(), idx.end(), [&](int a, int b) { return lengths[a] < lengths[b]; });
      const size_t half = idx.size() / 2;
      std::vector<int> shorter(idx.begin(), idx.begin() + static_cast<long>(half));
      std::vector<int> longer(idx.begin() + static_cast<long>(half), idx.end());
      plan_group(shorter, lengths, threshold, out);
      plan_group(longer, lengths, threshold, out);
      return;
    }
  }
  out->push_back(std::move(idx));
}

// PlanBatches (reference src/sched/scheduler.cpp:54-75): caller-order chunks
// of at most max_batch_size (all, when <= 0), each planned by plan_group.
std::vector<std::vector<int>> plan_batches(const int32_t* lengths, int n, float threshold, int max_batch_size) {
  std::vector<std::vector<int>> out;
  const int chunk = max_batch_size > 0 ? max_batch_size : n;
  for (int s = 0; s < n; s += chunk) {
    std::vector<int> idx;
    for (int i = s; i < std::min(n, s + chunk); ++i) idx.push_back(i);
    plan_group(idx, lengths, threshold, &out);
  }
  return out;
}

}  // namespace

extern "C" int esm_gfx950_plan_batches(const int32_t* lengths, int n, float imbalance_threshold,
                                       int max_batch_size, int32_t* order, int32_t* group_sizes,
                                       int* num_groups) {
  if (n < 0 || !num_groups || (n > 0 && (!lengths || !order || !group_sizes))) return ESM_GFX950_INVALID_ARGUMENT;
  for (int i = 0; i < n; ++i)
    if (lengths[i] < 0) return ESM_GFX950_INVALID_ARGUMENT;
  const auto plan = plan_batches(lengths, n, imbalance_threshold, max_batch_size);
  int k = 0, g = 0;
  for (const auto& group : plan) {
    group_sizes[g++] = static_cast<int32_t>(group.size());
    for (int i : group) order[k++] = i;
  }
  *num_groups = g;
  return ESM_GFX950_OK;
}

extern "C" int esm_gfx950_forward_scheduled(esm_gfx950_ctx* ctx, esm_gfx950_model* m, const int32_t* const* ids,
                                            const int32_t* lengths, int n, float imbalance_threshold,
                                            int max_batch_size, float* const* logits) {
  if (!ctx || !m) return ESM_GFX950_INVALID_ARGUMENT;
  ESM_REQUIRE(ctx, n >= 0, "forward_scheduled: negative sequence count");
  if (n == 0) return ESM_GFX950_OK;
  ESM_REQUIRE(ctx, lengths && ids && logits, "forward_scheduled: null argument");
  for (int i = 0; i < n; ++i) {
    ESM_REQUIRE(ctx, lengths[i] >= 0, "forward_scheduled: negative length at " + std::to_string(i));
    ESM_REQUIRE(ctx, lengths[i] == 0 || (ids[i] && logits[i]),
                "forward_scheduled: null ids or logits at " + std::to_string(i));
  }
  const int V = m->cfg.vocab_size;
  const auto plan = plan_batches(lengths, n, imbalance_threshold, max_batch_size);
  size_t need = 0;
  for (const auto& group : plan) {
    size_t t = 0;
    for (int i : group) t += static_cast<size_t>(lengths[i]);
    need = std::max(need, t * V);
  }
  if (need == 0) return ESM_GFX950_OK;  // every sequence is empty
  if (need > m->sched_cap) {
    ESM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (int b = 0; b < 2; ++b) {
      if (m->sched_dev[b]) hipFree(m->sched_dev[b]);
      if (m->sched_host[b]) hipHostFree(m->sched_host[b]);
      m->sched_dev[b] = m->sched_host[b] = nullptr;
    }
    m->sched_cap = 0;
    for (int b = 0; b < 2; ++b) {
      ESM_HIP(ctx, hipMalloc(&m->sched_dev[b], need * 4));
      ESM_HIP(ctx, hipHostMalloc(&m->sched_host[b], need * 4, hipHostMallocDefault));
      if (!m->sched_copied[b]) ESM_HIP(ctx, hipEventCreateWithFlags(&m->sched_copied[b], hipEventDisableTiming));
    }
    m->sched_cap = need;
  }
  // Group g is packed, staged and launched while group g-1 still runs; its
  // logits are then copied to pinned memory, and group g-1's are scattered to
  // the callers' buffers once their copy has landed.
  auto scatter = [&](int g) -> int {
    ESM_HIP(ctx, hipEventSynchronize(m->sched_copied[g & 1]));
    const float* src = m->sched_host[g & 1];
    for (int i : plan[g]) {
      const size_t rows = static_cast<size_t>(lengths[i]) * V;
      std::memcpy(logits[i], src, rows * 4);
      src += rows;
    }
    return ESM_GFX950_OK;
  };
  std::vector<int32_t> packed, cu;
  for (size_t g = 0; g < plan.size(); ++g) {
    const auto& group = plan[g];
    packed.clear();
    cu.assign(1, 0);
    for (int i : group) {
      packed.insert(packed.end(), ids[i], ids[i] + lengths[i]);
      cu.push_back(cu.back() + lengths[i]);
    }
    const int B = static_cast<int>(group.size()), T = cu.back();
    ESM_TRY(esm_gfx950_batch_upload(ctx, m, packed.data(), cu.data(), B, T));
    if (T > 0) {
      ESM_TRY(esm_gfx950_forward_device(ctx, m, m->sched_dev[g & 1]));
      ESM_HIP(ctx, hipMemcpyAsync(m->sched_host[g & 1], m->sched_dev[g & 1], static_cast<size_t>(T) * V * 4,
                                  hipMemcpyDeviceToHost, ctx->stream));
    }
    ESM_HIP(ctx, hipEventRecord(m->sched_copied[g & 1], ctx->stream));
    if (g > 0) ESM_TRY(scatter(static_cast<int>(g) - 1));
  }
  ESM_TRY(scatter(static_cast<int>(plan.size()) - 1));
  return ESM_GFX950_OK;
}

// ---------------------------------------------------------------- GGUF load
// Model::LoadFromGguf (reference src/model.cpp:229-298; tensor names and
// shapes as Model::SaveToGguf writes them, :562-700): metadata esm.* gives
// the shape, esm.weights_quantized selects Q8_ESM ([N, K] int8 + [N] scales,
// wire shape [K, N]) or F32 layer linears; embeddings, LayerNorms, biases and
// the lm head are F32. Vocabulary 33 and mask id 32 are the tokenizer's
// (include/esm_cpp/tokenizer.h:30-31).
extern "C" int esm_gfx950_model_create_from_gguf(esm_gfx950_ctx* ctx, const char* path, int act_quant_mode,
                                                 int attention_mode, esm_gfx950_model** out) {
  if (!ctx || !out) return ESM_GFX950_INVALID_ARGUMENT;
  *out = nullptr;
  ESM_REQUIRE(ctx, path, "model_create_from_gguf: null path");
  gguf::File f;
  std::string err;
  if (!f.open(path, &err)) return ctx->fail(ESM_GFX950_IO_ERROR, err);
  const gguf::Value* arch = f.meta("general.architecture");
  if (!arch || arch->kind != gguf::Value::kString || arch->s != "esm")
    return ctx->fail(ESM_GFX950_INVALID_ARGUMENT,
                     "gguf: not an esm-arch file (general.architecture must be 'esm')");
  auto meta_int = [&](const char* key, int* v) -> int {
    const gguf::Value* x = f.meta(key);
    if (!x) return ctx->fail(ESM_GFX950_NOT_FOUND, std::string("gguf: missing metadata ") + key);
    if (x->kind != gguf::Value::kInt) return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, std::string("gguf: metadata ") + key + " is not int");
    if (x->i <= 0 || x->i > (1 << 20)) return ctx->fail(ESM_GFX950_OUT_OF_RANGE, std::string("gguf: metadata ") + key + " out of range");
    *v = static_cast<int>(x->i);
    return ESM_GFX950_OK;
  };
  auto meta_bool = [&](const char* key) {
    const gguf::Value* x = f.meta(key);
    return x && x->kind == gguf::Value::kBool && x->b;
  };
  esm_gfx950_model_desc desc{};
  esm_gfx950_model_config& c = desc.cfg;
  ESM_TRY(meta_int("esm.block_count", &c.num_layers));
  ESM_TRY(meta_int("esm.embedding_length", &c.hidden_size));
  ESM_TRY(meta_int("esm.feed_forward_length", &c.intermediate_size));
  ESM_TRY(meta_int("esm.attention.head_count", &c.num_heads));
  ESM_TRY(meta_int("esm.rope.dimension_count", &c.head_dim));
  c.layer_norm_eps = 1e-5f;
  if (const gguf::Value* eps = f.meta("esm.attention.layer_norm_epsilon"); eps && eps->kind == gguf::Value::kFloat)
    c.layer_norm_eps = static_cast<float>(eps->f);
  c.vocab_size = 33;
  c.mask_token_id = 32;
  c.weights_int8 = meta_bool("esm.weights_quantized") ? 1 : 0;
  c.act_quant_mode = act_quant_mode;
  c.attention_mode = attention_mode;
  const size_t d = c.hidden_size, ffn = c.intermediate_size, V = c.vocab_size;

  auto f32 = [&](const std::string& name, size_t count, const float** dst) -> int {
    const gguf::Tensor* t = f.tensor(name);
    if (!t) return ctx->fail(ESM_GFX950_NOT_FOUND, "gguf: missing tensor " + name);
    if (t->type != gguf::kF32) return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "gguf: expected F32 for " + name);
    if (t->bytes != count * 4)
      return ctx->fail(ESM_GFX950_SHAPE_MISMATCH, "gguf: " + name + " holds " + std::to_string(t->bytes / 4) +
                                                      " floats, expected " + std::to_string(count));
    if (reinterpret_cast<uintptr_t>(t->data) % 4 != 0)
      return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "gguf: misaligned tensor " + name);
    *dst = reinterpret_cast<const float*>(t->data);
    return ESM_GFX950_OK;
  };
  std::vector<std::vector<float>> scale_copies;  // Q8 scales realigned to 4 bytes when needed
  auto linear = [&](const std::string& name, size_t N, size_t K, esm_gfx950_linear_desc* L) -> int {
    if (!c.weights_int8) return f32(name + ".weight", N * K, &L->w_f32);
    const gguf::Tensor* t = f.tensor(name + ".weight");
    if (!t) return ctx->fail(ESM_GFX950_NOT_FOUND, "gguf: missing tensor " + name + ".weight");
    if (t->type != gguf::kQ8Esm) return ctx->fail(ESM_GFX950_INVALID_ARGUMENT, "gguf: expected Q8_ESM for " + name + ".weight");
    if (t->shape.size() != 2 || t->shape[0] != K || t->shape[1] != N)
      return ctx->fail(ESM_GFX950_SHAPE_MISMATCH, "gguf: Q8_ESM " + name + ".weight shape mismatch");
    L->w_i8 = reinterpret_cast<const int8_t*>(t->data);
    // The scales follow the N*K int8 bytes, so they are 4-byte aligned only
    // when N*K is; otherwise they are copied out.
    const uint8_t* sp = t->data + N * K;
    if (reinterpret_cast<uintptr_t>(sp) % 4 == 0) {
      L->w_scale = reinterpret_cast<const float*>(sp);
    } else {
      scale_copies.emplace_back(N);
      std::memcpy(scale_copies.back().data(), sp, N * 4);
      L->w_scale = scale_copies.back().data();
    }
    return ESM_GFX950_OK;
  };
  std::vector<esm_gfx950_layer_desc> layers(c.num_layers);
  ESM_TRY(f32("token_embd.weight", V * d, &desc.embed));
  for (int i = 0; i < c.num_layers; ++i) {
    esm_gfx950_layer_desc& L = layers[i];
    const std::string b = "blk." + std::to_string(i) + ".";
    ESM_TRY(f32(b + "attn_norm.weight", d, &L.attn_ln_w));
    ESM_TRY(f32(b + "attn_norm.bias", d, &L.attn_ln_b));
    ESM_TRY(linear(b + "attn_q", d, d, &L.q));
    ESM_TRY(linear(b + "attn_k", d, d, &L.k));
    ESM_TRY(linear(b + "attn_v", d, d, &L.v));
    ESM_TRY(linear(b + "attn_output", d, d, &L.out));
    ESM_TRY(f32(b + "attn_q.bias", d, &L.q.bias));
    ESM_TRY(f32(b + "attn_k.bias", d, &L.k.bias));
    ESM_TRY(f32(b + "attn_v.bias", d, &L.v.bias));
    ESM_TRY(f32(b + "attn_output.bias", d, &L.out.bias));
    ESM_TRY(f32(b + "ffn_norm.weight", d, &L.ffn_ln_w));
    ESM_TRY(f32(b + "ffn_norm.bias", d, &L.ffn_ln_b));
    ESM_TRY(linear(b + "ffn_up", ffn, d, &L.fc1));
    ESM_TRY(linear(b + "ffn_down", d, ffn, &L.fc2));
    ESM_TRY(f32(b + "ffn_up.bias", ffn, &L.fc1.bias));
    ESM_TRY(f32(b + "ffn_down.bias", d, &L.fc2.bias));
  }
  desc.layers = layers.data();
  ESM_TRY(f32("enc_norm.weight", d, &desc.final_ln_w));
  ESM_TRY(f32("enc_norm.bias", d, &desc.final_ln_b));
  ESM_TRY(f32("lm_head.weight", d * d, &desc.lm_dense_w));
  ESM_TRY(f32("lm_head.bias", d, &desc.lm_dense_b));
  ESM_TRY(f32("lm_head_norm.weight", d, &desc.lm_ln_w));
  ESM_TRY(f32("lm_head_norm.bias", d, &desc.lm_ln_b));
  ESM_TRY(f32("output.bias", V, &desc.lm_decoder_bias));
  ESM_TRY(esm_gfx950_model_create(ctx, &desc, out));
  (*out)->first_block_fc1_fp16 = meta_bool("esm.first_block_fc1_fp16");
  return ESM_GFX950_OK;
}
