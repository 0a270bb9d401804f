/*
 * esm_gfx950.h -- C ABI of the MI355X (gfx950) backend for the packed ESM-2
 * encoder hot path of esm.cpp: varlen attention with rotary Q/K and the W8A8
 * INT8 linear layers around it.
 *
 * Plain C: opaque handles, plain pointers and sizes, int status codes. No
 * HIP or C++ types appear in the signatures, so the reference's C++ host
 * (src/kernels/dispatch.cpp) can bind it from a new `case Isa::Gfx950:` arm,
 * and Python can bind it with ctypes.
 *
 * Conventions
 *  - Every call returns ESM_GFX950_OK (0) or a status code that mirrors
 *    esm::StatusCode (reference include/esm_cpp/status.h:9-36);
 *    esm_gfx950_last_error() gives the message. Nothing fails silently and
 *    nothing falls back to a CPU path.
 *  - Tensor arguments of the op-level entry points are DEVICE pointers
 *    (esm_gfx950_malloc or any hipMalloc'd memory); batch descriptions
 *    (token ids, cu_seqlens) are HOST arrays, as in the reference's
 *    BatchView (include/esm_cpp/batch.h:16-36).
 *  - A context owns one HIP stream. Calls are stream-ordered and return
 *    after enqueue; esm_gfx950_sync() waits. One context = one forward in
 *    flight, the reference Model's threading contract
 *    (include/esm_cpp/model.h:176-181).
 *  - Layouts are the reference's: row-major, W as [N, K] (out, in),
 *    q/k/v token-major [T, H, head_dim], attention out [T, H*head_dim].
 */
#ifndef ESM_GFX950_H_
#define ESM_GFX950_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: values of esm::StatusCode (status.h:9-17) plus kHipError. */
enum {
  ESM_GFX950_OK = 0,
  ESM_GFX950_INVALID_ARGUMENT = 1,
  ESM_GFX950_OUT_OF_RANGE = 2,
  ESM_GFX950_NOT_FOUND = 3,
  ESM_GFX950_IO_ERROR = 4,
  ESM_GFX950_SHAPE_MISMATCH = 5,
  ESM_GFX950_INTERNAL = 6,
  ESM_GFX950_HIP_ERROR = 7
};

/* Activation quantisation granularity for W8A8 linears.
 * PER_TENSOR reproduces the reference's dynamic per-tensor scale
 * (src/kernels/gemm_int8.cpp:391-508: scale = max|A|/127 over the whole
 * [M,K] input, 1 when all zero); PER_TOKEN uses one such scale per row. */
enum { ESM_GFX950_ACT_PER_TENSOR = 0, ESM_GFX950_ACT_PER_TOKEN = 1 };

/* Attention arithmetic for esm_gfx950_attention_varlen. FP32: scalar fp32
 * kernel in the reference's operation order. BF16_MFMA: q/k rounded to bf16,
 * v and the probabilities to fp16, on MFMA. F16X3_MFMA: fp32 inputs, every
 * operand split into fp16 hi + lo and each product formed by three fp16
 * MFMAs (hi*hi + lo*hi + hi*lo), i.e. fp32-level results at MFMA speed;
 * needs |8*q|, |k|, |v| < 65504 (fp16 range). */
enum { ESM_GFX950_ATTN_FP32 = 0, ESM_GFX950_ATTN_BF16_MFMA = 1, ESM_GFX950_ATTN_F16X3_MFMA = 2 };

/* Attention inside the W8A8 forward. F16X3 (default): the QKV epilogue
 * writes fp32 Q/K/V (Q scaled, RoPE applied) and the split-fp16 MFMA kernel
 * runs -- logits track the reference's fp32 attention. FP16: Q/K/V stored as
 * fp16, single fp16 MFMAs; BF16: Q/K as bf16. Those two halve the Q/K/V
 * traffic but round every attention operand once (about 3e-4 off the logit
 * correlation of a W8A8 network, whose int8 rounding amplifies any
 * perturbation). FP32: fp32 Q/K/V and the scalar fp32 kernel. */
enum {
  ESM_GFX950_ATTN_MODE_FP16 = 0,
  ESM_GFX950_ATTN_MODE_BF16 = 1,
  ESM_GFX950_ATTN_MODE_FP32 = 2,
  ESM_GFX950_ATTN_MODE_F16X3 = 3
};

/* Arithmetic of the whole forward (esm_gfx950_model_set_numerics).
 * DEFAULT: the model's act_quant_mode / attention_mode on the fast kernels.
 * X86_AVX512: the reference's x86 AVX-512 CPU path reproduced bit for bit
 * -- the kernels its facade selects for Isa::Avx512Vnni
 * (src/kernels/dispatch.cpp): LayerNormAvx512, LinearVnni with the dynamic
 * per-tensor activation scale, RopeApplyVarlenAvx512,
 * AttentionVarlenAvx512, GeluAvx512, LinearAvx512 (lm head).
 * X86_AMX: the same for Isa::Amx, whose LinearAmx quantises the last T % 32
 * rows of each input with their own scale (src/kernels/gemm_amx.cpp:
 * 218-309; on shapes its gate admits: T >= 32, N % 32 == 0, K % 64 == 0). */
enum { ESM_GFX950_NUMERICS_DEFAULT = 0, ESM_GFX950_NUMERICS_X86_AVX512 = 1, ESM_GFX950_NUMERICS_X86_AMX = 2 };

typedef struct esm_gfx950_ctx esm_gfx950_ctx;
typedef struct esm_gfx950_weight esm_gfx950_weight;
typedef struct esm_gfx950_model esm_gfx950_model;
typedef struct esm_gfx950_observer esm_gfx950_observer;

/* ---------------------------------------------------------------- context
 * Device selection replaces the ISA probe (reference
 * src/kernels/cpu_features.cpp:69-87, 130-135): a successful init is what
 * makes the gfx950 arm selectable. Fails with ESM_GFX950_HIP_ERROR when no
 * gfx950 device is present. */
int esm_gfx950_init(int device, esm_gfx950_ctx** out);
int esm_gfx950_destroy(esm_gfx950_ctx* ctx);
const char* esm_gfx950_last_error(const esm_gfx950_ctx* ctx);
/* Device name (gcnArchName) of the context's device. */
const char* esm_gfx950_device_arch(const esm_gfx950_ctx* ctx);
int esm_gfx950_sync(esm_gfx950_ctx* ctx);

/* Device memory and copies (plumbing for callers without their own HIP). */
int esm_gfx950_malloc(esm_gfx950_ctx* ctx, size_t bytes, void** dptr);
int esm_gfx950_free(esm_gfx950_ctx* ctx, void* dptr);
int esm_gfx950_memcpy_h2d(esm_gfx950_ctx* ctx, void* dst, const void* src, size_t bytes);
int esm_gfx950_memcpy_d2h(esm_gfx950_ctx* ctx, void* dst, const void* src, size_t bytes);
int esm_gfx950_memcpy_d2d(esm_gfx950_ctx* ctx, void* dst, const void* src, size_t bytes);

/* Stream-ordered timer: start/stop record HIP events on the context stream;
 * elapsed is read after the stop event completes. */
int esm_gfx950_timer_start(esm_gfx950_ctx* ctx);
int esm_gfx950_timer_stop(esm_gfx950_ctx* ctx, float* elapsed_ms);

/* Per-kernel timing: while enabled, every launch of a timed site inside the
 * forward -- "qkv", "attention", "out", "fc1", "fc2" (INT8 GEMMs and the
 * attention kernel), "lm_dense", and in per-token W8A8 mode the row kernels
 * "ln_quant" (residual + LayerNorm + quant), "ln_quant_first" (the first
 * layer's, with no residual), "attn_quant", "gelu_quant" -- and of
 * esm_gfx950_attention_varlen_bf16 ("attention") is bracketed by HIP events
 * on the context stream. Enabling (or disabling) resets the record; the
 * query returns the number of timed launches of `site` and their summed
 * duration. */
int esm_gfx950_kernel_timing(esm_gfx950_ctx* ctx, int enable);
int esm_gfx950_kernel_timing_query(esm_gfx950_ctx* ctx, const char* site, int* launches, double* total_ms);

/* ------------------------------------------------------- weights (L2 pack)
 * Upload a per-channel symmetric INT8 weight: packed [N, K] int8 in
 * [-127, 127] and per_channel_scales [N] (host pointers) -- the
 * esm::quant::QuantizedTensor contents (reference include/esm_cpp/quant.h:
 * 17-56, produced by Quantize src/quant/pack.cpp:149-177). Builds the
 * device-resident gfx950 cache (rows padded to a 16-byte K pitch), the
 * analogue of BuildKernelCache (pack.cpp:107-117). */
int esm_gfx950_weight_upload_i8(esm_gfx950_ctx* ctx, const int8_t* packed, const float* scales,
                                int N, int K, esm_gfx950_weight** out);
int esm_gfx950_weight_free(esm_gfx950_ctx* ctx, esm_gfx950_weight* w);

/* --------------------------------------------------------------- INT8 ops
 * Raw int32 accumulators: C[m, n] = sum_k A[m, k] * W[n, k]. A is int8
 * [M, lda] (lda >= K, lda % 16 == 0), C int32 [M, N]. The bit-exact check
 * of the W8A8 inner product; no reference twin forms int32 (LinearInt8Ref
 * src/kernels/gemm_int8.cpp:49-64 is W8A16), so parity is the closed form. */
int esm_gfx950_gemm_i8_i32(esm_gfx950_ctx* ctx, const int8_t* A, int lda, const esm_gfx950_weight* W,
                           int M, int32_t* C);

/* Row height of the INT8 GEMM's workgroup tile for every later launch in the
 * process: 64, 128, 256, 320, or 0 (default) to pick per launch. The default
 * gives grids that fill the device's CUs the height whose grid needs the
 * fewer rows' worth of workgroup rounds (320 only for the plain dequant,
 * int32 and split-word outputs), and small-M grids 64, 128 or 256 rows by an
 * estimate of their time. Results do not depend on it; it exists for tuning
 * and tests. No reference counterpart. INVALID_ARGUMENT for other values. */
int esm_gfx950_set_gemm_tile_rows(int rows);

/* K splits of the model's out-proj and fc2 INT8 GEMMs for every later launch
 * in the process: 0 (default) chooses per launch, 1 never splits, 2..4 split
 * that many ways. A split grid writes int32 partial sums over contiguous K
 * ranges into the (then unused) FFN intermediate buffer and one pass sums
 * them and applies the dequant epilogue. The automatic choice splits only
 * grids that leave CUs idle (small batches), when the estimated time of the
 * split grid plus that pass is lower. int32 sums are exact, so results are
 * bit-identical for every setting; it exists for tuning and tests. No
 * reference counterpart. INVALID_ARGUMENT for other values. */
int esm_gfx950_set_gemm_split_k(int splits);

/* Quantised-activation linear: out = fma(float(acc), a_scale[m] * w_scale[n], bias[n]),
 * optionally followed by GELU (gelu != 0). The dequant expression of
 * FinalizeStore16 (gemm_int8.cpp:109-126) with a per-row activation scale.
 * A int8 [M, lda], a_scale fp32 [M], bias fp32 [N] or NULL, C fp32 [M, N]. */
int esm_gfx950_linear_i8_q(esm_gfx950_ctx* ctx, const int8_t* A, int lda, const float* a_scale,
                           const esm_gfx950_weight* W, const float* bias, float* C, int M, int gelu);

/* The per-token W8A8 FFN up-projection exactly as the default forward runs
 * it: fc1 (LinearInt8, src/model.cpp:1039-1045), Gelu (:1046-1048,
 * src/kernels/gelu.cpp:30-35) and the per-token quantisation of fc2's input
 * (gemm_int8.cpp:391-508 with one scale per row). fc1's dequantised value
 * fma(float(acc), a_scale[m] * w_scale[n], bias[n]) is rounded to its top 24
 * bits (0x80 added to the bit pattern, the low byte cleared: nearest, ties
 * away from zero; NaN becomes the quiet NaN 0x7fc00000) and stored as two
 * planes, inter_hi uint16 [M, N] (bits 31..16) and inter_lo uint8 of
 * (M + (M & 1)) * N bytes (bits 15..8, row pairs interleaved: byte
 * (m & ~1) N + 4 (p / 2) + 2 (m & 1) + (p & 1) holds row m, position p), in
 * both of which stored position p = 64 g + 2 i + j holds column
 * 64 g + 32 j + i; the GELU + quantisation pass reads them and writes q int8
 * [M, ldq] (zero past N) and q_scale fp32 [M]. A int8 [M, lda], a_scale
 * fp32 [M], bias fp32 [N] or NULL; all device pointers. Requires N % 64 == 0,
 * N <= 10240, K % 128 == 0, lda % 16 == 0, ldq >= N, ldq % 4 == 0. */
int esm_gfx950_linear_i8_gelu_quant_r24(esm_gfx950_ctx* ctx, const int8_t* A, int lda, const float* a_scale,
                                        const esm_gfx950_weight* W, const float* bias, int M, uint16_t* inter_hi,
                                        uint8_t* inter_lo, int8_t* q, int ldq, float* q_scale);

/* Activation quantisation: x fp32 [M, K] -> q int8 [M, ldq] (zero padded
 * past K) and scales fp32 [M] (all equal in PER_TENSOR mode). Reference
 * QuantizeActPrefixAvx512 (gemm_int8.cpp:391-508) / QuantizeActivation-
 * SymmetricRef (src/quant/pack.cpp:134-147). */
int esm_gfx950_quantize_act(esm_gfx950_ctx* ctx, const float* x, int M, int K, int mode, int8_t* q,
                            int ldq, float* scales);

/* The fc1 -> fc2 activation step of the INT8 FFN: kernels::Gelu
 * (include/esm_cpp/kernels.h:35, called at src/model.cpp:1044-1045, the
 * AVX-512 erf approximation of src/kernels/gelu.cpp:69-94) followed by the
 * per-token activation quantisation fc2's LinearInt8 applies to its input,
 * fused: x fp32 [M, K] -> q int8 [M, ldq] (zero padded past K) and scales
 * fp32 [M]. K % 4 == 0, K <= 10240. */
int esm_gfx950_gelu_quantize_act(esm_gfx950_ctx* ctx, const float* x, int M, int K, int8_t* q, int ldq,
                                 float* scales);

/* esm::kernels::LinearInt8 (include/esm_cpp/kernels.h:56-57,
 * dispatch.cpp:80-103): fp32 A [M, K] -> activation quant (mode) -> INT8
 * GEMM -> dequant + bias -> fp32 C [M, N]. M, N or K <= 0 zeroes C as the
 * reference does (gemm_int8.cpp:513-520). */
int esm_gfx950_linear_i8(esm_gfx950_ctx* ctx, const float* A, const esm_gfx950_weight* W,
                         const float* bias, float* C, int M, int N, int K, int act_mode);

/* esm_gfx950_linear_i8 for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): no counterpart in the reference. Same arguments, arithmetic
 * and results as esm_gfx950_linear_i8, but its quantised activations and
 * scales live in a static device array of 64 MiB that every GPU the library
 * runs on holds until the process ends, so it never allocates. Limit:
 * align256(M * pad16(K)) + align256(4 * M) + 256 <= 64 MiB (e.g. M = 30,700
 * at K = 1280); larger calls return ESM_GFX950_OUT_OF_RANGE. All calls on
 * one GPU share the array: calls that overlap on one GPU (contexts on
 * different streams) race. */
int esm_gfx950_linear_i8_noalloc(esm_gfx950_ctx* ctx, const float* A, const esm_gfx950_weight* W,
                                 const float* bias, float* C, int M, int N, int K, int act_mode);

/* ----------------------------------------------------------- FP32 / misc ops
 * esm::kernels::Linear (kernels.h:19-20; LinearRef gemm_fp32.cpp:33-46):
 * C[M, N] = A[M, K] W[N, K]^T + bias (bias may be NULL). */
int esm_gfx950_linear_f32(esm_gfx950_ctx* ctx, const float* A, const float* W, const float* bias,
                          float* C, int M, int N, int K);
/* esm::kernels::LayerNorm (kernels.h:32-33; LayerNormRef layernorm.cpp:23-44). */
int esm_gfx950_layernorm(esm_gfx950_ctx* ctx, const float* x, const float* gamma, const float* beta,
                         float eps, float* out, int num_rows, int d);
/* esm::kernels::Gelu (kernels.h:35; GeluRef gelu.cpp:30-35), exact erf form. */
int esm_gfx950_gelu(esm_gfx950_ctx* ctx, const float* x, float* out, size_t n);
/* esm::kernels::ResidualAddInplace (kernels.h:24): y[i] += x[i]. */
int esm_gfx950_residual_add(esm_gfx950_ctx* ctx, float* y, const float* x, size_t n);
/* esm::kernels::ScaleInplace (kernels.h:29): x[i] *= scale. */
int esm_gfx950_scale(esm_gfx950_ctx* ctx, float* x, size_t n, float scale);

/* esm::kernels::RopeBuildTables (kernels.h:67; rope_tables.cpp:14-29),
 * host-side: cos/sin [seq_len, head_dim] half-then-half tables written to
 * HOST memory with the reference formula. */
int esm_gfx950_rope_build_tables(int seq_len, int head_dim, float* cos_out, float* sin_out);
/* Host only, no counterpart in the reference (whose AttentionVarlen
 * parallelises over (sequence, head) with no work list): the number of
 * attention work items a batch with these cu_seqlens produces (mfma != 0:
 * the MFMA kernels' per-XCD queues of 128-query tiles; 0: the fp32 kernel's
 * list) and the number the model's per-batch metadata region reserves for
 * them (items <= capacity for every valid batch). */
int esm_gfx950_attention_work_items(const int32_t* cu_seqlens, int batch_size, int num_heads, int mfma,
                                    size_t* items, size_t* capacity);
/* esm::kernels::RopeApplyVarlen (kernels.h:84-92; rope.cpp:47-70):
 * x fp32 [T, H, head_dim] rotated in place with device tables cos/sin
 * [max_seqlen, head_dim]; positions restart at each cu_seqlens boundary.
 * cu_seqlens is a HOST array of batch_size + 1 entries. */
int esm_gfx950_rope_apply_varlen(esm_gfx950_ctx* ctx, float* x, const float* cos, const float* sin,
                                 const int* cu_seqlens, int batch_size, int num_heads, int head_dim);

/* esm::kernels::AttentionVarlen (kernels.h:104-121; AttentionVarlenRef
 * attention.cpp:99-144): q, k, v fp32 [T, H, head_dim] (Q pre-scaled),
 * out fp32 [T, H*head_dim]. precision FP32 is the exact path (any
 * head_dim <= 128); BF16_MFMA rounds q/k to bf16 and v to fp16 on device
 * and runs the MFMA kernel (head_dim == 64); F16X3_MFMA runs the split-fp16
 * MFMA kernel on the fp32 inputs directly (head_dim == 64). cu_seqlens is a
 * HOST array. */
int esm_gfx950_attention_varlen(esm_gfx950_ctx* ctx, const float* q, const float* k, const float* v,
                                const int* cu_seqlens, int batch_size, int num_heads, int head_dim,
                                float* out, int precision);
/* The MFMA kernel on bf16 inputs: q, k, v bf16 bits [T, H, 64] (v may be
 * fp16 when v_is_fp16 != 0), out fp32 [T, H*64]. cu_seqlens HOST. */
int esm_gfx950_attention_varlen_bf16(esm_gfx950_ctx* ctx, const uint16_t* q, const uint16_t* k,
                                     const uint16_t* v, int v_is_fp16, const int* cu_seqlens,
                                     int batch_size, int num_heads, float* out);

/* ----------------------------------------------- the reference's x86 kernels
 * Device counterparts of the AVX-512 arms of the reference's facade, equal
 * to them bit for bit (same operation order lane by lane, the same fused
 * multiply-adds, _mm512_reduce_add_ps's tree as GCC builds it). Same
 * arguments as the plain ops above; tensors are DEVICE pointers,
 * cu_seqlens HOST arrays.
 * LayerNormAvx512 (src/kernels/layernorm.cpp:59-149), d <= 2560. */
int esm_gfx950_layernorm_avx512(esm_gfx950_ctx* ctx, const float* x, const float* gamma, const float* beta,
                                float eps, float* out, int num_rows, int d);
/* GeluAvx512 (src/kernels/gelu.cpp:98-148): erf of Abramowitz-Stegun 7.1.26
 * with the file's polynomial exp (which returns garbage for |x| above about
 * 13.2, where its 2^n exponent bits wrap -- reproduced as is). */
int esm_gfx950_gelu_avx512(esm_gfx950_ctx* ctx, const float* x, float* out, size_t n);
/* std::exp as AttentionVarlenAvx512 uses it on a sequence's last L % 16 keys
 * (src/kernels/attention.cpp:376-381): glibc's expf, restated from its
 * published algorithm; equal to glibc 2.35's expf on every float. */
int esm_gfx950_expf_glibc(esm_gfx950_ctx* ctx, const float* x, float* out, size_t n);
/* LinearAvx512 (src/kernels/gemm_fp32.cpp:194-294): C = A W^T + bias. */
int esm_gfx950_linear_f32_avx512(esm_gfx950_ctx* ctx, const float* A, const float* W, const float* bias, float* C,
                                 int M, int N, int K);
/* RopeApplyVarlenAvx512 (src/kernels/rope.cpp:90-152). */
int esm_gfx950_rope_apply_varlen_avx512(esm_gfx950_ctx* ctx, float* x, const float* cos, const float* sin,
                                        const int* cu_seqlens, int batch_size, int num_heads, int head_dim);
/* AttentionVarlenAvx512 (src/kernels/attention.cpp:240-430, 770-811),
 * head_dim 16, 32 or 64. Runs the forward's kernel: the context's op
 * scratch grows to hold every score once, num_heads x sum over sequences of
 * roundup(L, 64) x L floats (391 MB for config 2's 256 sequences of
 * 20 heads). */
int esm_gfx950_attention_varlen_avx512(esm_gfx950_ctx* ctx, const float* q, const float* k, const float* v,
                                       const int* cu_seqlens, int batch_size, int num_heads, int head_dim,
                                       float* out);

/* ------------------------------------------------------------------ model
 * Forward-level fast path: the device-resident replacement of
 * Model::ForwardPackedInto (reference src/model.cpp:1093-1255, layer body
 * TransformerBlock :932-1066). Host pointers in the descriptors are read
 * once at create time; weights then live on the device. */
typedef struct {
  int num_layers;
  int hidden_size;
  int num_heads;
  int head_dim;
  int intermediate_size;
  int vocab_size;
  float layer_norm_eps;
  int mask_token_id;   /* 32 for ESM-2 (src/tokenizer.cpp:12-17) */
  int weights_int8;    /* 1: W8A8 layer linears; 0: fp32 layer linears */
  int act_quant_mode;  /* ESM_GFX950_ACT_PER_TENSOR / _PER_TOKEN */
  int attention_mode;  /* W8A8 models: ESM_GFX950_ATTN_MODE_* */
} esm_gfx950_model_config;

typedef struct {
  const float* w_f32;    /* [N, K] fp32 (weights_int8 == 0) */
  const int8_t* w_i8;    /* [N, K] int8 (weights_int8 == 1) */
  const float* w_scale;  /* [N] per-channel scales (weights_int8 == 1) */
  const float* bias;     /* [N] */
} esm_gfx950_linear_desc;

typedef struct {
  const float* attn_ln_w;
  const float* attn_ln_b;
  esm_gfx950_linear_desc q, k, v, out;
  const float* ffn_ln_w;
  const float* ffn_ln_b;
  esm_gfx950_linear_desc fc1, fc2;
} esm_gfx950_layer_desc;

typedef struct {
  esm_gfx950_model_config cfg;
  const float* embed;                  /* [vocab, hidden]; also the tied decoder */
  const esm_gfx950_layer_desc* layers; /* [num_layers] */
  const float* final_ln_w;
  const float* final_ln_b;
  const float* lm_dense_w;             /* [hidden, hidden] fp32 */
  const float* lm_dense_b;
  const float* lm_ln_w;
  const float* lm_ln_b;
  const float* lm_decoder_bias;        /* [vocab] */
} esm_gfx950_model_desc;

int esm_gfx950_model_create(esm_gfx950_ctx* ctx, const esm_gfx950_model_desc* desc,
                            esm_gfx950_model** out);
int esm_gfx950_model_free(esm_gfx950_ctx* ctx, esm_gfx950_model* model);
/* Model::SetFirstBlockFc1Fp16 (reference include/esm_cpp/model.h:228-230):
 * when enabled, layer 0's fc1 input (the ffn LayerNorm output) is rounded to
 * the nearest fp16 and back before it is quantised or multiplied
 * (src/model.cpp:1028-1033). Off by default. */
int esm_gfx950_model_set_first_block_fc1_fp16(esm_gfx950_ctx* ctx, esm_gfx950_model* model, int enabled);
/* Width of the per-token W8A8 FFN intermediate, 24 (default) or 32 bits. No
 * counterpart in the reference, whose fc1 output stays an fp32 array until
 * Gelu and the next LinearInt8 quantise it (src/model.cpp:1036-1052). At 24
 * fc1's GEMM stores each output rounded to its top 24 bits (sign, exponent,
 * 15 mantissa bits; nearest, ties away from zero) and the GELU + per-token
 * quantisation pass reads those: 3 bytes per value instead of 4 each way. An
 * int8 code can then differ by one from the fp32 intermediate's only where
 * the rounding (relative 2^-16 at most) crosses a quantisation midpoint.
 * Per-tensor mode and the x86 numerics keep fp32; observed forwards keep the
 * setting. */
int esm_gfx950_model_set_ffn_intermediate_bits(esm_gfx950_ctx* ctx, esm_gfx950_model* model, int bits);
/* Model::LoadFromGguf (reference src/model.cpp:229-298): creates a model
 * from an esm.cpp GGUF v3 file (src/io/gguf.cpp) -- esm.* metadata for the
 * shape; Q8_ESM layer linears ([N, K] int8 + [N] fp32 scales) when
 * esm.weights_quantized is true, else F32; F32 embeddings, LayerNorms,
 * biases and lm head. act_quant_mode / attention_mode as in
 * esm_gfx950_model_config. The file is memory-mapped and released before
 * return. Errors: IO_ERROR (open / malformed file, the reference reader's
 * messages), NOT_FOUND (missing tensor or metadata), INVALID_ARGUMENT (not
 * an esm file, wrong tensor type), SHAPE_MISMATCH (tensor size against the
 * metadata). esm.first_block_fc1_fp16 = true enables that escape. */
int esm_gfx950_model_create_from_gguf(esm_gfx950_ctx* ctx, const char* path, int act_quant_mode,
                                      int attention_mode, esm_gfx950_model** out);
/* ESM_GFX950_NUMERICS_*: X86_AVX512 (X86_AMX) makes every later forward
 * reproduce the reference's ForwardPackedInto on an AVX-512-VNNI (AMX) host
 * bit for bit: same logits, every bit, as that CPU path on the same weights
 * and batch. W8A8 models then quantise activations per tensor whatever
 * their act_quant_mode, and run as one sequence group. head_dim must be 16,
 * 32 or 64 and hidden_size <= 2560. Switching drops the staged batch
 * (upload it again). Reference counterpart: ESM_FORCE_ISA=avx512vnni / amx
 * (src/kernels/cpu_features.cpp:130-135). */
int esm_gfx950_model_set_numerics(esm_gfx950_ctx* ctx, esm_gfx950_model* model, int numerics);
/* Switch the activation quantisation mode of a W8A8 model. */
int esm_gfx950_model_set_act_mode(esm_gfx950_ctx* ctx, esm_gfx950_model* model, int act_mode);

/* Packed forward. ids [T] and cu_seqlens [batch_size + 1] are HOST arrays
 * validated like BatchView (batch.cpp:8-46); every token is real (pads:
 * esm_gfx950_forward_packed_masked). logits fp32 [T, vocab] is written to DEVICE memory when
 * logits_on_device != 0, else to HOST memory (the call then synchronises).
 * Equivalent to esm_gfx950_batch_upload + esm_gfx950_forward_device.
 * The device arena grows only when T exceeds every earlier batch. */
int esm_gfx950_forward_packed(esm_gfx950_ctx* ctx, esm_gfx950_model* model, const int32_t* ids,
                              const int32_t* cu_seqlens, int batch_size, int total_tokens,
                              float* logits, int logits_on_device);
/* Model::ForwardWithHiddenStates / ForwardPackedInto's hidden_packed_out
 * (include/esm_cpp/model.h:184-191, src/model.cpp:1149-1189): the packed
 * forward of esm_gfx950_forward_packed_masked with HOST ids, masks (or NULL),
 * cu_seqlens and logits
 * [T, vocab], that also writes every hidden state to HOST hidden
 * [num_layers + 1, T, hidden_size]: [0] after the embedding, [i] after layer
 * i, and [num_layers] the post-final-LayerNorm state in place of the last
 * layer's output. The logits equal esm_gfx950_forward_packed's (the layers
 * add fc2's output into the hidden state in its GEMM; split-K partial sums
 * are not carried across a layer boundary in this call). Synchronises. */
int esm_gfx950_forward_hidden_states(esm_gfx950_ctx* ctx, esm_gfx950_model* model, const int32_t* ids,
                                     const int32_t* masks, const int32_t* cu_seqlens, int batch_size,
                                     int total_tokens, float* logits, float* hidden);
/* esm_gfx950_forward_packed with BatchView's packed_masks (batch.h:16-36):
 * masks HOST int32 [T] or NULL (every token real); a 0 marks a pad. As in
 * the reference's Embed (src/model.cpp:737-778), a pad's embedding row is
 * zero and only real tokens count towards a sequence's length in the
 * token-dropout ratio; nothing else changes (the attention takes no mask,
 * AttentionVarlen, kernels.h:104-118). */
int esm_gfx950_forward_packed_masked(esm_gfx950_ctx* ctx, esm_gfx950_model* model, const int32_t* ids,
                                     const int32_t* masks, const int32_t* cu_seqlens, int batch_size,
                                     int total_tokens, float* logits, int logits_on_device);
/* Stages a packed batch in the model's device buffers: ids, per-token
 * embedding scale, in-sequence positions, cu_seqlens, the attention work
 * list and the RoPE tables (one pinned host-to-device copy). */
int esm_gfx950_batch_upload(esm_gfx950_ctx* ctx, esm_gfx950_model* model, const int32_t* ids,
                            const int32_t* cu_seqlens, int batch_size, int total_tokens);
/* The same with pad masks (HOST int32 [T] or NULL), as in
 * esm_gfx950_forward_packed_masked. */
int esm_gfx950_batch_upload_masked(esm_gfx950_ctx* ctx, esm_gfx950_model* model, const int32_t* ids,
                                   const int32_t* masks, const int32_t* cu_seqlens, int batch_size,
                                   int total_tokens);
/* Runs the forward on the staged batch with every input already in HBM;
 * logits fp32 [T, vocab] go to DEVICE memory. Stream-ordered, no host sync. */
int esm_gfx950_forward_device(esm_gfx950_ctx* ctx, esm_gfx950_model* model, float* logits);
/* Splits every later staged batch into `parts` (1..4) contiguous groups of
 * whole sequences with about equal token counts; each group gets its own
 * arena, group 0 runs on the context stream and every other group on a HIP
 * stream of its own (default priority) that forward_device forks from / joins
 * back to the context stream, so the groups' kernels run concurrently on
 * different CUs. parts = 0 (every new model's setting)
 * chooses per batch: one group per 6e11 int8 operations of a layer's four
 * linears (24 T d^2 for T tokens), between 1 and 3 -- small batches keep
 * whole GEMM grids, large ones overlap one group's GEMMs with another's
 * attention. Per-tensor activation scales and the x86 numerics always take
 * one group. Results are identical for every count (every row depends only
 * on its own sequence). No reference counterpart: the reference's
 * ForwardPacked (model.cpp:1093-1255) runs one thread pool. */
int esm_gfx950_model_set_parts(esm_gfx950_ctx* ctx, esm_gfx950_model* model, int parts);
/* The model's configuration as created (Model::config, model.h:174). */
int esm_gfx950_model_get_config(const esm_gfx950_model* model, esm_gfx950_model_config* out);
/* The number of groups the last staged batch was split into (0 when none is
 * staged). No reference counterpart. */
int esm_gfx950_model_staged_parts(const esm_gfx950_model* model, int* parts);
/* PlanBatches (reference src/sched/scheduler.cpp:54-75, SchedulerConfig in
 * include/esm_cpp/scheduler.h:8-21), host only: splits n sequences of the
 * given lengths into caller-order chunks of at most max_batch_size (all when
 * <= 0); a chunk whose max/mean length exceeds imbalance_threshold is sorted
 * by length and halved recursively. Writes the caller indices of every group
 * back to back into order[n], the group sizes into group_sizes[n], and the
 * group count into *num_groups. */
int esm_gfx950_plan_batches(const int32_t* lengths, int n, float imbalance_threshold, int max_batch_size,
                            int32_t* order, int32_t* group_sizes, int* num_groups);
/* Model::ForwardScheduled (reference src/model.cpp:1298-1421) without masks:
 * plans the n sequences (ids[i], lengths[i]; HOST arrays) with
 * esm_gfx950_plan_batches, runs each group as one packed forward and writes
 * sequence i's logits fp32 [lengths[i], vocab] to the HOST buffer logits[i].
 * Group g+1 is packed and staged while group g runs, and group g's logits are
 * copied out through pinned memory while group g+1 runs. Returns after the
 * last group's logits are written. */
int esm_gfx950_forward_scheduled(esm_gfx950_ctx* ctx, esm_gfx950_model* model, const int32_t* const* ids,
                                 const int32_t* lengths, int n, float imbalance_threshold, int max_batch_size,
                                 float* const* logits);
/* ------------------------------------------------------ activation observer
 * esm::ActivationObserver (reference include/esm_cpp/observer.h:13-47,
 * src/quant/observer.cpp:8-51) for static-quantisation calibration on the
 * device: per site key, a reservoir of at most 65536 |values| kept by
 * Algorithm R with the reference's generator (std::mt19937 seeded 0xc1b1ce
 * per site, std::uniform_int_distribution over [0, total_seen]), so that the
 * same sequence of calls keeps the same positions. The host draws which
 * positions survive; only those values are gathered from the device. Not
 * thread-safe (one call at a time, like the reference). A call that fails
 * leaves every site as it was before the call. */
int esm_gfx950_observer_create(esm_gfx950_ctx* ctx, esm_gfx950_observer** out);
int esm_gfx950_observer_free(esm_gfx950_ctx* ctx, esm_gfx950_observer* obs);
/* ActivationObserver::Clear (observer.cpp:51): every site removed. */
int esm_gfx950_observer_clear(esm_gfx950_observer* obs);
/* ActivationObserver::Observe (observer.cpp:8-30): feeds |values[0, n)| (fp32,
 * DEVICE memory, n < 2^32 - 1) into site's reservoir; n == 0 is a no-op that
 * creates no site. Returns after the reservoir is updated. */
int esm_gfx950_observer_observe(esm_gfx950_ctx* ctx, esm_gfx950_observer* obs, const char* site,
                                const float* values, size_t n);
/* The sites observed so far, in byte order of their keys. The name pointer
 * stays valid until the observer is cleared or freed. */
int esm_gfx950_observer_site_count(const esm_gfx950_observer* obs, size_t* count);
int esm_gfx950_observer_site_name(const esm_gfx950_observer* obs, size_t i, const char** name);
/* ActivationObserver::Percentile (observer.cpp:32-49) for one site: the
 * sample at floor(clamp(pctile / 100, 0, 1) * (size - 1)) of the sorted
 * reservoir (float arithmetic as the reference). NOT_FOUND for an unknown
 * site; NaN pctile is INVALID_ARGUMENT. */
int esm_gfx950_observer_percentile(const esm_gfx950_observer* obs, const char* site, float pctile, float* out);
/* Model::ForwardPackedInto with an observer (reference src/model.cpp:1093-1255;
 * Model::ForwardWithObserver :1084-1091 is the B = 1 case): the packed
 * forward of esm_gfx950_forward_packed (HOST ids, cu, logits [T, vocab]) that
 * also observes, per layer i, "layer{i}.attn_ln_output", "layer{i}.attn_out",
 * "layer{i}.ffn_ln_output" (before the first-block fp16 rounding) and
 * "layer{i}.inter_gelu" over the batch's [T, d] / [T, ffn] values in packed
 * row order (model.cpp:952-955,996-999,1023-1026,1047-1050). The batch runs as
 * one sequence group with the model's FFN intermediate width
 * (esm_gfx950_model_set_ffn_intermediate_bits; at 24 bits "inter_gelu" samples
 * GELU of the rounded values the quantisation reads), so its logits equal
 * esm_gfx950_forward_packed's. T == 0 observes nothing. */
int esm_gfx950_forward_with_observer(esm_gfx950_ctx* ctx, esm_gfx950_model* model, const int32_t* ids,
                                     const int32_t* cu_seqlens, int batch_size, int total_tokens, float* logits,
                                     esm_gfx950_observer* obs);
/* The lm head's dense d x d linear (reference src/model.cpp:1209-1215, FP32
 * Linear) on the split-fp16 GEMM (enabled != 0: each operand carried as two
 * fp16 parts, three fp16 MFMA products per multiply, fp32 accumulation) or on
 * fp32 MFMA (0). Both are fp32-accurate; W8A8 models start with the split
 * form, all-fp32 models with fp32 MFMA. INVALID_ARGUMENT when the hidden size
 * is not a multiple of 32 (no split weights). No reference counterpart. */
int esm_gfx950_model_set_lm_dense_split(esm_gfx950_ctx* ctx, esm_gfx950_model* model, int enabled);
/* Bytes currently held by the model's device arena (for zero-growth checks). */
int esm_gfx950_model_arena_bytes(const esm_gfx950_model* model, size_t* bytes);

#ifdef __cplusplus
}
#endif

#endif /* ESM_GFX950_H_ */
