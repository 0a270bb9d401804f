/*
 * oracle.h -- CPU restatement of esm.cpp's packed ESM-2 encoder hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (libesm_gfx950.so, its
 * Python binding) links, loads or calls this code; only tests/, the smoke
 * check and bench.py's cpu_baseline leg use it, as the checker.
 *
 * Each function restates one reference function, cited by file:line
 * relative to the reference tree; arithmetic follows the reference's scalar
 * (*Ref) op order and is compiled with the reference's Release flags, so the
 * compiler forms the same fused multiply-adds the reference build does.
 */
#ifndef ESM_ORACLE_H_
#define ESM_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* int32 accumulators C[m,n] = sum_k A[m,k] * W[n,k] (closed form of the
 * VNNI/AMX inner product after zero-point correction,
 * src/kernels/gemm_int8.cpp:109-126 and src/kernels/gemm_amx.cpp:114-127). */
void or_gemm_i8_i32(const int8_t* A, int lda, const int8_t* W, int ldw, int M, int N, int K, int32_t* C);

/* Dynamic per-tensor activation quantisation (gemm_int8.cpp:391-508):
 * scale = absmax/127 (1 if absmax == 0), q = clamp(rne(x * (1/scale)), +-127).
 * The reference's vector body rounds with cvtps (RNE); its scalar tail uses
 * lround, which differs only on exact .5 ties. */
void or_quant_act_tensor(const float* x, size_t n, int8_t* q, float* scale_out);
/* Per-token variant: the same rule applied to each row of [M, K]. */
void or_quant_act_rows(const float* x, int M, int K, int8_t* q, float* scales);

/* Dequant epilogue of FinalizeStore16 (gemm_int8.cpp:109-126):
 * out = fma(float(acc), w_scale[n] * a_scale[m], bias[n]), then GELU when
 * gelu != 0. bias may be NULL (0). */
void or_dequant(const int32_t* acc, const float* a_scale, const float* w_scale, const float* bias, int M, int N,
                int gelu, float* out);

/* Per-channel weight quantisation (src/quant/pack.cpp:149-177). */
void or_quantize_weight(const float* W, int N, int K, int8_t* q, float* scales);

/* LinearInt8Ref (gemm_int8.cpp:49-64): W8A16, fp32 activations. */
void or_linear_int8_w8a16(const float* A, const int8_t* Wq, const float* scales, const float* bias, float* C, int M,
                          int N, int K);

/* LinearRef (src/kernels/gemm_fp32.cpp:33-46). */
void or_linear_f32(const float* A, const float* W, const float* bias, float* C, int M, int N, int K);
/* LayerNormRef (src/kernels/layernorm.cpp:23-44). */
void or_layernorm(const float* x, const float* gamma, const float* beta, float eps, float* out, int rows, int d);
/* RoundToFp16Inplace (src/model.cpp:912-930): nearest fp16 and back. */
void or_round_fp16(float* x, size_t n);
/* GeluRef (src/kernels/gelu.cpp:30-35). */
void or_gelu(const float* x, float* out, size_t n);
/* RopeBuildTables (src/kernels/rope_tables.cpp:14-29). */
void or_rope_tables(int seq_len, int head_dim, float* cos_t, float* sin_t);
/* RopeApplyVarlenRef (src/kernels/rope.cpp:47-70). */
void or_rope_varlen(float* x, const float* cos_t, const float* sin_t, const int* cu, int B, int H, int dh);
/* AttentionVarlenRef (src/kernels/attention.cpp:99-144). */
void or_attention_varlen(const float* q, const float* k, const float* v, const int* cu, int B, int H, int dh,
                         float* out);

/* ---- oracle_x86.c: the reference's AVX-512 kernels (the facade's choice
 * for Isa::Avx512, Avx512Vnni and Amx, src/kernels/dispatch.cpp), lane by
 * lane. */
/* ExpAvx512 (gelu.cpp:40-68; attention.cpp:156-175, same code). */
float or_x86_exp(float x);
/* GeluAvx512 (gelu.cpp:98-148), one value and an array. */
float or_x86_gelu1(float v);
void or_x86_gelu(const float* x, float* out, size_t n);
/* LayerNormAvx512 (layernorm.cpp:59-149). */
void or_x86_layernorm(const float* x, const float* gamma, const float* beta, float eps, float* out, int rows,
                      int d);
/* RopeApplyVarlenAvx512 (rope.cpp:90-152). */
void or_x86_rope_varlen(float* x, const float* cos_t, const float* sin_t, const int* cu, int B, int H, int dh);
/* AttentionVarlenAvx512 (attention.cpp:240-430, 770-811). */
void or_x86_attention_varlen(const float* q, const float* k, const float* v, const int* cu, int B, int H, int dh,
                             float* out);
/* LinearAvx512 (gemm_fp32.cpp:194-294). */
void or_x86_linear_f32(const float* A, const float* W, const float* bias, float* C, int M, int N, int K);
/* QuantizeActPrefixAvx512 (gemm_int8.cpp:391-508) as signed int8 (the u8
 * offset of 128 is removed again by LinearVnni's col_sum correction). */
void or_x86_quant_act(const float* x, size_t n, int8_t* q, float* scale_out);
/* expf (glibc: the reference's std::exp) of every element. */
void or_expf_array(const float* x, float* out, size_t n);

/* Model descriptor for the restated forward: host pointers. */
typedef struct {
  int num_layers, hidden, heads, head_dim, ffn, vocab;
  float eps;
  int mask_token_id;
  int weights_int8;    /* 1: W8A8 linears, 0: fp32 linears */
  int act_per_token;   /* W8A8 only: 1 per-token scales, 0 per-tensor */
  const float* embed;  /* [vocab, hidden] */
  /* per layer, arrays of num_layers pointers */
  const float* const* ln1_w; const float* const* ln1_b;
  const float* const* ln2_w; const float* const* ln2_b;
  /* linears: index 0..5 = q, k, v, out, fc1, fc2; [layer * 6 + j] */
  const float* const* w_f32;
  const int8_t* const* w_i8;
  const float* const* w_scale;
  const float* const* bias;
  const float* final_ln_w; const float* final_ln_b;
  const float* lm_dense_w; const float* lm_dense_b;
  const float* lm_ln_w; const float* lm_ln_b;
  const float* lm_decoder_bias;
  int fc1_fp16;        /* 1: layer 0's fc1 input rounded to fp16 (model.cpp:1028-1033) */
  int x86;             /* 1: the reference's x86 AVX-512 kernels (oracle_x86.c) for LayerNorm,
                          GELU, RoPE, attention, FP32 Linear and activation quantisation
                          (Isa::Avx512Vnni: LinearVnni); 2: the same with LinearAmx's row
                          split (Isa::Amx); requires weights_int8 == 0 or act_per_token == 0 */
  int ffn_round24;     /* W8A8 per-token only: 1 rounds fc1's output to its top 24 bits
                          (or_round24) before GELU, the FFN intermediate of the GPU's default
                          per-token forward; not a reference mode (the reference keeps fp32) */
} or_model;

/* Embed (src/model.cpp:737-778) + TransformerBlock per layer (:932-1066) +
 * final LN and lm head (:1181-1239): packed logits [T, vocab]. Returns 0,
 * or -1 on allocation failure. */
int or_forward_packed(const or_model* m, const int32_t* ids, const int32_t* cu, int B, int T, float* logits);
/* The same, also writing every hidden state to hidden [num_layers + 1, T,
 * hidden] when it is not NULL: [0] post-embed, [i] after layer i, and [N]
 * the post-final-LN state in place of the last layer's output
 * (ForwardPackedInto's hidden_packed_out, model.cpp:1149-1189). */
int or_forward_packed_hidden(const or_model* m, const int32_t* ids, const int32_t* cu, int B, int T, float* logits,
                             float* hidden_out);
/* The same with BatchView's packed_masks (masks [T], 0 = pad; NULL: every
 * token real): Embed zeroes pad rows and counts only real tokens in the
 * token-dropout ratio's length (model.cpp:745-775); nothing else uses them. */
int or_forward_packed_masked(const or_model* m, const int32_t* ids, const int32_t* masks, const int32_t* cu, int B,
                             int T, float* logits, float* hidden_out);

/* x rounded to its top 24 bits (sign, exponent, 15 mantissa bits): 0x80
 * added to the bit pattern, then the low byte cleared, i.e. round to
 * nearest with ties away from zero; values that round past the largest
 * finite float become infinity; NaN becomes the quiet NaN 0x7fc00000.
 * Not a reference function: the GPU's default FFN intermediate format. */
float or_round24(float x);
void or_round24_array(const float* x, float* out, size_t n);

#ifdef __cplusplus
}
#endif

#endif
