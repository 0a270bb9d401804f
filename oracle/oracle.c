/*
 * oracle.c -- CPU restatement of esm.cpp's packed ESM-2 encoder hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker): see oracle.h. Built with the
 * flags the reference's Release build uses (-O3 -march=x86-64-v3, where
 * GCC contracts a*b+c into an FMA), so each restated *Ref function rounds
 * exactly as the compiled reference does; libm float functions (expf,
 * erff, powf, cosf, sinf, sqrtf, nearbyintf) are what the reference's
 * std:: calls resolve to.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* gemm_int8.cpp:109-126 / gemm_amx.cpp:114-127: after the zero-point
 * correction acc - 128*col_sum the VNNI/AMX accumulator is exactly
 * sum_k q[m,k] * w[n,k]; this is that closed form. */
void or_gemm_i8_i32(const int8_t* A, int lda, const int8_t* W, int ldw, int M, int N, int K, int32_t* C) {
#pragma omp parallel for schedule(dynamic, 4)
  for (int m = 0; m < M; ++m) {
    const int8_t* a = A + (size_t)m * lda;
    for (int n = 0; n < N; ++n) {
      const int8_t* w = W + (size_t)n * ldw;
      int32_t acc = 0;
      for (int k = 0; k < K; ++k) acc += (int32_t)a[k] * (int32_t)w[k];
      C[(size_t)m * N + n] = acc;
    }
  }
}

static float absmax_f(const float* x, size_t n) {
  float m = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    const float v = fabsf(x[i]);
    if (v > m) m = v;
  }
  return m;
}

static void quant_block(const float* x, size_t n, float inv, int8_t* q) {
  for (size_t i = 0; i < n; ++i) {
    float r = nearbyintf(x[i] * inv);
    if (r > 127.0f) r = 127.0f;
    if (r < -127.0f) r = -127.0f;
    q[i] = (int8_t)(int)r;
  }
}

/* gemm_int8.cpp:434-436,476 (scale rule), :491-496 (quantise). */
void or_quant_act_tensor(const float* x, size_t n, int8_t* q, float* scale_out) {
  const float amax = absmax_f(x, n);
  const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
  *scale_out = scale;
  quant_block(x, n, 1.0f / scale, q);
}

void or_quant_act_rows(const float* x, int M, int K, int8_t* q, float* scales) {
  for (int m = 0; m < M; ++m) or_quant_act_tensor(x + (size_t)m * K, (size_t)K, q + (size_t)m * K, scales + m);
}

/* RoundToFp16Inplace (model.cpp:912-930, x86 F16C branch): each value to
 * the nearest fp16 (ties to even) and back. */
void or_round_fp16(float* x, size_t n) {
  for (size_t i = 0; i < n; ++i)
    x[i] = _cvtsh_ss(_cvtss_sh(x[i], _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
}

/* GeluRef (gelu.cpp:30-35). */
static float gelu1(float x) {
  const float kInvSqrt2 = 0.70710678118654752440f;
  return x * 0.5f * (1.0f + erff(x * kInvSqrt2));
}

void or_dequant(const int32_t* acc, const float* a_scale, const float* w_scale, const float* bias, int M, int N,
                int gelu, float* out) {
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      const float combined = w_scale[n] * a_scale[m];
      float v = fmaf((float)acc[(size_t)m * N + n], combined, bias ? bias[n] : 0.0f);
      if (gelu) v = gelu1(v);
      out[(size_t)m * N + n] = v;
    }
}

/* Quantize (pack.cpp:149-177). */
void or_quantize_weight(const float* W, int N, int K, int8_t* q, float* scales) {
  for (int n = 0; n < N; ++n) {
    const float* row = W + (size_t)n * K;
    float row_max = 0.0f;
    for (int k = 0; k < K; ++k) {
      const float a = fabsf(row[k]);
      if (a > row_max) row_max = a;
    }
    int8_t* qr = q + (size_t)n * K;
    if (row_max == 0.0f) {
      scales[n] = 0.0f;
      memset(qr, 0, (size_t)K);
      continue;
    }
    const float scale = row_max / 127.0f;
    scales[n] = scale;
    quant_block(row, (size_t)K, 1.0f / scale, qr);
  }
}

/* LinearInt8Ref (gemm_int8.cpp:49-64). */
void or_linear_int8_w8a16(const float* A, const int8_t* Wq, const float* scales, const float* bias, float* C, int M,
                          int N, int K) {
  for (int m = 0; m < M; ++m) {
    const float* a = A + (size_t)m * K;
    for (int n = 0; n < N; ++n) {
      const int8_t* w = Wq + (size_t)n * K;
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) acc += a[k] * (float)w[k];
      C[(size_t)m * N + n] = acc * scales[n] + (bias ? bias[n] : 0.0f);
    }
  }
}

/* LinearRef (gemm_fp32.cpp:33-46): the bias seeds the accumulator, then
 * k = 0..K-1 in order. Eight outputs are carried side by side; each keeps
 * its own sequential sum, so every result is the reference's bit for bit. */
void or_linear_f32(const float* A, const float* W, const float* bias, float* C, int M, int N, int K) {
#pragma omp parallel for schedule(dynamic, 4)
  for (int m = 0; m < M; ++m) {
    const float* a = A + (size_t)m * K;
    int n = 0;
    for (; n + 8 <= N; n += 8) {
      float acc[8];
      const float* w[8];
      for (int j = 0; j < 8; ++j) {
        acc[j] = bias ? bias[n + j] : 0.0f;
        w[j] = W + (size_t)(n + j) * K;
      }
      for (int k = 0; k < K; ++k) {
        const float ak = a[k];
        for (int j = 0; j < 8; ++j) acc[j] += ak * w[j][k];
      }
      for (int j = 0; j < 8; ++j) C[(size_t)m * N + n + j] = acc[j];
    }
    for (; n < N; ++n) {
      const float* w = W + (size_t)n * K;
      float acc = bias ? bias[n] : 0.0f;
      for (int k = 0; k < K; ++k) acc += a[k] * w[k];
      C[(size_t)m * N + n] = acc;
    }
  }
}

/* LayerNormRef (layernorm.cpp:23-44): mean and variance in double. */
void or_layernorm(const float* x, const float* gamma, const float* beta, float eps, float* out, int rows, int d) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * d;
    float* yr = out + (size_t)r * d;
    double mean = 0.0;
    for (int i = 0; i < d; ++i) mean += xr[i];
    mean /= d;
    double var = 0.0;
    for (int i = 0; i < d; ++i) {
      const double diff = xr[i] - mean;
      var += diff * diff;
    }
    var /= d;
    const float inv_std = 1.0f / sqrtf((float)var + eps);
    for (int i = 0; i < d; ++i) {
      const float normed = (xr[i] - (float)mean) * inv_std;
      yr[i] = normed * gamma[i] + beta[i];
    }
  }
}

void or_gelu(const float* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = gelu1(x[i]);
}

/* RopeBuildTables (rope_tables.cpp:14-29). */
void or_rope_tables(int seq_len, int head_dim, float* cos_t, float* sin_t) {
  const int half = head_dim / 2;
  for (int i = 0; i < half; ++i) {
    const float exponent = (float)(2 * i) / (float)head_dim;
    const float inv_freq = powf(10000.0f, -exponent);
    for (int t = 0; t < seq_len; ++t) {
      const float angle = (float)t * inv_freq;
      const float c = cosf(angle);
      const float s = sinf(angle);
      cos_t[t * head_dim + i] = c;
      cos_t[t * head_dim + i + half] = c;
      sin_t[t * head_dim + i] = s;
      sin_t[t * head_dim + i + half] = s;
    }
  }
}

/* RopeApplyVarlenRef (rope.cpp:47-70). */
void or_rope_varlen(float* x, const float* cos_t, const float* sin_t, const int* cu, int B, int H, int dh) {
  const int half = dh / 2;
  for (int b = 0; b < B; ++b) {
    for (int p = 0; p < cu[b + 1] - cu[b]; ++p) {
      const int t = cu[b] + p;
      const float* crow = cos_t + (size_t)p * dh;
      const float* srow = sin_t + (size_t)p * dh;
      for (int h = 0; h < H; ++h) {
        float* xr = x + ((size_t)t * H + h) * dh;
        for (int i = 0; i < half; ++i) {
          const float x1 = xr[i], x2 = xr[i + half];
          xr[i] = x1 * crow[i] + (-x2) * srow[i];
          xr[i + half] = x2 * crow[i + half] + x1 * srow[i + half];
        }
      }
    }
  }
}

/* AttentionVarlenRef (attention.cpp:99-144): fp32 dots, max, expf, double
 * sum, float(1/sum), out += (e * inv) * v in key order. */
void or_attention_varlen(const float* q, const float* k, const float* v, const int* cu, int B, int H, int dh,
                         float* out) {
  int maxL = 0;
  for (int b = 0; b < B; ++b)
    if (cu[b + 1] - cu[b] > maxL) maxL = cu[b + 1] - cu[b];
  float* scores = (float*)malloc(sizeof(float) * (size_t)(maxL > 0 ? maxL : 1));
  for (int b = 0; b < B; ++b) {
    const int s0 = cu[b], L = cu[b + 1] - cu[b];
    if (L <= 0) continue;
    for (int h = 0; h < H; ++h)
      for (int i = 0; i < L; ++i) {
        const float* qi = q + ((size_t)(s0 + i) * H + h) * dh;
        float mx = -INFINITY;
        for (int j = 0; j < L; ++j) {
          const float* kj = k + ((size_t)(s0 + j) * H + h) * dh;
          float dot = 0.0f;
          for (int d = 0; d < dh; ++d) dot += qi[d] * kj[d];
          scores[j] = dot;
          if (dot > mx) mx = dot;
        }
        double sum = 0.0;
        for (int j = 0; j < L; ++j) {
          const float e = expf(scores[j] - mx);
          scores[j] = e;
          sum += e;
        }
        const float inv = sum > 0.0 ? (float)(1.0 / sum) : 0.0f;
        float* o = out + ((size_t)(s0 + i) * H + h) * dh;
        for (int d = 0; d < dh; ++d) o[d] = 0.0f;
        for (int j = 0; j < L; ++j) {
          const float w = scores[j] * inv;
          if (w == 0.0f) continue;
          const float* vj = v + ((size_t)(s0 + j) * H + h) * dh;
          for (int d = 0; d < dh; ++d) o[d] += w * vj[d];
        }
      }
  }
  free(scores);
}

/* One Linear call of TransformerBlock (LinearProj, model.cpp:877-905). */
static void linear_call(const or_model* m, int layer, int j, const float* A, float* C, int M, int N, int K,
                        int8_t* qbuf, float* sbuf, int32_t* accbuf) {
  const int idx = layer * 6 + j;
  if (!m->weights_int8) {
    (m->x86 ? or_x86_linear_f32 : or_linear_f32)(A, m->w_f32[idx], m->bias[idx], C, M, N, K);
    return;
  }
  if (m->x86) {
    float s;
    or_x86_quant_act(A, (size_t)M * K, qbuf, &s);
    for (int r = 0; r < M; ++r) sbuf[r] = s;
    /* LinearAmx (gemm_amx.cpp:218-309): for M >= 32, N % 32 == 0 and
     * K % 64 == 0 the first M & ~31 rows run on AMX with the scale of the
     * whole input, and the last M % 32 rows go to LinearVnni as a call of
     * their own, which quantises them with their own per-tensor scale. */
    const int m_main = M & ~31;
    if (m->x86 == 2 && M >= 32 && N % 32 == 0 && K % 64 == 0 && m_main < M) {
      or_x86_quant_act(A + (size_t)m_main * K, (size_t)(M - m_main) * K, qbuf + (size_t)m_main * K, &s);
      for (int r = m_main; r < M; ++r) sbuf[r] = s;
    }
  } else if (m->act_per_token) {
    or_quant_act_rows(A, M, K, qbuf, sbuf);
  } else {
    float s;
    or_quant_act_tensor(A, (size_t)M * K, qbuf, &s);
    for (int r = 0; r < M; ++r) sbuf[r] = s;
  }
  or_gemm_i8_i32(qbuf, K, m->w_i8[idx], K, M, N, K, accbuf);
  or_dequant(accbuf, sbuf, m->w_scale[idx], m->bias[idx], M, N, 0, C);
}

float or_round24(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  if ((b & 0x7fffffffu) > 0x7f800000u)
    b = 0x7fc00000u; /* NaN: the quiet NaN (an add could carry into the sign) */
  else
    b += 0x80u;
  b &= 0xffffff00u;
  memcpy(&x, &b, 4);
  return x;
}

void or_round24_array(const float* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = or_round24(x[i]);
}

int or_forward_packed(const or_model* m, const int32_t* ids, const int32_t* cu, int B, int T, float* logits) {
  return or_forward_packed_masked(m, ids, NULL, cu, B, T, logits, NULL);
}

int or_forward_packed_hidden(const or_model* m, const int32_t* ids, const int32_t* cu, int B, int T, float* logits,
                             float* hidden_out) {
  return or_forward_packed_masked(m, ids, NULL, cu, B, T, logits, hidden_out);
}

int or_forward_packed_masked(const or_model* m, const int32_t* ids, const int32_t* masks, const int32_t* cu, int B,
                             int T, float* logits, float* hidden_out) {
  const int d = m->hidden, H = m->heads, dh = m->head_dim, f = m->ffn, V = m->vocab;
  const size_t Td = (size_t)T * d, Tf = (size_t)T * f;
  int maxL = 0;
  for (int b = 0; b < B; ++b)
    if (cu[b + 1] - cu[b] > maxL) maxL = cu[b + 1] - cu[b];
  float* hidden = (float*)malloc(Td * 4);
  float* ln = (float*)malloc(Td * 4);
  float* qkv = (float*)malloc(3 * Td * 4);
  float* attn = (float*)malloc(Td * 4);
  float* proj = (float*)malloc(Td * 4);
  float* inter = (float*)malloc(Tf * 4);
  float* inter_g = (float*)malloc(Tf * 4);
  float* cos_t = (float*)malloc((size_t)(maxL > 0 ? maxL : 1) * dh * 4);
  float* sin_t = (float*)malloc((size_t)(maxL > 0 ? maxL : 1) * dh * 4);
  int8_t* qbuf = (int8_t*)malloc(Tf > Td ? Tf : Td);
  float* sbuf = (float*)malloc((size_t)T * 4);
  int32_t* acc = (int32_t*)malloc((Tf > Td ? Tf : Td) * 4);
  if (!hidden || !ln || !qkv || !attn || !proj || !inter || !inter_g || !cos_t || !sin_t || !qbuf || !sbuf || !acc)
    return -1;

  /* Embed (model.cpp:737-778): src_len counts real tokens (masks[t] != 0,
   * every token when masks is NULL), mask tokens are counted over all
   * tokens; mask-token and pad rows are zero. */
  const float k_drop = 0.15f * 0.8f;
  for (int b = 0; b < B; ++b) {
    int src_len = 0, mask_tokens = 0;
    for (int t = cu[b]; t < cu[b + 1]; ++t) {
      if (!masks || masks[t] != 0) ++src_len;
      if (ids[t] == m->mask_token_id) ++mask_tokens;
    }
    const float ratio = src_len > 0 ? (float)mask_tokens / (float)src_len : 0.0f;
    float denom = 1.0f - ratio;
    if (denom < 1e-12f) denom = 1e-12f;
    const float scale = (1.0f - k_drop) / denom;
    for (int t = cu[b]; t < cu[b + 1]; ++t) {
      const float* row = m->embed + (size_t)ids[t] * d;
      float* o = hidden + (size_t)t * d;
      const int zero = ids[t] == m->mask_token_id || (masks && masks[t] == 0);
      for (int i = 0; i < d; ++i) o[i] = zero ? 0.0f : row[i] * scale;
    }
  }

  if (hidden_out) memcpy(hidden_out, hidden, Td * 4);

  const float q_scale = 1.0f / sqrtf((float)dh);
  void (*layernorm)(const float*, const float*, const float*, float, float*, int, int) =
      m->x86 ? or_x86_layernorm : or_layernorm;
  void (*gelu)(const float*, float*, size_t) = m->x86 ? or_x86_gelu : or_gelu;
  void (*rope)(float*, const float*, const float*, const int*, int, int, int) =
      m->x86 ? or_x86_rope_varlen : or_rope_varlen;
  void (*attention)(const float*, const float*, const float*, const int*, int, int, int, float*) =
      m->x86 ? or_x86_attention_varlen : or_attention_varlen;
  void (*linear_f32)(const float*, const float*, const float*, float*, int, int, int) =
      m->x86 ? or_x86_linear_f32 : or_linear_f32;
  for (int l = 0; l < m->num_layers; ++l) {
    float* q = qkv;
    float* k = qkv + Td;
    float* v = qkv + 2 * Td;
    layernorm(hidden, m->ln1_w[l], m->ln1_b[l], m->eps, ln, T, d);
    linear_call(m, l, 0, ln, q, T, d, d, qbuf, sbuf, acc);
    linear_call(m, l, 1, ln, k, T, d, d, qbuf, sbuf, acc);
    linear_call(m, l, 2, ln, v, T, d, d, qbuf, sbuf, acc);
    for (size_t i = 0; i < Td; ++i) q[i] *= q_scale;
    or_rope_tables(maxL, dh, cos_t, sin_t);
    rope(q, cos_t, sin_t, cu, B, H, dh);
    rope(k, cos_t, sin_t, cu, B, H, dh);
    attention(q, k, v, cu, B, H, dh, attn);
    linear_call(m, l, 3, attn, proj, T, d, d, qbuf, sbuf, acc);
    for (size_t i = 0; i < Td; ++i) hidden[i] += proj[i];
    layernorm(hidden, m->ln2_w[l], m->ln2_b[l], m->eps, ln, T, d);
    if (m->fc1_fp16 && l == 0) or_round_fp16(ln, Td);
    linear_call(m, l, 4, ln, inter, T, f, d, qbuf, sbuf, acc);
    if (m->ffn_round24 && m->weights_int8 && m->act_per_token && !m->x86) or_round24_array(inter, inter, Tf);
    gelu(inter, inter_g, Tf);
    linear_call(m, l, 5, inter_g, proj, T, d, f, qbuf, sbuf, acc);
    for (size_t i = 0; i < Td; ++i) hidden[i] += proj[i];
    if (hidden_out) memcpy(hidden_out + (size_t)(l + 1) * Td, hidden, Td * 4);
  }
  layernorm(hidden, m->final_ln_w, m->final_ln_b, m->eps, ln, T, d);
  if (hidden_out) memcpy(hidden_out + (size_t)m->num_layers * Td, ln, Td * 4);
  linear_f32(ln, m->lm_dense_w, m->lm_dense_b, proj, T, d, d);
  gelu(proj, attn, Td);
  layernorm(attn, m->lm_ln_w, m->lm_ln_b, m->eps, ln, T, d);
  linear_f32(ln, m->embed, m->lm_decoder_bias, logits, T, V, d);

  free(hidden); free(ln); free(qkv); free(attn); free(proj); free(inter); free(inter_g);
  free(cos_t); free(sin_t); free(qbuf); free(sbuf); free(acc);
  return 0;
}
