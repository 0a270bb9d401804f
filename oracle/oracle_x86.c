/*
 * oracle_x86.c -- CPU restatement of the reference's x86 AVX-512 kernels
 * (the ones its facade selects for Isa::Avx512 / Avx512Vnni / Amx,
 * src/kernels/dispatch.cpp), lane by lane in scalar C.
 *
 * TEST INFRASTRUCTURE ONLY (the checker): see oracle.h.
 *
 * Compiled with -ffp-contract=off: every fused multiply-add below is an
 * explicit fmaf(). Those are the reference's explicit _mm512_fmadd_ps /
 * _mm512_fnmadd_ps, plus the products GCC contracts in the reference's own
 * build (-O3, -ffp-contract=fast by default): the range reduction
 * x - n*ln2_hi - n*ln2_lo of ExpAvx512 (gelu.cpp:40-68, attention.cpp:
 * 156-175), written there with vector operators, and LayerNormAvx512's
 * var = sum * (1/d) feeding var + eps (layernorm.cpp:121-123). Which form
 * the compiled reference uses was settled against the compiled reference
 * itself: the contracted forms match it bit for bit on every input tried,
 * the uncontracted ones do not.
 *
 * Horizontal sums follow _mm512_reduce_add_ps as GCC 11 defines it
 * (avx512fintrin.h): lanes 8..15 added to 0..7, then 4..7 to 0..3, then
 * a [2,3,0,1] shuffle-add, then lane 0 + lane 1.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static float bits_f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t f_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* _mm512_reduce_add_ps (GCC 11). */
static float red16(const float v[16]) {
  float t3[8], t6[4];
  for (int j = 0; j < 8; ++j) t3[j] = v[8 + j] + v[j];
  for (int j = 0; j < 4; ++j) t6[j] = t3[4 + j] + t3[j];
  const float a = t6[0] + t6[2];
  const float b = t6[1] + t6[3];
  return a + b;
}

/* _mm512_cvtps_epi32 on an integral value: out-of-range and NaN give the
 * integer indefinite 0x80000000. */
static int32_t cvt_i32(float x) {
  if (!(x > -2147483648.0f && x < 2147483648.0f)) return INT32_MIN;
  return (int32_t)x;
}

/* ExpAvx512 / ExpAvx512Attn (gelu.cpp:40-68, attention.cpp:156-175): 2^n
 * built from the exponent bits ((n + 127) << 23, wrapping for n < -127),
 * times a 5-term Taylor polynomial of r. */
float or_x86_exp(float x) {
  const float log2e = 1.44269504088896340736f;
  const float ln2_hi = 6.93145752e-1f;
  const float ln2_lo = 1.42860677e-6f;
  const float n = rintf(x * log2e);
  const float r = fmaf(-n, ln2_lo, fmaf(-n, ln2_hi, x));
  float p = 1.0f / 120.0f;
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const uint32_t e = (uint32_t)(cvt_i32(n) + 127) << 23;
  return p * bits_f(e);
}

/* ErfAvx512 (gelu.cpp:74-94): Abramowitz-Stegun 7.1.26. */
static float erf_x86(float x) {
  const uint32_t sign = f_bits(x) & 0x80000000u;
  const float ax = bits_f(f_bits(x) & 0x7fffffffu);
  const float t = 1.0f / fmaf(0.3275911f, ax, 1.0f);
  float poly = 1.061405429f;
  poly = fmaf(poly, t, -1.453152027f);
  poly = fmaf(poly, t, 1.421413741f);
  poly = fmaf(poly, t, -0.284496736f);
  poly = fmaf(poly, t, 0.254829592f);
  poly = poly * t;
  const float xx = x * x;
  const float neg_x2 = 0.0f - xx;
  const float e = or_x86_exp(neg_x2);
  const float abs_erf = fmaf(-poly, e, 1.0f);
  return bits_f(f_bits(abs_erf) | sign);
}

/* GeluAvx512 (gelu.cpp:98-148): (v * 0.5) * (1 + erf(v / sqrt 2)). */
float or_x86_gelu1(float v) {
  const float x = v * 0.70710678118654752440f;
  const float e = erf_x86(x);
  const float h = v * 0.5f;
  const float o = 1.0f + e;
  return h * o;
}

void or_x86_gelu(const float* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = or_x86_gelu1(x[i]);
}

/* LayerNormAvx512 (layernorm.cpp:59-149). Pass 1: four 16-lane sums over
 * 64-element blocks, leftover 16-blocks into the first, then a scalar
 * tail; mean = (hsum + tail) * (1/d). Pass 2: the same shape with
 * fma(x - mean, x - mean, acc); inv_std = 1 / sqrt(var * (1/d) + eps), the
 * product and sum fused as GCC compiles them. Pass 3:
 * fma((x - mean) * inv_std, gamma, beta). */
void or_x86_layernorm(const float* x, const float* gamma, const float* beta, float eps, float* out, int rows,
                      int d) {
  const float inv_d = 1.0f / (float)d;
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * d;
    float* yr = out + (size_t)r * d;
    float s[4][16];
    memset(s, 0, sizeof(s));
    int i = 0;
    for (; i + 64 <= d; i += 64)
      for (int k = 0; k < 4; ++k)
        for (int l = 0; l < 16; ++l) s[k][l] = s[k][l] + xr[i + 16 * k + l];
    for (; i + 16 <= d; i += 16)
      for (int l = 0; l < 16; ++l) s[0][l] = s[0][l] + xr[i + l];
    float tail = 0.0f;
    for (; i < d; ++i) tail += xr[i];
    float v[16];
    for (int l = 0; l < 16; ++l) v[l] = (s[0][l] + s[1][l]) + (s[2][l] + s[3][l]);
    const float mean = (red16(v) + tail) * inv_d;

    memset(s, 0, sizeof(s));
    i = 0;
    for (; i + 64 <= d; i += 64)
      for (int k = 0; k < 4; ++k)
        for (int l = 0; l < 16; ++l) {
          const float df = xr[i + 16 * k + l] - mean;
          s[k][l] = fmaf(df, df, s[k][l]);
        }
    for (; i + 16 <= d; i += 16)
      for (int l = 0; l < 16; ++l) {
        const float df = xr[i + l] - mean;
        s[0][l] = fmaf(df, df, s[0][l]);
      }
    float vtail = 0.0f;
    for (; i < d; ++i) {
      /* scalar tail of the reference: diff * diff added, contracted by GCC */
      const float df = xr[i] - mean;
      vtail = fmaf(df, df, vtail);
    }
    for (int l = 0; l < 16; ++l) v[l] = (s[0][l] + s[1][l]) + (s[2][l] + s[3][l]);
    /* var = sum * inv_d feeds only var + eps: GCC fuses the two. */
    const float inv_std = 1.0f / sqrtf(fmaf(red16(v) + vtail, inv_d, eps));
    for (int j = 0; j < d; ++j) {
      const float normed = (xr[j] - mean) * inv_std;
      yr[j] = fmaf(normed, gamma[j], beta[j]);
    }
  }
}

/* RopeApplyVarlenAvx512 (rope.cpp:90-152): lo' = fnmadd(hi, s, lo*c),
 * hi' = fmadd(hi, c, lo*s), per first-half index i. */
void or_x86_rope_varlen(float* x, const float* cos_t, const float* sin_t, const int* cu, int B, int H, int dh) {
  const int half = dh / 2;
  for (int b = 0; b < B; ++b)
    for (int p = 0; p < cu[b + 1] - cu[b]; ++p) {
      const float* c = cos_t + (size_t)p * dh;
      const float* s = sin_t + (size_t)p * dh;
      for (int h = 0; h < H; ++h) {
        float* xr = x + ((size_t)(cu[b] + p) * H + h) * dh;
        for (int i = 0; i < half; ++i) {
          const float lo = xr[i], hi = xr[i + half];
          const float lo_c = lo * c[i];
          const float lo_s = lo * s[i];
          xr[i] = fmaf(-hi, s[i], lo_c);
          xr[i + half] = fmaf(hi, c[i], lo_s);
        }
      }
    }
}

/* DotAvx512 / the 16-accumulator score loop (attention.cpp:199-214,
 * 281-343): lane l accumulates q[d]*k[d] for d = l (mod 16), d ascending;
 * a partial last chunk reads zeros past head_dim. */
static float dot_x86(const float* a, const float* b, int n) {
  float acc[16] = {0};
  int d = 0;
  for (; d + 16 <= n; d += 16)
    for (int l = 0; l < 16; ++l) acc[l] = fmaf(a[d + l], b[d + l], acc[l]);
  if (d < n)
    for (int l = 0; l < 16; ++l) acc[l] = fmaf(d + l < n ? a[d + l] : 0.0f, d + l < n ? b[d + l] : 0.0f, acc[l]);
  return red16(acc);
}

/* AttentionVarlenAvx512 / RunOneHeadAvx512Impl (attention.cpp:240-430,
 * 770-811). Per query: scores by dot_x86; max over all; whole 16-key
 * chunks exponentiated by ExpAvx512Attn and summed lane-wise (lane l: keys
 * l mod 16, chunk order), then reduced; keys past the last whole chunk use
 * std::exp (expf) and are added one by one; inv = 1/sum; out = sum over
 * keys in order of fma(e * inv, v, out), zero weights skipped. */
void or_x86_attention_varlen(const float* q, const float* k, const float* v, const int* cu, int B, int H, int dh,
                             float* out) {
  int maxL = 0;
  for (int b = 0; b < B; ++b)
    if (cu[b + 1] - cu[b] > maxL) maxL = cu[b + 1] - cu[b];
  /* (sequence, head) pairs are independent, as in the reference's parallel_for. */
#pragma omp parallel
  {
  float* sc = (float*)malloc(sizeof(float) * (size_t)(maxL > 0 ? maxL : 1));
  float* o = (float*)malloc(sizeof(float) * (size_t)(dh > 0 ? dh : 1));
#pragma omp for schedule(dynamic, 1)
  for (int bh = 0; bh < B * H; ++bh) {
    const int b = bh / H, h = bh % H;
    const int s0 = cu[b], L = cu[b + 1] - cu[b];
    if (L <= 0) continue;
    const int Lfull = L & ~15;
    {
      for (int i = 0; i < L; ++i) {
        const float* qi = q + ((size_t)(s0 + i) * H + h) * dh;
        float mx = -INFINITY;
        for (int j = 0; j < L; ++j) {
          sc[j] = dot_x86(qi, k + ((size_t)(s0 + j) * H + h) * dh, dh);
          if (sc[j] > mx) mx = sc[j];
        }
        float vs[16] = {0};
        for (int j = 0; j < Lfull; j += 16)
          for (int l = 0; l < 16; ++l) {
            const float e = or_x86_exp(sc[j + l] - mx);
            sc[j + l] = e;
            vs[l] = vs[l] + e;
          }
        float sum = red16(vs);
        for (int j = Lfull; j < L; ++j) {
          const float e = expf(sc[j] - mx);
          sc[j] = e;
          sum += e;
        }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (int d = 0; d < dh; ++d) o[d] = 0.0f;
        for (int j = 0; j < L; ++j) {
          const float w = sc[j] * inv;
          if (w == 0.0f) continue;
          const float* vj = v + ((size_t)(s0 + j) * H + h) * dh;
          for (int d = 0; d < dh; ++d) o[d] = fmaf(w, vj[d], o[d]);
        }
        memcpy(out + ((size_t)(s0 + i) * H + h) * dh, o, sizeof(float) * (size_t)dh);
      }
    }
  }
  free(sc);
  free(o);
  }
}

/* glibc's expf over an array: the reference's std::exp, as the checker of
 * the device restatement (several threads; each value on its own). */
void or_expf_array(const float* x, float* out, size_t n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)n; ++i) out[i] = expf(x[i]);
}

/* LinearAvx512 (gemm_fp32.cpp:272-294, Dot1Row8N / Dot1Row1N :194-270):
 * C[m, n] = bias[n] + hsum(lane-wise fma over K in 16-wide steps). */
void or_x86_linear_f32(const float* A, const float* W, const float* bias, float* C, int M, int N, int K) {
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      const float b = bias ? bias[n] : 0.0f;
      C[(size_t)m * N + n] = b + dot_x86(A + (size_t)m * K, W + (size_t)n * K, K);
    }
}

/* QuantizeActPrefixAvx512 (gemm_int8.cpp:391-508) with the u8 offset
 * removed (LinearVnni subtracts 128 * col_sum again, gemm_int8.cpp:
 * 109-126): whole 16-element blocks round with cvtps (nearest even), the
 * last n % 16 elements with lround (half away from zero). */
void or_x86_quant_act(const float* x, size_t n, int8_t* q, float* scale_out) {
  float amax = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    const float a = fabsf(x[i]);
    if (a > amax) amax = a;
  }
  const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
  const float inv = 1.0f / scale;
  *scale_out = scale;
  const size_t body = n & ~(size_t)15;
  for (size_t i = 0; i < n; ++i) {
    const float y = x[i] * inv;
    long r = i < body ? (long)rintf(y) : lroundf(y);
    if (r < -127) r = -127;
    if (r > 127) r = 127;
    q[i] = (int8_t)r;
  }
}
