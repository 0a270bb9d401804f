// Kernel launch interface shared by the gfx950 translation units. Every
// launcher enqueues on the given stream and returns the launch status; no
// launcher allocates memory.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace esm_gfx950 {

// ---------------------------------------------------------------- INT8 GEMM
// C[m, n] = sum_k A[m, k] * W[n, k]  (int8 x int8 -> int32), then one of the
// epilogues below. A is row-major [M, lda], W row-major [N, ldw]; K must be a
// multiple of 16 (callers zero-pad rows to that width).
enum GemmEpilogue : int {
  kEpiI32 = 0,        // C_i32[m*ldc + n] = acc
  kEpiF32 = 1,        // C_f32 = fma(acc, a_scale[m]*w_scale[n], bias[n])
  kEpiF32Gelu = 2,    // C_f32 = gelu(...) (+ optional absmax outputs)
  kEpiF32Resid = 3,   // C_f32 += fma(...)   (residual add into hidden)
  kEpiQkvRope = 4,    // split Q|K|V, Q*q_scale, RoPE on Q and K, bf16/fp16 out
  kEpiF32GeluQ = 5,   // gelu(...) -> fp16 store + per-row absmax (atomic)
  kEpiQkvRopeF32 = 6, // fp32 [M, 3*d_model] (ldc): Q*q_scale and RoPE on Q, K
  kEpiQkvSplit = 7,   // as kEpiQkvRopeF32, then Q *= q_prescale and every value
                      // stored as a split-fp16 word (C_f32 reinterpreted)
  kEpiF32R24 = 8,     // kEpiF32's value rounded to its top 24 bits (sign,
                      // exponent, 15 mantissa bits; nearest, ties away;
                      // NaN -> the quiet NaN 0x7fc00000):
                      // bits 31..16 to C_f16 [M, ldc], bits 15..8 to C_u8;
                      // in each aligned group of 64 columns, stored position
                      // 2 i + j holds column 32 j + i (i < 32, j < 2). C_u8
                      // interleaves row pairs: byte (r & ~1) ldc + 4 (p / 2)
                      // + 2 (r & 1) + (p & 1) holds row r, position p, so it
                      // spans (M + (M & 1)) ldc bytes. Pipelined kernel only;
                      // N % 64 == 0.
  kEpiF32GeluAs = 9,  // as kEpiF32Gelu with the erf of Abramowitz & Stegun
                      // 7.1.26 (gelu2_as / 2, the GELU of the fused GELU +
                      // quantisation passes and of the reference's AVX-512
                      // Gelu) instead of erff
  kEpiF32GeluX86 = 10,  // as kEpiF32Gelu with the reference's GeluAvx512
                        // (gelu_x86) on the dequantised value: the x86-exact
                        // forward's fc1 + Gelu, bit for bit
};

// Split-fp16 word of an fp32 value x: low half fp16(x), high half
// fp16(x - fp16(x)); hi + lo carries 22 significant bits.

struct GemmI8Args {
  const int8_t* A = nullptr;
  int lda = 0;
  const int8_t* W = nullptr;
  int ldw = 0;
  int M = 0, N = 0, K = 0;
  int32_t* C_i32 = nullptr;
  float* C_f32 = nullptr;
  uint16_t* C_f16 = nullptr;
  uint8_t* C_u8 = nullptr;  // kEpiF32R24: the low byte plane
  int ldc = 0;
  const float* a_scale = nullptr;  // [M]
  const float* w_scale = nullptr;  // [N]
  const float* bias = nullptr;     // [N] or null
  float* row_absmax = nullptr;     // [M] (atomic max of |out|) or null
  float* tensor_absmax = nullptr;  // scalar (atomic max of |out|) or null
  // kEpiQkvRope
  uint16_t* q_out = nullptr;  // bf16 or fp16 [M, d_model]
  uint16_t* k_out = nullptr;  // bf16 or fp16 [M, d_model]
  uint16_t* v_out = nullptr;  // fp16 [M, d_model]
  int qk_fp16 = 0;            // Q/K stored as fp16 (else bf16)
  int d_model = 0;
  const int* pos = nullptr;          // [M] position inside the sequence
  const float* rope_cos = nullptr;   // [max_len, 64]
  const float* rope_sin = nullptr;   // [max_len, 32]
  float q_scale = 1.0f;
  float q_prescale = 1.0f;  // kEpiQkvSplit: power of two applied to Q before the split
  // kEpiQkvRopeF32, pipelined kernel: rotate as RopeApplyVarlenAvx512 does
  // (reference src/kernels/rope.cpp:90-152), the first element of each pair
  // as fma(-hi, s, lo * c) instead of fma(lo, c, -(hi * s)).
  int rope_x86 = 0;
  int cus = 0;              // CUs the launch can expect to have to itself (0: the device's)
  // Split-K, int32 output (kEpiI32): the grid holds splits x tiles
  // workgroups, and C_i32 holds `splits` consecutive [M, ldc] planes of
  // partial sums over contiguous ranges of K.
  int splits = 1;
  // kEpiF32 launches: int32 workspace of splitk_ws_elems elements that a grid
  // too small for the device may split K into (partial planes, then one
  // dequant pass); null: never split.
  int32_t* splitk_ws = nullptr;
  size_t splitk_ws_elems = 0;
};

// Picks the pipelined 256- or 320-row-tile kernel when gemm_i8_pipelined_ok(p) (K a
// multiple of 128, 16-byte aligned rows, M*lda and N*ldw at most 2^32 bytes),
// else the general 256x128 kernel.
hipError_t launch_gemm_i8(const GemmI8Args& p, int epilogue, hipStream_t s);
bool gemm_i8_pipelined_ok(const GemmI8Args& p);
// variant 1: general kernel; 2: pipelined kernel (fails on shapes it cannot take).
hipError_t launch_gemm_i8_variant(const GemmI8Args& p, int epilogue, int variant, hipStream_t s);
// Row height of the pipelined kernel's tile for every later launch in the
// process: 64, 128, 256, 320, or 0 to pick per launch (gemm_i8_tile_rows).
// False for other values.
bool set_gemm_tile_rows(int rows);
// The pipelined kernel's tile height for an M x N x K launch with epilogue
// epi on `cus` CUs (0: the current device's): grids of at least one 256-row
// workgroup per CU take 256 or 320 rows, whichever needs the fewer rows'
// worth of workgroup rounds (320 on a tie, for the epilogues that fit it);
// smaller grids take 64, 128 or 256 rows by an estimate of their time.
int gemm_i8_tile_rows(int M, int N, int K, int epi, int cus);
// Compute units of the current device (queried once per device; 256 if the
// query fails).
int device_cus();
// K splits of a kEpiF32 launch with a workspace (1: none): grids that leave
// CUs idle split K when the estimated time of the split grid plus its dequant
// pass beats the unsplit one's. *rows receives the tile height to use.
// fused: the partial planes are summed by the kernel that reads the result
// (launch_layernorm_quant_split) instead of a pass of their own, which then
// costs only that kernel's extra reads.
int gemm_i8_split_k(int M, int N, int K, int cus, bool fused, int* rows);
// The kEpiI32 split-K grid alone: p.C_i32 receives `splits` [M, p.ldc] planes
// of partial sums (p.ldc >= N), at tile height rows.
hipError_t launch_gemm_i8_partials(const GemmI8Args& p, int splits, int rows, hipStream_t s);
// Process-wide override of gemm_i8_split_k for later launches: 0 automatic,
// 1 never, 2..4 that many splits wherever a launch qualifies (workspace large
// enough, kEpiF32 without absmax outputs). False for other values.
bool set_gemm_split_k(int splits);

// ---------------------------------------------------------------- FP32 GEMM
enum GemmF32Epilogue : int {
  kF32Store = 0,   // C = A W^T + bias
  kF32Gelu = 1,    // C = gelu(A W^T + bias)
  kF32Resid = 2,   // C += A W^T + bias
};
struct GemmF32Args {
  const float* A = nullptr;
  int lda = 0;
  const float* W = nullptr;
  int ldw = 0;
  const float* bias = nullptr;
  float* C = nullptr;
  int ldc = 0;
  int M = 0, N = 0, K = 0;
};
hipError_t launch_gemm_f32(const GemmF32Args& p, int epilogue, hipStream_t s);
// C = A W^T + bias for N <= 48 (the tied vocabulary decoder), fp32 MFMA, one
// wave per 16 rows; K % 16 == 0, lda and ldw multiples of 4.
hipError_t launch_gemm_narrow(const GemmF32Args& p, hipStream_t s);

// FP32-accurate GEMM on fp16 MFMA ("split-fp16"): every operand x is carried
// as hi = fp16(x) and lo = fp16(x - hi), and every product as hi*hi + lo*hi +
// hi*lo (22 significant bits per operand; the dropped lo*lo term is below
// 2^-22 relative), accumulated in fp32. A is fp32 and split on the fly; W
// arrives pre-split as two fp16 planes [N, ldw] holding W * 2^w_shift (the
// shift keeps the lo parts of small weights out of the fp16 subnormal
// range), which the epilogue undoes exactly. K % 32 == 0.
struct GemmX3Args {
  const float* A = nullptr;
  int lda = 0;
  const uint16_t* w_hi = nullptr;
  const uint16_t* w_lo = nullptr;
  int ldw = 0;
  float w_unscale = 1.0f;  // 2^-w_shift
  const float* bias = nullptr;
  float* C = nullptr;
  int ldc = 0;
  int M = 0, N = 0, K = 0;
};
hipError_t launch_gemm_x3(const GemmX3Args& p, int epilogue, hipStream_t s);

// ------------------------------------------------------------- attention
// One work item per (sequence, head, query tile); built on the host from
// cu_seqlens, longest sequences first.
struct AttnWork {
  int seq;
  int head;
  int q0;
  int pad;
};
// Q/K bf16 or fp16 (QK^T on the matching MFMA), V bf16 or fp16 (PV on fp16
// MFMA with fp16 probabilities), fp32 online softmax, head_dim 64.
// q/k/v rows: token t, head h at base + t*ld + h*64.
hipError_t launch_attention_mfma(const uint16_t* q, const uint16_t* k,
                                 const uint16_t* v, int qk_is_fp16, int v_is_bf16,
                                 int ld, const int* cu_seqlens,
                                 const AttnWork* work, int num_work, float* out,
                                 int ld_out, float* tensor_absmax,
                                 hipStream_t s);
// Split-fp16 MFMA path, head_dim 64, three MFMAs per product (fp32-level
// accuracy on the fp16 matrix cores). Operands in the layout the QKV
// epilogue (kEpiQkvSplit) writes: within each 64-wide head, positions hold
// dims 0, 32, 1, 33, ..., 31, 63; q as split-fp16 words (row stride ldq
// words, already multiplied by q_prescale); K and V as fp16 hi planes (kh,
// vh) and lo planes (kl, vl), row stride ldp elements, 16-byte aligned rows.
// out is written in natural dim order. Softmax logits are (q.k) / q_prescale.
// max_len: the batch's longest sequence; past kAttnLongSeq tokens the
// long-sequence variant runs (same results, bit for bit).
// part_max (optional, 4 * num_work floats): each item's four waves' largest
// |output|; launch_max_of over them gives the output's maximum.
constexpr int kAttnLongSeq = 256;
hipError_t launch_attention_x3(const uint32_t* q, int ldq, const uint16_t* kh, const uint16_t* kl, const uint16_t* vh,
                               const uint16_t* vl, int ldp, float q_prescale, const int* cu_seqlens,
                               const AttnWork* work, int num_work, float* out, int ld_out, int max_len,
                               hipStream_t s, float* part_max = nullptr);
// fp32 [rows, d] (row stride ld_x, d % 64 == 0) -> that layout: split words
// of x * scale (words != null, row stride ld_out words) or hi / lo planes
// (planes != null: hi at [r * ld_out + c], lo d elements further).
hipError_t launch_pack_x3(const float* x, int ld_x, int rows, int d, float scale, uint32_t* words, uint16_t* planes,
                          int ld_out, hipStream_t s);
// Exact fp32 path for any head_dim <= 128 (one thread per query).
hipError_t launch_attention_f32(const float* q, const float* k, const float* v,
                                int ld, int head_dim, const int* cu_seqlens,
                                const AttnWork* work, int num_work, float* out,
                                int ld_out, hipStream_t s);
constexpr int kAttnMfmaQTile = 128;
constexpr int kAttnF32QTile = 64;

// ------------------------------------------------------------ elementwise
// LayerNorm of x [rows, d]; with resid != null x is first updated in place
// (x += resid) and normalised after the add.
// round16: round each output to the nearest fp16 and back (the reference's
// first-block fc1 escape, src/model.cpp:1028-1033).
// tensor_absmax != null: the maximum |output| is folded into it (atomic
// max); out may then be null (the maximum alone, for
// launch_layernorm_quant_tensor).
hipError_t launch_layernorm(float* x, const float* resid, const float* gamma,
                            const float* beta, float eps, float* out,
                            int rows, int d, float* tensor_absmax,
                            hipStream_t s, int round16 = 0);
// The same LayerNorm (no residual add: x already holds the sum) quantised
// with the per-tensor scale of launch_quant_tensor, scale = absmax / 127 from
// the device value absmax that launch_layernorm folded: the codes and scales
// of launch_layernorm followed by launch_quant_tensor, without the fp32
// output. d % 4 == 0, d <= 2560.
hipError_t launch_layernorm_quant_tensor(float* x, const float* gamma, const float* beta, float eps, int rows, int d,
                                         const float* absmax, int8_t* q, int ldq, float* scales, hipStream_t s,
                                         int round16 = 0);
// LayerNorm (with the same optional residual add) fused with per-token
// symmetric int8 quantisation.
hipError_t launch_layernorm_quant(float* x, const float* resid, const float* gamma,
                                  const float* beta, float eps, int rows,
                                  int d, int8_t* q, int ldq, float* scales,
                                  hipStream_t s, int round16 = 0);
// A residual left as split-K int32 partial sums: planes [splits][rows][d]
// of a GEMM whose dequant epilogue is fma(float(sum), a_scale[row] *
// w_scale[col], bias[col]) (bias may be null).
struct SplitResid {
  const int32_t* planes = nullptr;
  int splits = 0;
  const float* a_scale = nullptr;
  const float* w_scale = nullptr;
  const float* bias = nullptr;
};
// launch_layernorm_quant with its residual given as split-K partial sums:
// the planes are summed and dequantised by that expression, bit for bit the
// GEMM epilogue's value, before the add. r.a_scale may be `scales` itself
// (each row's scale is read before it is written). d % 4 == 0, d <= 2560.
hipError_t launch_layernorm_quant_split(float* x, const SplitResid& r, const float* gamma, const float* beta,
                                        float eps, int rows, int d, int8_t* q, int ldq, float* scales,
                                        hipStream_t s, int round16 = 0);
// GELU (erf of Abramowitz & Stegun 7.1.26) fused with per-token int8
// quantisation of fp32 rows (cols % 4 == 0, cols <= 10240).
hipError_t launch_gelu_quant_rows(const float* x, int ldx, int rows, int cols,
                                  int8_t* q, int ldq, float* scales,
                                  hipStream_t s);
// The same pass over the INT8 GEMM's kEpiF32R24 output (high plane xh, low
// plane xl, row pitch ldx elements): the 24-bit values are exact floats, so
// this is the pass above on them; cols % 64 == 0, cols <= 10240.
hipError_t launch_gelu_quant_rows_r24(const uint16_t* xh, const uint8_t* xl, int ldx, int rows, int cols, int8_t* q,
                                      int ldq, float* scales, hipStream_t s);
// Per-row (per-token) quantisation. src_kind: 0 fp32, 1 fp16, 2 bf16.
hipError_t launch_quant_rows(const void* x, int src_kind, int ldx, int rows,
                             int cols, int8_t* q, int ldq, float* scales,
                             hipStream_t s);
// Per-tensor quantisation with scale = absmax/127 (absmax read on device).
hipError_t launch_quant_tensor(const float* x, int ldx, int rows, int cols,
                               const float* absmax, int8_t* q, int ldq,
                               float* scales, hipStream_t s);
hipError_t launch_absmax(const float* x, size_t n, float* absmax,
                         hipStream_t s);
// *out = the largest of n non-negative floats x (NaNs ignored), one
// workgroup; *out need not be cleared.
hipError_t launch_max_of(const float* x, size_t n, float* out, hipStream_t s);
hipError_t launch_fill_f32(float* x, size_t n, float v, hipStream_t s);
// Activation observer gather: out[w] = |x[pos[w]]| (gelu != 0: |GELU(x[pos[w]])|
// with the Abramowitz & Stegun erf of the fused GELU + quantisation kernel).
hipError_t launch_observe_gather(const float* x, const uint32_t* pos, int count, int gelu, float* out,
                                 hipStream_t s);
// The same (with GELU) over kEpiF32R24's two planes, flat positions
// row * cols + column; cols % 64 == 0.
hipError_t launch_observe_gather_r24(const uint16_t* xh, const uint8_t* xl, int cols, const uint32_t* pos, int count,
                                     float* out, hipStream_t s);
hipError_t launch_gelu(const float* x, float* out, size_t n, hipStream_t s);
hipError_t launch_residual_add(float* y, const float* x, size_t n,
                               hipStream_t s);
hipError_t launch_scale(float* x, size_t n, float scale, hipStream_t s);
// In-place RoPE on fp32 rows: x[t*ld + h*dh + i] for h < heads, each value
// first multiplied by pre_scale (the Q scale; 1 for K).
hipError_t launch_rope_f32(float* x, int ld, const int* pos, int T, int heads,
                           int head_dim, const float* cos_tab,
                           const float* sin_tab, int tab_ld, float pre_scale,
                           hipStream_t s);
hipError_t launch_embed(const int* ids, const float* tok_scale,
                        const float* embed, int T, int d, int mask_token_id,
                        float* out, hipStream_t s);
// fp32 -> bf16 / fp16 conversion (for the MFMA attention op).
hipError_t launch_cast_f32(const float* x, size_t n, uint16_t* out,
                           int to_bf16, hipStream_t s);

// ------------------------------------------- the reference's x86 kernels
// Bit-exact counterparts of the reference's AVX-512 kernels (x86_exact.hip):
// LayerNormAvx512 (optional residual add before, per-tensor absmax and fp16
// rounding after; d <= 2560), GeluAvx512 (optional absmax; in place
// allowed), glibc's expf, ScaleInplace + RopeApplyVarlenAvx512,
// AttentionVarlenAvx512 (head_dim 16, 32 or 64; q/k/v rows at t*ld + h*dh,
// cu_seqlens on the device), LinearAvx512 (C = A W^T + bias with a kF32*
// epilogue; GELU is GeluAvx512).
// launch_layernorm_x86: out may be null for d = 320 or 1280
// (layernorm_x86_rows_ok), the maxima alone; tail_absmax (same widths) also
// receives max |out| of rows >= tail_row.
hipError_t launch_layernorm_x86(float* x, const float* resid, const float* gamma, const float* beta, float eps,
                                float* out, int rows, int d, float* absmax, int round16, hipStream_t s,
                                float* tail_absmax = nullptr, int tail_row = 0x7fffffff);
bool layernorm_x86_rows_ok(int d);
// LayerNormAvx512 of x (no residual) quantised as QuantizeActPrefixAvx512 with
// the per-tensor scale of *absmax, rows >= tail_row with *tail_absmax's: the
// codes and scales of launch_layernorm_x86 then launch_quant_tensor (d = 320
// or 1280, ldq >= d, the codes past d zeroed).
hipError_t launch_layernorm_x86_quant(const float* x, const float* gamma, const float* beta, float eps, int rows,
                                      int d, const float* absmax, const float* tail_absmax, int tail_row, int8_t* q,
                                      int ldq, float* scales, int round16, hipStream_t s);
hipError_t launch_gelu_x86(const float* x, float* out, size_t n, float* absmax, hipStream_t s);
hipError_t launch_expf_glibc(const float* x, float* out, size_t n, hipStream_t s);
hipError_t launch_rope_x86(float* x, int ld, const int* pos, int T, int heads, int head_dim, const float* cos_t,
                           const float* sin_t, int ldt, float scale, hipStream_t s);
bool attention_x86_supported(int head_dim);
// scores: null, or a scratch of attention_x86_score_floats(cu, batch, heads)
// floats (host cu) for the kernel to keep each score and exponential it
// computes instead of recomputing them in the later passes (same results).
// The scratch must fit 32-bit float offsets per head (cu's total below 2^32).
// work: null (every (64-query tile, head, sequence) of a 3-D grid), or
// build_work's list at 64-query tiles without XCD queues (nwork items).
// part_max (with work only, nwork floats): each item's largest |output|.
hipError_t launch_attention_x86(const float* q, const float* k, const float* v, int ld, int head_dim, const int* cu,
                                int batch, int heads, int max_len, float* out, int ldo, hipStream_t s,
                                float* scores = nullptr, const AttnWork* work = nullptr, int nwork = 0,
                                float* part_max = nullptr);
size_t attention_x86_score_floats(const int* cu, int batch, int heads);
hipError_t launch_linear_x86(const float* A, int lda, const float* W, int ldw, const float* bias, float* C, int ldc,
                             int M, int N, int K, int epi, hipStream_t s);

}  // namespace esm_gfx950
