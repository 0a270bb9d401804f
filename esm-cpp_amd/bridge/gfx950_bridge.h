// Reference-side bridge to the gfx950 backend: the code a maintainer of
// esm.cpp adds as src/kernels/gfx950_bridge.{h,cpp} so that the facade's
// `case Isa::Gfx950:` arms (src/kernels/dispatch.cpp:40-262) can forward to
// libesm_gfx950.so. It is compiled against the reference's own headers
// (include/esm_cpp/kernels.h, include/esm_cpp/quant.h), so the signatures
// below are checked against the facade they stand in for.
//
// Every arm takes the facade's arguments in the facade's order, all host
// pointers, stages them on the device, runs the gfx950 kernel and copies the
// result back. It returns false when no gfx950 device is present or the
// device call fails; the facade then takes its CPU arm, the convention
// LinearProj follows for the Apple backends (src/model.cpp:877-905):
//
//   case Isa::Gfx950:
//     if (gfx950::LinearInt8(A, W, bias, C, M, N, K)) return;
//     return LinearInt8Ref(A, W, bias, C, M, N, K);
//
// Threading follows the reference's Model contract (model.h:176-181): one
// process-wide context, one stream; calls from several threads serialise on
// a mutex.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "esm_cpp/batch.h"
#include "esm_cpp/quant.h"
#include "esm_cpp/scheduler.h"
#include "esm_gfx950.h"

namespace esm::gfx950 {

// The process-wide context on device 0, created on first use; null when no
// gfx950 device is present (then every arm returns false).
esm_gfx950_ctx* Ctx();

// The last device error message ("" when none).
const char* LastError();

// esm::kernels::Linear (kernels.h:19-20).
bool Linear(const float* A, const float* W, const float* bias, float* C, int M, int N, int K);

// esm::kernels::LinearInt8 (kernels.h:56-57, dispatch.cpp:80-103) with the
// reference's dynamic per-tensor activation scale. The weight's device copy
// is built on first use (BuildKernelCache's role, pack.cpp:107-117) and kept
// until ReleaseWeight or exit. It is found again by the tensor's address and
// checked against its packed data pointer, shape, a checksum of its scales
// and a checksum of 4096 of its int8 values spread evenly over the tensor;
// a change in place that none of these sees (a few int8 values rewritten)
// keeps the old device copy, so call ReleaseWeight after changing a tensor in
// place and before destroying it (the integration that owns QuantizedTensor
// frees the copy in its destructor).
bool LinearInt8(const float* A, const esm::quant::QuantizedTensor& W, const float* bias, float* C, int M, int N,
                int K);
void ReleaseWeight(const esm::quant::QuantizedTensor& W);

// esm::kernels::LayerNorm (kernels.h:32-33).
bool LayerNorm(const float* x, const float* gamma, const float* beta, float eps, float* out, int num_rows, int d);

// esm::kernels::Gelu (kernels.h:35).
bool Gelu(const float* x, float* out, std::size_t n);

// esm::kernels::ResidualAddInplace (kernels.h:24) and ScaleInplace (:29).
bool ResidualAddInplace(float* y, const float* x, std::size_t n);
bool ScaleInplace(float* x, std::size_t n, float scale);

// esm::kernels::RopeApplyVarlen (kernels.h:90-92): x [T, H, head_dim] in
// place; cos/sin [max_seqlen, head_dim], of which the rows up to the longest
// sequence of cu_seqlens are read.
bool RopeApplyVarlen(float* x, const float* cos, const float* sin, const int* cu_seqlens, int batch_size,
                     int num_heads, int head_dim);

// esm::kernels::AttentionVarlen (kernels.h:119-121): the split-fp16 MFMA
// kernel at head_dim 64 (fp32-level results), the scalar fp32 kernel for any
// other head_dim <= 128.
bool AttentionVarlen(const float* q, const float* k, const float* v, const int* cu_seqlens, int batch_size,
                     int num_heads, int head_dim, float* out);

// Model::ForwardPackedInto's device path (model.cpp:1093-1255) for a model
// built on the device (esm_gfx950_model_create from the Model's tensors, or
// esm_gfx950_model_create_from_gguf): the packed forward of `batch`, masks
// included (pads: esm_gfx950_forward_packed_masked), split into one logits
// buffer per sequence, each [L_b * vocab_size], as model.cpp:1240-1252 does.
// hidden_packed_out (nullable) receives num_hidden_layers + 1 packed [T, d]
// states in ForwardPackedInto's layout (:1149-1189). An empty batch clears
// logits_per_seq_out. Returns false when the device call fails.
bool ForwardPacked(esm_gfx950_model* model, const esm::BatchView& batch,
                   std::vector<std::vector<float>>* logits_per_seq_out,
                   std::vector<std::vector<float>>* hidden_packed_out = nullptr);

// Model::ForwardScheduled's device path (model.cpp:1298-1421): the
// sequences planned as PlanBatches does (scheduler.cpp:54-75) and returned
// in input order, one [L_i * vocab_size] buffer each. Without masks the
// library runs the groups pipelined (esm_gfx950_forward_scheduled); with
// masks (attention_masks.size() == input_ids.size()) each planned group runs
// as one masked packed forward. Returns false when the device call fails or
// the mask list does not match (the reference throws; the caller decides).
bool ForwardScheduled(esm_gfx950_model* model, const std::vector<std::vector<std::int32_t>>& input_ids,
                      const std::vector<std::vector<std::int32_t>>& attention_masks,
                      const esm::SchedulerConfig& cfg, std::vector<std::vector<float>>* out);

}  // namespace esm::gfx950
