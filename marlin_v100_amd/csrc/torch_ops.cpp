// torch_ops.cpp -- thin TORCH_LIBRARY binding of the reference op schemas over the C ABI.
//
// Built twice: with MMI_EXT_NAME=_C it registers torch.ops._C.{marlin_gemm,
// gptq_marlin_repack, awq_marlin_repack, marlin_int4_fp8_preprocess} (schemas byte-identical to the reference
// csrc/torch_bindings_marlin.cpp:6-21); with MMI_EXT_NAME=_moe_C it registers
// torch.ops._moe_C.{topk_softmax, topk_sigmoid, grouped_topk, moe_align_block_size,
// moe_wna16_marlin_gemm, moe_sum} (csrc/moe/torch_bindings_marlin.cpp:5-54).  The _C build also registers the inspection op
// torch.ops._marlin_mi355x.dequantize.  Tensor-level checks (device, contiguity, ranks,
// shapes) mirror the reference's TORCH_CHECKs; everything else is validated by the C ABI,
// whose messages are rethrown unchanged.
#include <Python.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/all.h>
#include <torch/library.h>

#include "../../include/marlin_mi355x.h"

#ifndef MMI_EXT_NAME
#error "MMI_EXT_NAME must be _C or _moe_C"
#endif
#define MMI_STR2(x) #x
#define MMI_STR(x) MMI_STR2(x)

namespace {

marlin_dtype_t to_mdt(at::ScalarType t) {
  switch (t) {
    case at::kHalf: return MARLIN_DTYPE_FLOAT16;
    case at::kBFloat16: return MARLIN_DTYPE_BFLOAT16;
    case at::kFloat: return MARLIN_DTYPE_FLOAT32;
    case at::kFloat8_e4m3fn: return MARLIN_DTYPE_FLOAT8_E4M3FN;
    case at::kFloat8_e8m0fnu: return MARLIN_DTYPE_FLOAT8_E8M0FNU;
    case at::kInt: return MARLIN_DTYPE_INT32;
    case at::kLong: return MARLIN_DTYPE_INT64;
    case at::kByte: return MARLIN_DTYPE_UINT8;
    case at::kChar: return MARLIN_DTYPE_INT8;
    case at::kUInt32: return MARLIN_DTYPE_UINT32;
    default: return (marlin_dtype_t)-1;
  }
}

marlin_stream_t cur_stream(const at::Tensor& t) {
  return reinterpret_cast<marlin_stream_t>(
      c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void rethrow(marlin_status_t st) {
  TORCH_CHECK(st == MARLIN_STATUS_OK, marlin_get_last_error());
}

const void* opt_ptr(const std::optional<at::Tensor>& t) {
  return (t.has_value() && t->numel() > 0) ? t->data_ptr() : nullptr;
}
int64_t opt_numel(const std::optional<at::Tensor>& t) { return t.has_value() ? t->numel() : 0; }
marlin_dtype_t opt_dtype(const std::optional<at::Tensor>& t) {
  return t.has_value() ? to_mdt(t->scalar_type()) : MARLIN_DTYPE_FLOAT16;
}

void check_cuda_contig(const std::optional<at::Tensor>& t, const char* name) {
  if (!t.has_value()) return;
  TORCH_CHECK(t->device().is_cuda(), name, " is not on GPU");
  TORCH_CHECK(t->is_contiguous(), name, " is not contiguous");
}

}  // namespace

#if defined(MMI_BUILD_C)

// reference gptq_marlin_repack.cu:399-469
at::Tensor op_gptq_marlin_repack(at::Tensor& b_q_weight, at::Tensor& perm, int64_t size_k,
                              int64_t size_n, int64_t num_bits, bool is_a_8bit) {
  TORCH_CHECK(num_bits == 4 || num_bits == 8, "num_bits must be 4 or 8. Got = ", num_bits);
  const int64_t pack = 32 / num_bits;
  TORCH_CHECK((size_k / pack) == b_q_weight.size(0), "Shape mismatch: b_q_weight.size(0) = ",
              b_q_weight.size(0), ", size_k = ", size_k, ", pack_factor = ", pack);
  TORCH_CHECK(b_q_weight.size(1) == size_n, "b_q_weight.size(1) = ", b_q_weight.size(1),
              " is not size_n = ", size_n);
  TORCH_CHECK(b_q_weight.device().is_cuda(), "b_q_weight is not on GPU");
  TORCH_CHECK(b_q_weight.is_contiguous(), "b_q_weight is not contiguous");
  TORCH_CHECK(b_q_weight.dtype() == at::kInt, "b_q_weight type is not kInt");
  TORCH_CHECK(perm.device().is_cuda(), "perm is not on GPU");
  TORCH_CHECK(perm.is_contiguous(), "perm is not contiguous");
  TORCH_CHECK(perm.dtype() == at::kInt, "perm type is not at::kInt");
  const at::OptionalDeviceGuard guard(b_q_weight.device());
  at::Tensor out = torch::empty({size_k / 16, size_n * 16 / pack}, b_q_weight.options());
  rethrow(marlin_gptq_marlin_repack(b_q_weight.data_ptr<int32_t>(), b_q_weight.numel(),
                                    perm.numel() ? perm.data_ptr<int32_t>() : nullptr,
                                    perm.numel(), size_k, size_n, num_bits, is_a_8bit,
                                    out.data_ptr<int32_t>(), out.numel(), cur_stream(b_q_weight)));
  return out;
}

// reference awq_marlin_repack.cu:300-381
at::Tensor op_awq_marlin_repack(at::Tensor& b_q_weight, int64_t size_k, int64_t size_n,
                             int64_t num_bits, bool is_a_8bit) {
  TORCH_CHECK(num_bits == 4 || num_bits == 8, "num_bits must be 4 or 8. Got = ", num_bits);
  const int64_t pack = 32 / num_bits;
  TORCH_CHECK(b_q_weight.size(0) == size_k, "b_q_weight.size(0) = ", b_q_weight.size(0),
              " is not size_k = ", size_k);
  TORCH_CHECK((size_n / pack) == b_q_weight.size(1), "Shape mismatch: b_q_weight.size(1) = ",
              b_q_weight.size(1), ", size_n = ", size_n, ", pack_factor = ", pack);
  TORCH_CHECK(b_q_weight.device().is_cuda(), "b_q_weight is not on GPU");
  TORCH_CHECK(b_q_weight.is_contiguous(), "b_q_weight is not contiguous");
  TORCH_CHECK(b_q_weight.dtype() == at::kInt, "b_q_weight type is not kInt");
  const at::OptionalDeviceGuard guard(b_q_weight.device());
  at::Tensor out = torch::empty({size_k / 16, size_n * 16 / pack}, b_q_weight.options());
  rethrow(marlin_awq_marlin_repack(b_q_weight.data_ptr<int32_t>(), b_q_weight.numel(), size_k,
                                   size_n, num_bits, is_a_8bit, out.data_ptr<int32_t>(),
                                   out.numel(), cur_stream(b_q_weight)));
  return out;
}

// reference marlin_int4_fp8_preprocess.cu:58-97
at::Tensor op_marlin_int4_fp8_preprocess(at::Tensor& qweight,
                                         std::optional<at::Tensor> qzeros_or_none, bool inplace) {
  TORCH_CHECK(qweight.device().is_cuda(), "qweight is not on GPU");
  TORCH_CHECK(qweight.scalar_type() == at::ScalarType::Int, "qweight.dtype != torch.int32");
  TORCH_CHECK(qweight.is_contiguous(), "qweight is not contiguous");
  const at::OptionalDeviceGuard guard(qweight.device());
  at::Tensor output = inplace ? qweight : torch::empty_like(qweight);
  const int64_t rows = qweight.dim() >= 1 ? qweight.size(0) : 1;
  const int64_t cols = rows ? qweight.numel() / rows : 0;
  if (!qzeros_or_none.has_value()) {
    rethrow(marlin_int4_fp8_preprocess(qweight.data_ptr<int32_t>(), rows, cols, nullptr, 0, 0,
                                       output.data_ptr<int32_t>(), cur_stream(qweight)));
    return output;
  }
  at::Tensor qzeros = *qzeros_or_none;
  TORCH_CHECK(qweight.dim() == 2, "qweight must be [size_k, size_n / 8] with qzeros");
  TORCH_CHECK(qzeros.device().is_cuda(), "qzeros is not on GPU");
  TORCH_CHECK(qzeros.scalar_type() == at::ScalarType::Int, "qweight.dtype != torch.int32");
  TORCH_CHECK(qzeros.device() == qweight.device(),
              "qzeros is not on the same device with qweight");
  TORCH_CHECK(qzeros.dim() == 2 && qzeros.is_contiguous(), "qzeros must be a contiguous 2-D tensor");
  rethrow(marlin_int4_fp8_preprocess(qweight.data_ptr<int32_t>(), qweight.size(0),
                                     qweight.size(1), qzeros.data_ptr<int32_t>(), qzeros.size(0),
                                     qzeros.size(1), output.data_ptr<int32_t>(),
                                     cur_stream(qweight)));
  return output;
}

// reference marlin.cu:83-506
at::Tensor op_marlin_gemm(at::Tensor& a, std::optional<at::Tensor> c_or_none, at::Tensor& b_q_weight,
                       std::optional<at::Tensor> const& b_bias_or_none, at::Tensor& b_scales,
                       std::optional<at::Tensor> const& a_scales_or_none,
                       std::optional<at::Tensor> const& global_scale_or_none,
                       std::optional<at::Tensor> const& b_zeros_or_none,
                       std::optional<at::Tensor> const& g_idx_or_none,
                       std::optional<at::Tensor> const& perm_or_none, at::Tensor& workspace,
                       int64_t b_type_id, int64_t size_m, int64_t size_n, int64_t size_k,
                       bool is_k_full, bool use_atomic_add, bool use_fp32_reduce,
                       bool is_zp_float) {
  TORCH_CHECK(a.scalar_type() == at::kHalf || a.scalar_type() == at::kBFloat16,
              "only float16 and bfloat16 activations are supported (8-bit activations are not "
              "implemented).");
  TORCH_CHECK(a.size(0) == size_m, "Shape mismatch: a.size(0) = ", a.size(0), ", size_m = ",
              size_m);
  TORCH_CHECK(a.size(1) == size_k, "Shape mismatch: a.size(1) = ", a.size(1), ", size_k = ",
              size_k);
  TORCH_CHECK(size_k % 16 == 0, "size_k = ", size_k, " is not divisible by tile_size = ", 16);
  TORCH_CHECK(b_q_weight.dim() == 2, "b_q_weight rank must be 2");
  TORCH_CHECK((size_k / 16) == b_q_weight.size(0), "Shape mismatch: b_q_weight.size(0) = ",
              b_q_weight.size(0), ", size_k = ", size_k, ", tile_size = ", 16);
  TORCH_CHECK(b_q_weight.size(1) % 16 == 0, "b_q_weight.size(1) = ", b_q_weight.size(1),
              " is not divisible by tile_size = ", 16);
  TORCH_CHECK(a.device().is_cuda(), "A is not on GPU");
  TORCH_CHECK(a.stride(1) == 1, "A.stride(1) is not 1");
  TORCH_CHECK(b_q_weight.device().is_cuda(), "b_q_weight is not on GPU");
  TORCH_CHECK(b_q_weight.is_contiguous(), "b_q_weight is not contiguous");
  TORCH_CHECK(b_q_weight.scalar_type() == at::kInt, "expects int32 packed weights.");
  TORCH_CHECK(b_scales.device().is_cuda(), "b_scales is not on GPU");
  TORCH_CHECK(b_scales.is_contiguous(), "b_scales is not contiguous");
  TORCH_CHECK(b_scales.dim() == 2, "b_scales rank = ", b_scales.dim(), " is not 2");
  TORCH_CHECK(b_scales.size(1) == size_n, "b_scales dim 1 = ", b_scales.size(1),
              " is not size_n = ", size_n);
  check_cuda_contig(global_scale_or_none, "global_scale");
  check_cuda_contig(b_bias_or_none, "b_bias");
  check_cuda_contig(b_zeros_or_none, "b_zeros");
  if (global_scale_or_none.has_value())
    TORCH_CHECK(global_scale_or_none->scalar_type() == at::kFloat,
                "nvfp4 expects fp32 global_scale.");
  if (b_bias_or_none.has_value()) {
    TORCH_CHECK(b_bias_or_none->scalar_type() == a.scalar_type(),
                "b_bias must have the activation dtype.");
    TORCH_CHECK(b_bias_or_none->size(0) == size_n, "b_bias.size(0) != size_n");
  }
  if (b_zeros_or_none.has_value() && b_zeros_or_none->size(-1) > 0) {
    TORCH_CHECK(b_zeros_or_none->dim() == 2, "b_zeros rank = ", b_zeros_or_none->dim(),
                " is not 2");
    // float zero points [G, N]; packed integer zero points [G, N / pack_factor] int32
    // (ScalarType id: exponent | mantissa << 8 | signed << 16 ..., vllm/scalar_type.py:25-43)
    const int64_t bits = (b_type_id & 0xff) + ((b_type_id >> 8) & 0xff) + ((b_type_id >> 16) & 1);
    const int64_t zn = is_zp_float ? size_n : size_n / (32 / std::max<int64_t>(bits, 1));
    TORCH_CHECK(b_zeros_or_none->size(1) == zn, "b_zeros dim 1 = ", b_zeros_or_none->size(1),
                " is not ", is_zp_float ? "size_n = " : "size_n / pack_factor = ", zn);
    TORCH_CHECK(b_zeros_or_none->size(0) == b_scales.size(0), "b_zeros dim 0 = ",
                b_zeros_or_none->size(0), " is not num_groups = ", b_scales.size(0));
  }
  check_cuda_contig(g_idx_or_none, "g_idx");
  check_cuda_contig(perm_or_none, "perm");
  const bool act = (g_idx_or_none.has_value() && g_idx_or_none->numel() > 0) ||
                   (perm_or_none.has_value() && perm_or_none->numel() > 0);
  if (act) {
    TORCH_CHECK(g_idx_or_none.has_value() && g_idx_or_none->scalar_type() == at::kInt,
                "g_idx must be int32");
    TORCH_CHECK(perm_or_none.has_value() && perm_or_none->scalar_type() == at::kInt,
                "perm must be int32");
  }

  const at::OptionalDeviceGuard guard(a.device());
  at::Tensor c;
  if (c_or_none.has_value()) {
    c = c_or_none.value();
    TORCH_CHECK(c.device().is_cuda(), "c is not on GPU");
    TORCH_CHECK(c.is_contiguous(), "c is not contiguous");
    TORCH_CHECK(c.scalar_type() == a.scalar_type(),
                "scalar type of a must be the same with c for 16 bit activation");
    TORCH_CHECK(c.size(0) == size_m, "Shape mismatch: c.size(0) = ", c.size(0), ", size_m = ",
                size_m);
    TORCH_CHECK(c.size(1) == size_n, "Shape mismatch: c.size(1) = ", c.size(1), ", size_n = ",
                size_n);
  } else {
    c = torch::empty({size_m, size_n}, a.options());
  }
  if (size_m == 0) return c;

  const int64_t zeros_numel =
      (b_zeros_or_none.has_value() && b_zeros_or_none->size(-1) > 0) ? b_zeros_or_none->numel() : 0;
  rethrow(marlin_gemm(a.data_ptr(), to_mdt(a.scalar_type()), a.stride(0), c.data_ptr(),
                      b_q_weight.data_ptr<int32_t>(), b_q_weight.numel(), opt_ptr(b_bias_or_none),
                      opt_numel(b_bias_or_none), b_scales.data_ptr(),
                      to_mdt(b_scales.scalar_type()), b_scales.numel(), b_scales.size(0),
                      opt_numel(a_scales_or_none),
                      reinterpret_cast<const float*>(opt_ptr(global_scale_or_none)),
                      opt_numel(global_scale_or_none), opt_ptr(b_zeros_or_none),
                      opt_dtype(b_zeros_or_none), zeros_numel,
                      reinterpret_cast<const int32_t*>(opt_ptr(g_idx_or_none)),
                      opt_numel(g_idx_or_none),
                      reinterpret_cast<const int32_t*>(opt_ptr(perm_or_none)),
                      opt_numel(perm_or_none), workspace.numel() ? workspace.data_ptr() : nullptr,
                      workspace.nbytes(), b_type_id, size_m, size_n, size_k, is_k_full,
                      use_atomic_add, use_fp32_reduce, is_zp_float, cur_stream(a)));
  return c;
}

// Inspection op: dequantize repacked weights with the GEMM's device routines.
at::Tensor mmi_dequantize(at::Tensor& b_q_weight, at::Tensor& b_scales,
                          std::optional<at::Tensor> const& b_zeros_or_none,
                          std::optional<at::Tensor> const& global_scale_or_none,
                          int64_t b_type_id, int64_t size_k, int64_t size_n,
                          at::ScalarType out_dtype) {
  TORCH_CHECK(b_q_weight.is_cuda() && b_q_weight.is_contiguous(), "b_q_weight");
  TORCH_CHECK(b_scales.is_cuda() && b_scales.is_contiguous() && b_scales.dim() == 2 &&
                  b_scales.size(1) == size_n,
              "b_scales must be a contiguous [num_groups, size_n] GPU tensor");
  check_cuda_contig(b_zeros_or_none, "b_zeros");
  check_cuda_contig(global_scale_or_none, "global_scale");
  const at::OptionalDeviceGuard guard(b_q_weight.device());
  at::Tensor out = torch::empty({size_k, size_n}, b_q_weight.options().dtype(out_dtype));
  rethrow(marlin_dequantize(b_q_weight.data_ptr<int32_t>(), b_q_weight.numel(),
                            b_scales.data_ptr(), to_mdt(b_scales.scalar_type()), b_scales.numel(),
                            b_scales.size(0), opt_ptr(b_zeros_or_none), opt_dtype(b_zeros_or_none),
                            opt_numel(b_zeros_or_none),
                            reinterpret_cast<const float*>(opt_ptr(global_scale_or_none)),
                            opt_numel(global_scale_or_none), b_type_id, size_k, size_n,
                            to_mdt(out_dtype), out.data_ptr(), cur_stream(b_q_weight)));
  return out;
}

TORCH_LIBRARY(_C, ops) {
  ops.def(
      "marlin_gemm(Tensor a, Tensor? c_or_none, Tensor b_q_weight, "
      "Tensor? b_bias_or_none,Tensor b_scales, "
      "Tensor? a_scales, Tensor? global_scale, Tensor? b_zeros_or_none, "
      "Tensor? g_idx_or_none, Tensor? perm_or_none, Tensor workspace, "
      "int b_type_id, SymInt size_m, SymInt size_n, SymInt size_k, "
      "bool is_k_full, bool use_atomic_add, bool use_fp32_reduce, "
      "bool is_zp_float) -> Tensor");
  ops.def(
      "gptq_marlin_repack(Tensor b_q_weight, Tensor perm, "
      "SymInt size_k, SymInt size_n, int num_bits, bool is_a_8bit) -> Tensor");
  ops.def(
      "awq_marlin_repack(Tensor b_q_weight, SymInt size_k, "
      "SymInt size_n, int num_bits, bool is_a_8bit) -> Tensor");
  ops.def(
      "marlin_int4_fp8_preprocess(Tensor qweight, "
      "Tensor? qzeros_or_none, bool inplace) -> Tensor");
}

TORCH_LIBRARY_IMPL(_C, CUDA, ops) {
  ops.impl("marlin_gemm", &op_marlin_gemm);
  ops.impl("gptq_marlin_repack", &op_gptq_marlin_repack);
  ops.impl("awq_marlin_repack", &op_awq_marlin_repack);
  ops.impl("marlin_int4_fp8_preprocess", &op_marlin_int4_fp8_preprocess);
}

TORCH_LIBRARY(_marlin_mi355x, ops) {
  ops.def(
      "dequantize(Tensor b_q_weight, Tensor b_scales, Tensor? b_zeros, Tensor? global_scale, "
      "int b_type_id, SymInt size_k, SymInt size_n, ScalarType out_dtype) -> Tensor");
}
TORCH_LIBRARY_IMPL(_marlin_mi355x, CUDA, ops) { ops.impl("dequantize", &mmi_dequantize); }

#elif defined(MMI_BUILD_MOE_C)

// reference moe_align_sum_kernels.cu:477-569
void op_moe_align_block_size(at::Tensor topk_ids, int64_t num_experts, int64_t block_size,
                          at::Tensor sorted_token_ids, at::Tensor experts_ids,
                          at::Tensor num_tokens_post_pad,
                          std::optional<at::Tensor> maybe_expert_map) {
  TORCH_CHECK(topk_ids.is_cuda() && topk_ids.is_contiguous(), "topk_ids must be a contiguous GPU tensor");
  TORCH_CHECK(topk_ids.scalar_type() == at::kInt || topk_ids.scalar_type() == at::kLong,
              "topk_ids must be int32 or int64");
  for (const at::Tensor* t : {&sorted_token_ids, &experts_ids, &num_tokens_post_pad}) {
    TORCH_CHECK(t->is_cuda() && t->is_contiguous() && t->scalar_type() == at::kInt,
                "moe_align_block_size outputs must be contiguous int32 GPU tensors");
  }
  if (maybe_expert_map.has_value()) {
    TORCH_CHECK(maybe_expert_map->is_cuda() && maybe_expert_map->is_contiguous() &&
                    maybe_expert_map->scalar_type() == at::kInt,
                "expert_map must be a contiguous int32 GPU tensor");
  }
  const at::OptionalDeviceGuard guard(topk_ids.device());
  rethrow(marlin_moe_align_block_size(
      topk_ids.data_ptr(), to_mdt(topk_ids.scalar_type()), topk_ids.numel(), num_experts,
      block_size, sorted_token_ids.data_ptr<int32_t>(), sorted_token_ids.numel(),
      experts_ids.data_ptr<int32_t>(), experts_ids.numel(), num_tokens_post_pad.data_ptr<int32_t>(),
      maybe_expert_map.has_value() ? maybe_expert_map->data_ptr<int32_t>() : nullptr,
      opt_numel(maybe_expert_map), cur_stream(topk_ids)));
}

// reference csrc/moe/marlin_moe_wna16/ops.cu:102-529
at::Tensor op_moe_wna16_marlin_gemm(
    at::Tensor& a, std::optional<at::Tensor> c_or_none, at::Tensor& b_q_weight,
    std::optional<at::Tensor> const& b_bias_or_none, at::Tensor& b_scales,
    std::optional<at::Tensor> const& a_scales_or_none,
    std::optional<at::Tensor> const& global_scale_or_none,
    std::optional<at::Tensor> const& b_zeros_or_none,
    std::optional<at::Tensor> const& g_idx_or_none, std::optional<at::Tensor> const& perm_or_none,
    at::Tensor& workspace, at::Tensor& sorted_token_ids, at::Tensor& expert_ids,
    at::Tensor& num_tokens_past_padded, at::Tensor& topk_weights, int64_t moe_block_size,
    int64_t top_k, bool mul_topk_weights, int64_t b_type_id, int64_t size_m, int64_t size_n,
    int64_t size_k, bool is_k_full, bool use_atomic_add, bool use_fp32_reduce, bool is_zp_float,
    int64_t thread_k, int64_t thread_n, int64_t blocks_per_sm) {
  TORCH_CHECK(a.scalar_type() == at::kHalf || a.scalar_type() == at::kBFloat16,
              "only float16 and bfloat16 activations are supported (8-bit activations are not "
              "implemented).");
  TORCH_CHECK(a.size(0) == size_m, "Shape mismatch: a.size(0) = ", a.size(0), ", size_m = ",
              size_m);
  TORCH_CHECK(a.size(1) == size_k, "Shape mismatch: a.size(1) = ", a.size(1), ", size_k = ",
              size_k);
  TORCH_CHECK(size_k % 16 == 0, "size_k = ", size_k, " is not divisible by tile_size = ", 16);
  TORCH_CHECK(b_q_weight.dim() == 3, "b_q_weight rank must be 3");
  TORCH_CHECK((size_k / 16) == b_q_weight.size(1), "Shape mismatch: b_q_weight.size(1) = ",
              b_q_weight.size(1), ", size_k = ", size_k, ", tile_size = ", 16);
  TORCH_CHECK(b_q_weight.size(2) % 16 == 0, "b_q_weight.size(2) = ", b_q_weight.size(2),
              " is not divisible by tile_size = ", 16);
  TORCH_CHECK(a.device().is_cuda(), "A is not on GPU");
  TORCH_CHECK(a.is_contiguous(), "A is not contiguous");
  TORCH_CHECK(b_q_weight.device().is_cuda(), "b_q_weight is not on GPU");
  TORCH_CHECK(b_q_weight.is_contiguous(), "b_q_weight is not contiguous");
  TORCH_CHECK(b_q_weight.scalar_type() == at::kInt, "expects int32 packed weights.");
  TORCH_CHECK(b_scales.device().is_cuda(), "b_scales is not on GPU");
  TORCH_CHECK(b_scales.is_contiguous(), "b_scales is not contiguous");
  TORCH_CHECK(b_scales.dim() == 3, "b_scales rank = ", b_scales.dim(), " is not 3");
  TORCH_CHECK(b_scales.size(2) == size_n, "b_scales dim 2 = ", b_scales.size(2),
              " is not size_n = ", size_n);
  const int64_t num_experts = b_q_weight.size(0);
  check_cuda_contig(global_scale_or_none, "global_scale");
  check_cuda_contig(b_bias_or_none, "b_bias");
  check_cuda_contig(b_zeros_or_none, "b_zeros");
  if (global_scale_or_none.has_value())
    TORCH_CHECK(global_scale_or_none->scalar_type() == at::kFloat,
                "nvfp4 expects fp32 global_scale.");
  if (b_bias_or_none.has_value()) {
    TORCH_CHECK(b_bias_or_none->scalar_type() == a.scalar_type(),
                "b_bias must have the activation dtype.");
    TORCH_CHECK(b_bias_or_none->size(0) == num_experts, "b_bias.size(0) != num_experts");
    TORCH_CHECK(b_bias_or_none->size(1) == size_n, "b_bias.size(1) != size_n");
  }
  if (b_zeros_or_none.has_value() && b_zeros_or_none->size(-1) > 0) {
    TORCH_CHECK(b_zeros_or_none->dim() == 3, "b_zeros rank = ", b_zeros_or_none->dim(),
                " is not 3");
    TORCH_CHECK(b_zeros_or_none->size(0) == num_experts, "b_zeros dim 0 = ",
                b_zeros_or_none->size(0), " is not num_experts = ", num_experts);
    TORCH_CHECK(b_zeros_or_none->size(1) == b_scales.size(1), "b_zeros dim 1 = ",
                b_zeros_or_none->size(1), " is not num_groups = ", b_scales.size(1));
    TORCH_CHECK(b_zeros_or_none->size(2) == size_n, "b_zeros dim 2 = ", b_zeros_or_none->size(2),
                " is not size_n = ", size_n);
  }
  for (const at::Tensor* t : {&sorted_token_ids, &expert_ids, &num_tokens_past_padded}) {
    TORCH_CHECK(t->is_cuda() && t->is_contiguous() && t->scalar_type() == at::kInt,
                "sorted_token_ids / expert_ids / num_tokens_past_padded must be contiguous "
                "int32 GPU tensors");
  }
  TORCH_CHECK(topk_weights.is_cuda() && topk_weights.is_contiguous() &&
                  topk_weights.scalar_type() == at::kFloat,
              "topk_weights must be a contiguous float32 GPU tensor");

  const at::OptionalDeviceGuard guard(a.device());
  at::Tensor c;
  if (c_or_none.has_value()) {
    c = c_or_none.value();
    TORCH_CHECK(c.device().is_cuda(), "c is not on GPU");
    TORCH_CHECK(c.is_contiguous(), "c is not contiguous");
    TORCH_CHECK(c.size(0) == size_m * top_k, "Shape mismatch: c.size(0) = ", c.size(0),
                ", size_m * topk = ", size_m * top_k);
    TORCH_CHECK(c.size(1) == size_n, "Shape mismatch: c.size(1) = ", c.size(1), ", size_n = ",
                size_n);
    TORCH_CHECK(c.scalar_type() == a.scalar_type(),
                "scalar type of a must be the same with c for 16 bit activation");
  } else {
    c = torch::empty({size_m * top_k, size_n}, a.options());
  }
  const int64_t zeros_numel =
      (b_zeros_or_none.has_value() && b_zeros_or_none->size(-1) > 0) ? b_zeros_or_none->numel() : 0;
  rethrow(marlin_moe_wna16_marlin_gemm(
      a.data_ptr(), to_mdt(a.scalar_type()), c.data_ptr(), b_q_weight.data_ptr<int32_t>(),
      b_q_weight.numel(), num_experts, opt_ptr(b_bias_or_none), opt_numel(b_bias_or_none),
      b_scales.data_ptr(), to_mdt(b_scales.scalar_type()), b_scales.numel(), b_scales.size(1),
      opt_numel(a_scales_or_none), reinterpret_cast<const float*>(opt_ptr(global_scale_or_none)),
      opt_numel(global_scale_or_none), opt_ptr(b_zeros_or_none), opt_dtype(b_zeros_or_none),
      zeros_numel, opt_numel(g_idx_or_none), opt_numel(perm_or_none),
      workspace.numel() ? workspace.data_ptr() : nullptr, workspace.nbytes(),
      sorted_token_ids.data_ptr<int32_t>(), sorted_token_ids.numel(), expert_ids.data_ptr<int32_t>(),
      expert_ids.numel(), num_tokens_past_padded.data_ptr<int32_t>(), topk_weights.data_ptr<float>(),
      topk_weights.numel(), moe_block_size, top_k, mul_topk_weights, b_type_id, size_m, size_n,
      size_k, is_k_full, use_atomic_add, use_fp32_reduce, is_zp_float, thread_k, thread_n,
      blocks_per_sm, cur_stream(a)));
  return c;
}

// upstream vLLM moe_sum: output[t, :] = sum over top_k of input[t, k, :]
void op_moe_sum(at::Tensor& input, at::Tensor& output) {
  TORCH_CHECK(input.is_cuda() && input.is_contiguous() && input.dim() == 3,
              "input must be a contiguous [tokens, topk, hidden] GPU tensor");
  TORCH_CHECK(output.is_cuda() && output.is_contiguous() && output.dim() == 2,
              "output must be a contiguous [tokens, hidden] GPU tensor");
  TORCH_CHECK(output.scalar_type() == input.scalar_type(), "dtype mismatch");
  TORCH_CHECK(output.size(0) == input.size(0) && output.size(1) == input.size(2), "shape mismatch");
  const at::OptionalDeviceGuard guard(input.device());
  rethrow(marlin_moe_sum(input.data_ptr(), to_mdt(input.scalar_type()), input.size(0),
                         input.size(1), input.size(2), output.data_ptr(), cur_stream(input)));
}

// reference topk_softmax / topk_sigmoid (csrc/moe/topk_softmax_kernels.cu:773-847): outputs
// are caller-allocated [tokens, topk]; topk = topk_weights.size(-1), experts =
// gating_output.size(-1), tokens = gating_output.numel() / experts.
template <bool Sigmoid>
void op_topk_gating(at::Tensor& topk_weights, at::Tensor& topk_indices,
                    at::Tensor& token_expert_indices, at::Tensor& gating_output, bool renormalize,
                    std::optional<at::Tensor> bias) {
  TORCH_CHECK(gating_output.is_cuda() && gating_output.is_contiguous(),
              "gating_output must be a contiguous GPU tensor");
  const int64_t num_experts = gating_output.size(-1);
  TORCH_CHECK(num_experts > 0, "gating_output has no experts");
  const int64_t num_tokens = gating_output.numel() / num_experts;
  const int64_t topk = topk_weights.size(-1);
  TORCH_CHECK(topk_weights.is_cuda() && topk_weights.is_contiguous() &&
                  topk_weights.scalar_type() == at::kFloat,
              "topk_weights must be a contiguous float32 GPU tensor");
  TORCH_CHECK(topk_indices.is_cuda() && topk_indices.is_contiguous(),
              "topk_indices must be a contiguous GPU tensor");
  TORCH_CHECK(token_expert_indices.is_cuda() && token_expert_indices.is_contiguous() &&
                  token_expert_indices.scalar_type() == at::kInt,
              "token_expert_indices must be a contiguous int32 GPU tensor");
  for (const at::Tensor* t : {&topk_weights, &topk_indices, &token_expert_indices}) {
    TORCH_CHECK(t->numel() == num_tokens * topk, "router output shape mismatch: expected ",
                num_tokens, " x ", topk, " elements");
  }
  if (bias.has_value()) {
    TORCH_CHECK(bias->scalar_type() == at::kFloat, "bias tensor must be float32");
    TORCH_CHECK(bias->dim() == 1, "bias tensor must be 1D");
    TORCH_CHECK(bias->size(0) == num_experts, "bias size mismatch, expected: ", num_experts);
    TORCH_CHECK(bias->is_contiguous(), "bias tensor must be contiguous");
    TORCH_CHECK(bias->is_cuda(), "bias tensor must be on the GPU");
  }
  TORCH_CHECK(to_mdt(topk_indices.scalar_type()) == MARLIN_DTYPE_INT32 ||
                  to_mdt(topk_indices.scalar_type()) == MARLIN_DTYPE_UINT32 ||
                  to_mdt(topk_indices.scalar_type()) == MARLIN_DTYPE_INT64,
              "topk_indices must be int32, uint32 or int64");
  const at::OptionalDeviceGuard guard(gating_output.device());
  const auto fn = Sigmoid ? marlin_topk_sigmoid : marlin_topk_softmax;
  rethrow(fn(topk_weights.data_ptr<float>(), topk_indices.data_ptr(),
             to_mdt(topk_indices.scalar_type()), token_expert_indices.data_ptr<int32_t>(), topk,
             gating_output.data_ptr(), to_mdt(gating_output.scalar_type()), num_tokens,
             num_experts, renormalize ? 1 : 0,
             bias.has_value() ? bias->data_ptr<float>() : nullptr,
             bias.has_value() ? bias->numel() : 0, cur_stream(gating_output)));
}

// reference grouped_topk (csrc/moe/grouped_topk_kernels.cu:987-1090): allocates and returns
// (topk_values fp32, topk_indices int32), both [num_tokens, topk].
std::tuple<at::Tensor, at::Tensor> op_grouped_topk(const at::Tensor& scores, int64_t n_group,
                                                   int64_t topk_group, int64_t topk,
                                                   bool renormalize,
                                                   double routed_scaling_factor,
                                                   const at::Tensor& bias,
                                                   int64_t scoring_func) {
  TORCH_CHECK(scores.dim() == 2, "scores must be a 2D Tensor");
  TORCH_CHECK(scores.is_cuda() && scores.is_contiguous(), "scores must be a contiguous GPU tensor");
  TORCH_CHECK(bias.is_cuda() && bias.is_contiguous() && bias.dim() == 1,
              "bias must be a contiguous 1D GPU tensor");
  const at::OptionalDeviceGuard guard(scores.device());
  const int64_t num_tokens = scores.size(0);
  auto values = torch::empty({num_tokens, std::max<int64_t>(topk, 0)},
                             scores.options().dtype(at::kFloat));
  auto indices = torch::empty({num_tokens, std::max<int64_t>(topk, 0)},
                              scores.options().dtype(at::kInt));
  rethrow(marlin_grouped_topk(scores.data_ptr(), to_mdt(scores.scalar_type()), num_tokens,
                              scores.size(1), n_group, topk_group, topk, renormalize ? 1 : 0,
                              routed_scaling_factor, bias.data_ptr(), to_mdt(bias.scalar_type()),
                              bias.numel(), scoring_func, values.data_ptr<float>(),
                              indices.data_ptr<int32_t>(), cur_stream(scores)));
  return {values, indices};
}

TORCH_LIBRARY(_moe_C, m) {
  m.def(
      "topk_softmax(Tensor! topk_weights, Tensor! topk_indices, Tensor! "
      "token_expert_indices, Tensor gating_output, bool renormalize, Tensor? "
      "bias) -> ()");
  m.impl("topk_softmax", torch::kCUDA, &op_topk_gating<false>);
  m.def(
      "topk_sigmoid(Tensor! topk_weights, Tensor! topk_indices, Tensor! "
      "token_expert_indices, Tensor gating_output, bool renormalize, Tensor? "
      "bias) -> ()");
  m.impl("topk_sigmoid", torch::kCUDA, &op_topk_gating<true>);
  m.def(
      "grouped_topk(Tensor scores, int n_group, int "
      "topk_group, int topk, bool renormalize, float "
      "routed_scaling_factor, Tensor bias, int scoring_func) -> (Tensor, "
      "Tensor)");
  m.impl("grouped_topk", torch::kCUDA, &op_grouped_topk);
  m.def(
      "moe_align_block_size(Tensor topk_ids, int num_experts,"
      "                     int block_size, Tensor! sorted_token_ids,"
      "                     Tensor! experts_ids,"
      "                     Tensor! num_tokens_post_pad,"
      "                     Tensor? maybe_expert_map) -> ()");
  m.impl("moe_align_block_size", torch::kCUDA, &op_moe_align_block_size);
  m.def(
      "moe_wna16_marlin_gemm(Tensor! a, Tensor? c_or_none,"
      "Tensor! b_q_weight, Tensor? b_bias_or_none,"
      "Tensor! b_scales, Tensor? a_scales, Tensor? global_scale, Tensor? "
      "b_zeros_or_none,"
      "Tensor? g_idx_or_none, Tensor? perm_or_none, Tensor! workspace,"
      "Tensor sorted_token_ids,"
      "Tensor! expert_ids, Tensor! num_tokens_past_padded,"
      "Tensor! topk_weights, int moe_block_size, int top_k, "
      "bool mul_topk_weights, int b_type_id,"
      "int size_m, int size_n, int size_k,"
      "bool is_k_full, bool use_atomic_add,"
      "bool use_fp32_reduce, bool is_zp_float,"
      "int thread_k, int thread_n, int blocks_per_sm) -> Tensor");
  m.impl("moe_wna16_marlin_gemm", torch::kCUDA, &op_moe_wna16_marlin_gemm);
  m.def("moe_sum(Tensor input, Tensor! output) -> ()");
  m.impl("moe_sum", torch::kCUDA, &op_moe_sum);
}

#endif

// `import marlin_v100_amd._C` / `._moe_C` runs the static registrars above
// (reference csrc/core/registration.h:22-27).
#define MMI_CONCAT2(a, b) a##b
#define MMI_CONCAT(a, b) MMI_CONCAT2(a, b)
PyMODINIT_FUNC MMI_CONCAT(PyInit_, MMI_EXT_NAME)() {
  static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, MMI_STR(MMI_EXT_NAME), nullptr, 0,
                                      nullptr};
  return PyModule_Create(&module);
}
