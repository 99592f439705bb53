// host_common.h -- host-side declarations shared by the launch and C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "stream_kernel.h"

namespace mmi {

// Launchers (defined in the .hip files).
hipError_t launch_gptq_repack(const uint32_t* src, const int* perm, uint32_t* out, int64_t size_k,
                              int64_t size_n, int bits, hipStream_t stream);
hipError_t launch_awq_repack(const uint32_t* src, uint32_t* out, int64_t size_k, int64_t size_n,
                             int bits, hipStream_t stream);
hipError_t launch_a8_repack(const uint32_t* src, bool awq, uint32_t* out, int64_t size_k,
                            int64_t size_n, int bits, hipStream_t stream);
hipError_t launch_int4_fp8_preprocess(const uint32_t* q, uint32_t* out, const uint32_t* zeros,
                                      int64_t words, int64_t row_words, int group_size,
                                      hipStream_t stream);
hipError_t launch_dequant(int fmt, const GemmParams& p, bool bf16, void* out, int gs_mode,
                          hipStream_t stream);
hipError_t launch_moe_align(const void* topk, bool is64, int64_t numel, int E, int bs, int* sorted,
                            int64_t sorted_numel, int* expert_ids, int64_t expert_ids_numel,
                            int* post_pad, const int* expert_map, hipStream_t stream);
// act-order: out[m, j] = a[m, perm[j]] (rows of size_k), NaN where perm[j] is out of range
// or, with grouped scales (group_shift >= 0), where the sorted g_idx[j] != j >> group_shift.
hipError_t launch_permute_cols(const void* a, bool bf16, int64_t lda, const int* perm,
                               const int* g_idx, int group_shift, int64_t size_k, int64_t size_m,
                               void* out, hipStream_t stream);
// packed integer zero points (int32 words, 32/bits codes each) -> 16-bit codes
hipError_t launch_expand_zeros(const void* words, int bits, int64_t n_codes, void* out,
                               hipStream_t stream);
hipError_t launch_silu_and_mul(const void* x, bool bf16, int64_t rows, int64_t d, void* out,
                               hipStream_t stream);
// kind: 0 fp16, 1 bf16, 2 fp32
hipError_t launch_moe_sum(const void* in, int kind, int64_t tokens, int topk, int64_t hidden,
                          void* out, hipStream_t stream);
// Router limits: experts per row held in one wavefront's registers, chosen experts per row.
constexpr int kRouterMaxExperts = 64 * 64;
constexpr int kMaxK = 256;
// in_kind 0 fp16 / 1 bf16 / 2 fp32; ids_kind 0 int32 / 1 uint32 / 2 int64.
hipError_t launch_topk_gating(bool sigmoid, int in_kind, const void* gating, const float* bias,
                              float* weights, void* ids, int ids_kind, int* tei, int64_t T, int E,
                              int k, bool renorm, hipStream_t stream);
// grouped_topk: scoring 0 none / 1 sigmoid; bias_kind like in_kind; E <= kGroupedMaxExperts.
constexpr int kGroupedMaxExperts = 1024;
hipError_t launch_grouped_topk(int scoring, int in_kind, int bias_kind, const void* scores,
                               const void* bias, float* values, int* ids, int64_t T, int E,
                               int n_group, int topk_group, int k, bool renorm, float rsf,
                               hipStream_t stream);

// One GEMM launch configuration.
struct GemmLaunch {
  int fmt;
  bool bf16;
  int gsm;   // GSM_CHANNEL / GSM_BIG / GSM_SMALL
  int bm;    // rows per workgroup
  int nt;    // n16 tiles per wave
  int ch;    // 1 KiB weight chunks per tile per K step
  int depth;  // > 0: decode kernel with this load ring depth (bm, ch unused)
  int wpb;    // decode kernel: waves per workgroup
  bool ksplit;  // decode kernel: the workgroup's waves split K (else: adjacent column groups)
  int occ;      // decode kernel: waves per SIMD its registers must allow (1: compiler's choice)
  bool stream;  // multistage kernel for 16..64-row blocks (bm, nt, moe; ch unused)
  bool moe;
  bool gated;   // multistage MoE stage 1 with the SiLU-gated activation fused (nt 4)
  unsigned grid;
  int* occupancy;  // when set: report workgroups per CU instead of launching
  int* scratch;    // with occupancy: also report the kernel's scratch bytes per lane
};
// Defined per format and activation type in gemm_<fmt>_<f16|bf16>.hip; each returns
// hipErrorInvalidValue for a configuration that is not instantiated.
#define MMI_DECLARE_LAUNCH(F)                                                          \
  hipError_t launch_gemm_##F##_f16(const GemmLaunch& l, const GemmParams& p, hipStream_t s); \
  hipError_t launch_gemm_##F##_bf16(const GemmLaunch& l, const GemmParams& p, hipStream_t s);
MMI_DECLARE_LAUNCH(u4b8)
MMI_DECLARE_LAUNCH(u4)
MMI_DECLARE_LAUNCH(u8b128)
MMI_DECLARE_LAUNCH(u8)
MMI_DECLARE_LAUNCH(fp8)
MMI_DECLARE_LAUNCH(mxfp4)
MMI_DECLARE_LAUNCH(nvfp4)
MMI_DECLARE_LAUNCH(u4z)
MMI_DECLARE_LAUNCH(u8z)
#undef MMI_DECLARE_LAUNCH

}  // namespace mmi
