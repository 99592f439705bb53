// gemm_instances.h -- instantiation table of the GEMM kernels for one weight format and one
// activation type.  Included by gemm_<fmt>_<f16|bf16>.hip with MMI_FMT, MMI_AT and MMI_FN
// defined, so the formats and activation types compile in parallel translation units.
#include "host_common.h"

namespace mmi {

// Launches the kernel, or, when l.occupancy is set, only reports how many of its workgroups
// fit on one CU.
template <typename Kernel>
static hipError_t launch_or_query(const GemmLaunch& l, Kernel kernel, unsigned threads,
                                  const GemmParams& p, hipStream_t s) {
  if (l.occupancy != nullptr) {
    if (l.scratch != nullptr) {
      hipFuncAttributes attr{};
      const hipError_t e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(kernel));
      if (e != hipSuccess) return e;
      *l.scratch = (int)attr.localSizeBytes;
    }
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(l.occupancy, kernel, threads, 0);
  }
  hipLaunchKernelGGL(kernel, dim3(l.grid), dim3(threads), 0, s, p);
  return hipGetLastError();
}

template <int FMT, class AT, int GSM>
static hipError_t launch_gsm(const GemmLaunch& l, const GemmParams& p, hipStream_t s) {
  if (l.gated && !l.stream && l.depth == 0) return hipErrorInvalidValue;  // no tiled form
  if (l.depth > 0) {
#define MMI_DECODE(NT_, D_, WPB_, KS_, MOE_, OCC_)                                           \
  if (l.nt == NT_ && l.depth == D_ && l.wpb == WPB_ && l.ksplit == KS_ && l.moe == MOE_ &&       \
      l.occ == OCC_ && !l.gated)                                                             \
    return launch_or_query(l, marlin_decode_kernel<FMT, AT, NT_, D_, WPB_, KS_, GSM, MOE_, OCC_>, \
                           64 * WPB_, p, s);
    if constexpr (FMT != FMT_MXFP4 && FMT != FMT_NVFP4 && GSM != GSM_SMALL) {
      // few-routes MoE stage 1 with the SiLU-gated activation fused (integer-operand formats,
      // the ones the few-routes plan takes)
      if (l.nt == 4 && l.depth == 2 && l.wpb == 1 && l.ksplit && l.moe && l.occ == 2 && l.gated)
        return launch_or_query(
            l, marlin_decode_kernel<FMT, AT, 4, 2, 1, true, GSM, true, 2, true>, 64, p, s);
    }
    MMI_DECODE(4, 3, 4, true, false, 1)
    MMI_DECODE(4, 3, 4, true, false, 3)
    MMI_DECODE(4, 2, 4, true, false, 3)
    MMI_DECODE(4, 2, 4, true, false, 4)
    MMI_DECODE(4, 3, 2, true, false, 1)
    MMI_DECODE(4, 4, 2, true, false, 1)
    MMI_DECODE(4, 3, 1, false, false, 1)
    MMI_DECODE(2, 4, 4, true, false, 1)
    MMI_DECODE(4, 4, 4, true, false, 1)
    MMI_DECODE(4, 3, 4, true, true, 1)
    MMI_DECODE(4, 3, 2, true, true, 1)
    MMI_DECODE(4, 4, 4, true, true, 1)
    MMI_DECODE(4, 4, 2, true, true, 1)
    MMI_DECODE(4, 3, 1, true, true, 1)
    MMI_DECODE(4, 3, 1, true, true, 2)
    MMI_DECODE(4, 2, 1, true, true, 2)
    MMI_DECODE(4, 4, 1, true, true, 1)
    if constexpr (FMT != FMT_MXFP4 && FMT != FMT_NVFP4 && GSM != GSM_SMALL) {
      // 16-column groups for small N at M <= 16: 16 waves split K, every step in flight
      MMI_DECODE(1, 3, 16, true, false, 1)
    }
#undef MMI_DECODE
    return hipErrorInvalidValue;
  }
  if (l.stream) {
// (per-32/64 group metadata for 48/64-row blocks over 256 columns does not fit the register
// budget: those stay on marlin_gemm_kernel)
#define MMI_STREAM(BM_, NT_, MOE_)                                                          \
  if constexpr (!(GSM == GSM_SMALL && BM_ >= 48 && NT_ >= 4)) {                             \
    if (l.bm == BM_ && l.nt == NT_ && l.moe == MOE_ && !l.gated)                            \
      return launch_or_query(l, marlin_stream_kernel<FMT, AT, BM_, NT_, GSM, MOE_>, 256, p, s); \
  }
// MoE stage 1 with the gated activation fused
#define MMI_STREAM_GATED(BM_)                                                                \
  if constexpr (!(GSM == GSM_SMALL && BM_ >= 48)) {                                          \
    if (l.bm == BM_ && l.nt == 4 && l.moe && l.gated)                                        \
      return launch_or_query(l, marlin_stream_kernel<FMT, AT, BM_, 4, GSM, true, true>, 256, p, s); \
  }
    MMI_STREAM_GATED(16)
    MMI_STREAM_GATED(32)
    MMI_STREAM_GATED(48)
    MMI_STREAM_GATED(64)
#undef MMI_STREAM_GATED
    MMI_STREAM(16, 1, false)
    MMI_STREAM(16, 2, false)
    MMI_STREAM(16, 4, false)
    MMI_STREAM(32, 2, false)
    MMI_STREAM(32, 4, false)
    MMI_STREAM(64, 2, false)
    MMI_STREAM(64, 4, false)
    MMI_STREAM(128, 4, false)
    MMI_STREAM(16, 4, true)
    MMI_STREAM(32, 4, true)
    MMI_STREAM(48, 4, true)
    MMI_STREAM(64, 4, true)
    // MoE with size_n % 256 != 0: 128- and 64-column blocks
    MMI_STREAM(16, 2, true)
    MMI_STREAM(32, 2, true)
    MMI_STREAM(48, 2, true)
    MMI_STREAM(64, 2, true)
    MMI_STREAM(16, 1, true)
    MMI_STREAM(32, 1, true)
    MMI_STREAM(48, 1, true)
    MMI_STREAM(64, 1, true)
#undef MMI_STREAM
    return hipErrorInvalidValue;
  }
#define MMI_CASE(BM_, NT_, CH_, MOE_)                                                     \
  if (l.bm == BM_ && l.nt == NT_ && l.ch == CH_ && l.moe == MOE_)                         \
    return launch_or_query(l, marlin_gemm_kernel<FMT, AT, BM_, NT_, CH_, GSM, MOE_>, 256, p, s);
  // dense: small-M weight streaming tiles, then MFMA tiles
  MMI_CASE(16, 1, 1, false)
  MMI_CASE(16, 1, 2, false)
  MMI_CASE(16, 2, 2, false)
  MMI_CASE(32, 2, 2, false)
  MMI_CASE(64, 4, 1, false)
  MMI_CASE(128, 4, 1, false)
  // MoE: one moe block per workgroup
  MMI_CASE(16, 4, 1, true)
  MMI_CASE(32, 4, 1, true)
  MMI_CASE(48, 4, 1, true)
  MMI_CASE(64, 4, 1, true)
#undef MMI_CASE
  return hipErrorInvalidValue;
}

template <int FMT, class AT>
static hipError_t launch_at(const GemmLaunch& l, const GemmParams& p, hipStream_t s) {
  if constexpr (FMT == FMT_MXFP4 || FMT == FMT_NVFP4) {
    if (l.gsm == GSM_SMALL) return launch_gsm<FMT, AT, GSM_SMALL>(l, p, s);
  } else if constexpr (FMT == FMT_FP8) {
    if (l.gsm == GSM_CHANNEL) return launch_gsm<FMT, AT, GSM_CHANNEL>(l, p, s);
    if (l.gsm == GSM_BIG) return launch_gsm<FMT, AT, GSM_BIG>(l, p, s);
  } else {
    if (l.gsm == GSM_CHANNEL) return launch_gsm<FMT, AT, GSM_CHANNEL>(l, p, s);
    if (l.gsm == GSM_BIG) return launch_gsm<FMT, AT, GSM_BIG>(l, p, s);
    if (l.gsm == GSM_SMALL) return launch_gsm<FMT, AT, GSM_SMALL>(l, p, s);
  }
  return hipErrorInvalidValue;
}

hipError_t MMI_FN(const GemmLaunch& l, const GemmParams& p, hipStream_t s) {
  if (l.fmt != MMI_FMT || l.bf16 != (MMI_AT::kId == 1)) return hipErrorInvalidValue;
  return launch_at<MMI_FMT, MMI_AT>(l, p, s);
}

}  // namespace mmi
