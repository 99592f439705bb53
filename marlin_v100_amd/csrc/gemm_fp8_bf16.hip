// gemm_fp8_bf16.hip -- GEMM kernel instances for fp8 weights and bf16 activations.
#define MMI_FMT mmi::FMT_FP8
#define MMI_AT mmi::BF16
#define MMI_FN launch_gemm_fp8_bf16
#include "gemm_instances.h"
