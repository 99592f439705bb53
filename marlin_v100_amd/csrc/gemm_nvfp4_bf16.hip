// gemm_nvfp4_bf16.hip -- GEMM kernel instances for nvfp4 weights and bf16 activations.
#define MMI_FMT mmi::FMT_NVFP4
#define MMI_AT mmi::BF16
#define MMI_FN launch_gemm_nvfp4_bf16
#include "gemm_instances.h"
