// gemm_u4_bf16.hip -- GEMM kernel instances for u4 weights and bf16 activations.
#define MMI_FMT mmi::FMT_U4
#define MMI_AT mmi::BF16
#define MMI_FN launch_gemm_u4_bf16
#include "gemm_instances.h"
