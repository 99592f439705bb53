// gemm_u8b128_bf16.hip -- GEMM kernel instances for u8b128 weights and bf16 activations.
#define MMI_FMT mmi::FMT_U8B128
#define MMI_AT mmi::BF16
#define MMI_FN launch_gemm_u8b128_bf16
#include "gemm_instances.h"
