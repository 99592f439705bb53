// gemm_u8z_bf16.hip -- GEMM kernel instances for u8 weights with integer zero points and bf16 activations.
#define MMI_FMT mmi::FMT_U8Z
#define MMI_AT mmi::BF16
#define MMI_FN launch_gemm_u8z_bf16
#include "gemm_instances.h"
