// gemm_u8b128_f16.hip -- GEMM kernel instances for u8b128 weights and f16 activations.
#define MMI_FMT mmi::FMT_U8B128
#define MMI_AT mmi::F16
#define MMI_FN launch_gemm_u8b128_f16
#include "gemm_instances.h"
