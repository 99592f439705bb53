// gemm_u4_f16.hip -- GEMM kernel instances for u4 weights and f16 activations.
#define MMI_FMT mmi::FMT_U4
#define MMI_AT mmi::F16
#define MMI_FN launch_gemm_u4_f16
#include "gemm_instances.h"
