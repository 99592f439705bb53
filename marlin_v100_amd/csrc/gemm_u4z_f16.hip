// gemm_u4z_f16.hip -- GEMM kernel instances for u4 weights with integer zero points and f16 activations.
#define MMI_FMT mmi::FMT_U4Z
#define MMI_AT mmi::F16
#define MMI_FN launch_gemm_u4z_f16
#include "gemm_instances.h"
