// gemm_fp8_f16.hip -- GEMM kernel instances for fp8 weights and f16 activations.
#define MMI_FMT mmi::FMT_FP8
#define MMI_AT mmi::F16
#define MMI_FN launch_gemm_fp8_f16
#include "gemm_instances.h"
