// gemm_nvfp4_f16.hip -- GEMM kernel instances for nvfp4 weights and f16 activations.
#define MMI_FMT mmi::FMT_NVFP4
#define MMI_AT mmi::F16
#define MMI_FN launch_gemm_nvfp4_f16
#include "gemm_instances.h"
