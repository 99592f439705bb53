// gemm_mxfp4_f16.hip -- GEMM kernel instances for mxfp4 weights and f16 activations.
#define MMI_FMT mmi::FMT_MXFP4
#define MMI_AT mmi::F16
#define MMI_FN launch_gemm_mxfp4_f16
#include "gemm_instances.h"
