// gemm_fp8.hip -- marlin_gemm_kernel instances for the fp8 weight format.
#define MMI_FMT mmi::FMT_FP8
#define MMI_FN launch_gemm_fp8
#include "gemm_instances.h"
