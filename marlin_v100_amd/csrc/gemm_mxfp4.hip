// gemm_mxfp4.hip -- marlin_gemm_kernel instances for the mxfp4 weight format.
#define MMI_FMT mmi::FMT_MXFP4
#define MMI_FN launch_gemm_mxfp4
#include "gemm_instances.h"
