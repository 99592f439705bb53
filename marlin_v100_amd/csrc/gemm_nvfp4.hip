// gemm_nvfp4.hip -- marlin_gemm_kernel instances for the nvfp4 weight format.
#define MMI_FMT mmi::FMT_NVFP4
#define MMI_FN launch_gemm_nvfp4
#include "gemm_instances.h"
