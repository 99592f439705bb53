// gemm_u4b8.hip -- marlin_gemm_kernel instances for the u4b8 weight format.
#define MMI_FMT mmi::FMT_U4B8
#define MMI_FN launch_gemm_u4b8
#include "gemm_instances.h"
