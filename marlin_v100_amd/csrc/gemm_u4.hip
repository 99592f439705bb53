// gemm_u4.hip -- marlin_gemm_kernel instances for the u4 weight format.
#define MMI_FMT mmi::FMT_U4
#define MMI_FN launch_gemm_u4
#include "gemm_instances.h"
