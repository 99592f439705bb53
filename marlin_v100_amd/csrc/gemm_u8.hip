// gemm_u8.hip -- marlin_gemm_kernel instances for the u8 weight format.
#define MMI_FMT mmi::FMT_U8
#define MMI_FN launch_gemm_u8
#include "gemm_instances.h"
