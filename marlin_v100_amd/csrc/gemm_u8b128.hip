// gemm_u8b128.hip -- marlin_gemm_kernel instances for the u8b128 weight format.
#define MMI_FMT mmi::FMT_U8B128
#define MMI_FN launch_gemm_u8b128
#include "gemm_instances.h"
