// Instantiates the trellis GEMM kernels for 4-bit tiles, grouped schedule (one translation unit per width: they compile slowly).
#include "trellis_gemm.h"

namespace exl3 {

int launch_gemm_b4g(int mode, const GemmParams& p, hipStream_t s)
{
    switch (mode)
    {
        case MODE_STORE_F16: return launch_gemm<4, MODE_STORE_F16, false>(p, s);
        case MODE_SCATTER_F32: return launch_gemm<4, MODE_SCATTER_F32, false>(p, s);
        case MODE_STORE_ROUTE_F32: return launch_gemm<4, MODE_STORE_ROUTE_F32, false>(p, s);
        case MODE_ATOMIC_F32: return launch_gemm<4, MODE_ATOMIC_F32, false>(p, s);
        default: break;
    }
    return fail("internal: no kernel for mode %d", mode);
}

int launch_gemm_actin_b4(const GemmParams& p, hipStream_t s) { return launch_gemm_actin<4>(p, s); }
}  // namespace exl3
