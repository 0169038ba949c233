// Instantiates the trellis GEMM kernels for 3-bit tiles (one translation unit per width: they compile slowly).
#include "trellis_gemm.h"

namespace exl3 {

int launch_gemm_b3(int mode, bool dense, const GemmParams& p, hipStream_t s)
{
    if (dense)
        switch (mode)
        {
            case MODE_STORE_F16: return launch_gemm<3, MODE_STORE_F16, true>(p, s);
            case MODE_SCATTER_F32: return launch_gemm<3, MODE_SCATTER_F32, true>(p, s);
            case MODE_STORE_F32: return launch_gemm<3, MODE_STORE_F32, true>(p, s);
            case MODE_ATOMIC_F32: return launch_gemm<3, MODE_ATOMIC_F32, true>(p, s);
            default: break;
        }
    else
        switch (mode)
        {
            case MODE_STORE_F16: return launch_gemm<3, MODE_STORE_F16, false>(p, s);
            case MODE_SCATTER_F32: return launch_gemm<3, MODE_SCATTER_F32, false>(p, s);
            case MODE_STORE_ROUTE_F32: return launch_gemm<3, MODE_STORE_ROUTE_F32, false>(p, s);
            case MODE_ATOMIC_F32: return launch_gemm<3, MODE_ATOMIC_F32, false>(p, s);
            default: break;
        }
    return fail("internal: no kernel for mode %d", mode);
}

int launch_gemm_kpair_b3(int mode, const GemmParams& p, hipStream_t s)
{
    switch (mode)
    {
        case MODE_STORE_F16: return launch_gemm_kpair<3, MODE_STORE_F16, true>(p, s);
        case MODE_STORE_F32: return launch_gemm_kpair<3, MODE_STORE_F32, true>(p, s);
        default: break;
    }
    return fail("internal: no K-pair kernel for mode %d", mode);
}

int launch_gemm_actin_b3(const GemmParams& p, hipStream_t s) { return launch_gemm_actin<3>(p, s); }
}  // namespace exl3
