// Instantiates the trellis GEMM kernels for 4-bit tiles, single-matrix schedule (one translation unit per width: they compile slowly).
#include "trellis_gemm.h"

namespace exl3 {

int launch_gemm_b4d(int mode, const GemmParams& p, hipStream_t s)
{
    switch (mode)
    {
        case MODE_STORE_F16: return launch_gemm<4, MODE_STORE_F16, true>(p, s);
        case MODE_SCATTER_F32: return launch_gemm<4, MODE_SCATTER_F32, true>(p, s);
        case MODE_STORE_F32: return launch_gemm<4, MODE_STORE_F32, true>(p, s);
        case MODE_ATOMIC_F32: return launch_gemm<4, MODE_ATOMIC_F32, true>(p, s);
        default: break;
    }
    return fail("internal: no kernel for mode %d", mode);
}

int launch_gemm_kpair_b4(int mode, const GemmParams& p, hipStream_t s)
{
    switch (mode)
    {
        case MODE_STORE_F16: return launch_gemm_kpair<4, MODE_STORE_F16, true>(p, s);
        case MODE_STORE_F32: return launch_gemm_kpair<4, MODE_STORE_F32, true>(p, s);
        default: break;
    }
    return fail("internal: no K-pair kernel for mode %d", mode);
}
}  // namespace exl3
