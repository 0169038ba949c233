// Hadamard helpers shared by the row Hadamard passes (hadamard.hip) and the decode path's fused preparation
// (moe_decode.hip): fp16 packing and the 128-point transform of the T16 passes.
#pragma once
#include "exl3_common.h"

namespace exl3 {

__device__ __forceinline__ void unpack8(const uint4 v, float (&x)[8])
{
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    #pragma unroll
    for (int i = 0; i < 4; ++i) { x[2 * i] = h2f(w[i] & 0xFFFF); x[2 * i + 1] = h2f(w[i] >> 16); }
}

__device__ __forceinline__ uint4 pack8(const float (&x)[8])
{
    uint32_t w[4];
    #pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (uint32_t) f2h(x[2 * i]) | ((uint32_t) f2h(x[2 * i + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// Butterfly stages len, 2 len, ... < end over the lane's 32 registers.
template <int LEN0, int END>
__device__ __forceinline__ void fwht_regs(float (&x)[32])
{
    #pragma unroll
    for (int len = LEN0; len < END; len <<= 1)
        #pragma unroll
        for (int i = 0; i < 32; ++i)
            if (!(i & len)) { const float a = x[i], b = x[i + len]; x[i] = a + b; x[i + len] = a - b; }
}

// Stages in column-bit order 0..6 (bits 0-2: registers 1, 2, 4; bits 3-4: lanes 16, 32; bits 5-6: registers 8, 16),
// the order of the row-major pass, so both layouts round identically.
__device__ __forceinline__ void had128_t16(float (&x)[32], int lane)
{
    fwht_regs<1, 8>(x);
    #pragma unroll
    for (int i = 0; i < 32; i += 2) pair_butterfly16(x[i], x[i + 1]);
    #pragma unroll
    for (int i = 0; i < 32; i += 2) pair_butterfly32(x[i], x[i + 1]);
    fwht_regs<8, 32>(x);
    #pragma unroll
    for (int i = 0; i < 32; ++i) x[i] *= HAD_SCALE;
}

}  // namespace exl3
