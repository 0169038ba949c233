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

// The products x = a * s of two packed fp16 pairs (exact in fp32) with the first butterfly stage fused in:
// sum = x_lo + x_hi, diff = x_lo - x_hi, each rounded once -- what the separate multiply and stage compute, in three
// mixed-precision FMAs instead of two unpacks, two conversions, a multiply and two FMAs. v_fma_mix_f32 reads an fp16
// source from the half op_sel picks (op_sel_hi marks it fp16) and writes a whole fp32 register.
__device__ __forceinline__ void mul_pair_butterfly(uint32_t a, uint32_t s, float& sum, float& diff)
{
    float hi;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "=v"(hi) : "v"(a), "v"(s));
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,1,0]" : "=v"(sum) : "v"(a), "v"(s), "v"(hi));
    asm("v_fma_mix_f32 %0, %1, %2, -%3 op_sel_hi:[1,1,0]" : "=v"(diff) : "v"(a), "v"(s), "v"(hi));
}

// x[8 i + 2 q], x[8 i + 2 q + 1] = the products of chunk i's word q of a and s after the first butterfly stage (the
// input of had128_t16_from2).
__device__ __forceinline__ void mul8_stage1(const uint4 a, const uint4 s, float* x)
{
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, sw[4] = {s.x, s.y, s.z, s.w};
    #pragma unroll
    for (int q = 0; q < 4; ++q) mul_pair_butterfly(aw[q], sw[q], x[2 * q], x[2 * q + 1]);
}

// Stages in column-bit order 0..6 (bits 0-2: registers 1, 2, 4; bits 3-4: lanes 16, 32; bits 5-6: registers 8, 16),
// the order of the row-major pass, so both layouts round identically. had128_t16_from2_unscaled starts after the
// first stage and leaves the 1/sqrt(128) to the fp16 packing (pack8_scaled).
__device__ __forceinline__ void had128_t16_from2_unscaled(float (&x)[32])
{
    fwht_regs<2, 8>(x);
    #pragma unroll
    for (int i = 0; i < 32; i += 2) pair_butterfly16(x[i], x[i + 1]);
    #pragma unroll
    for (int i = 0; i < 32; i += 2) pair_butterfly32(x[i], x[i + 1]);
    fwht_regs<8, 32>(x);
}

// Packed fp16 pairs {fp16(a0 * scale), fp16(a1 * scale)} and {fp16(b0 * scale), fp16(b1 * scale)}, each product rounded
// once to fp16. A high half is written two instructions after the low half it keeps (gfx950 forwards a partial
// register write stale to the next instruction), and an s_nop guards the last partial write for the code after.
__device__ __forceinline__ void scale_pack_2pairs(float a0, float a1, float b0, float b1, float scale, uint32_t& pa,
                                                  uint32_t& pb)
{
    asm("v_fma_mixlo_f16 %0, %2, %6, 0\n\t"
        "v_fma_mixlo_f16 %1, %4, %6, 0\n\t"
        "v_fma_mixhi_f16 %0, %3, %6, 0\n\t"
        "v_fma_mixhi_f16 %1, %5, %6, 0\n\t"
        "s_nop 1"
        : "=&v"(pa), "=&v"(pb) : "v"(a0), "v"(a1), "v"(b0), "v"(b1), "v"(scale));
}

// Eight values x[0..7] times HAD_SCALE as fp16, packed for one 16-byte store.
__device__ __forceinline__ uint4 pack8_scaled(const float* x)
{
    uint4 r;
    scale_pack_2pairs(x[0], x[1], x[2], x[3], HAD_SCALE, r.x, r.y);
    scale_pack_2pairs(x[4], x[5], x[6], x[7], HAD_SCALE, r.z, r.w);
    return r;
}

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
