// Hadamard helpers shared by the row Hadamard passes (hadamard.hip) and the decode path's fused preparation
// (moe_decode.hip), and the activation pass shared with the decode path's gate|up GEMM (trellis_gemm.h): fp16
// packing, the 128-point transform of the T16 passes and the clamped SwiGLU.
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

// H128 over 8 values per lane x 16 lanes (index = 8 (lane & 15) + i), scaled by 1/sqrt(128): the row-major passes'
// mapping. Its stages run in the same column-bit order as the T16 ones (bits 0-2 in registers, 3-6 across lanes), so
// both round identically.
__device__ __forceinline__ void had128_lane8(float (&x)[8], int lane)
{
    #pragma unroll
    for (int len = 1; len < 8; len <<= 1)
        #pragma unroll
        for (int i = 0; i < 8; ++i)
            if (!(i & len)) { const float a = x[i], b = x[i + len]; x[i] = a + b; x[i + len] = a - b; }
    #pragma unroll
    for (int i = 0; i < 8; ++i)
    {
        float v = x[i];
        v = lane_butterfly<1>(v, lane);
        v = lane_butterfly<2>(v, lane);
        v = lane_butterfly<4>(v, lane);
        v = lane_butterfly<8>(v, lane);
        x[i] = v * HAD_SCALE;
    }
}

__device__ __forceinline__ void had128_t16(float (&x)[32])
{
    fwht_regs<1, 2>(x);
    had128_t16_from2_unscaled(x);
    #pragma unroll
    for (int i = 0; i < 32; ++i) x[i] *= HAD_SCALE;
}

// silu(g) * u in fp32 with the hardware exp and reciprocal: the reference builds with --use_fast_math, so its
// g / (1 + __expf(-g)) is an approximate division too (kernel/exl3_grouped_prefill.cu:135); the result is rounded to
// fp16 next. An IEEE division here cost ~10 VALU per value in a VALU-heavy pass.
__device__ __forceinline__ float silu_mul(float g, float u)
{
#if EXL3_EXACT_SILU_DIV
    return g / (1.0f + __expf(-g)) * u;
#else
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
#endif
}

// 8 consecutive gate|up values: fp16 as stored, or fp32 partial sums rounded to fp16 first (the reference's gu is fp16).
// idx is the element offset of the first (8-aligned) value in gu's layout. COHERENT (fp32 only): device-scope atomic
// loads, which read sums that other workgroups' atomic adds completed during the same launch.
template <bool GU_F32, bool COHERENT = false>
__device__ __forceinline__ void load_gu8(const void* gu, int64_t idx, float (&x)[8])
{
    if constexpr (GU_F32)
    {
        float v[8];
        if constexpr (COHERENT)
        {
            const float* q = reinterpret_cast<const float*>(gu) + idx;
            #pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = __hip_atomic_load(q + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        else
        {
            const float4* q = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(gu) + idx);
            const float4 a = q[0], b = q[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        }
        #pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = h2f(f2h(v[j]));
    }
    else
    {
        // fp16 gate|up rows are read once here: non-temporal (act_had at the headline 0.058-0.059 vs 0.061 ms)
        typedef unsigned u4 __attribute__((ext_vector_type(4)));
        const u4 v = __builtin_nontemporal_load(reinterpret_cast<const u4*>(reinterpret_cast<const uint16_t*>(gu) + idx));
        unpack8(make_uint4(v[0], v[1], v[2], v[3]), x);
    }
}

// Element offset of (r, c) in a T16 [*, W] matrix (c a multiple of 8 here).
__device__ __forceinline__ int64_t t16_index(int64_t r, int64_t c, int64_t W)
{
    return (((r >> 4) * (W >> 3) + (c >> 3)) * 16 + (r & 15)) * 8 + (c & 7);
}

// act_had of row r over the 128-column block blk, in the T16 lane mapping (lane group cq holds columns
// blk * 128 + 8 (4 i + cq) + j as x[8 i + j]): clamped SwiGLU of gate column c and up column I + c, rounded to fp16,
// times suh_down, H128, times 1/sqrt(128) (pack8 rounds the result). gu is [rows, 2I]: fp16, or fp32 sums (GU_F32),
// row-major or T16 (GU_T16); COHERENT reads fp32 sums with device-scope atomic loads (load_gu8). suh_e is the row's
// expert's suh_down.
template <bool GU_F32, bool GU_T16, bool COHERENT = false>
__device__ __forceinline__ void act_had_row(const void* gu, int64_t r, int blk, int cq, int I, const uint16_t* suh_e,
                                            float limit, float (&x)[32])
{
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int c = blk * 128 + 8 * (4 * i + cq);
        float gs[8], us[8], ss[8];
        const int64_t W = 2 * (int64_t) I;
        load_gu8<GU_F32, COHERENT>(gu, GU_T16 ? t16_index(r, c, W) : r * W + c, gs);
        load_gu8<GU_F32, COHERENT>(gu, GU_T16 ? t16_index(r, I + c, W) : r * W + I + c, us);
        unpack8(*reinterpret_cast<const uint4*>(suh_e + c), ss);
        #pragma unroll
        for (int j = 0; j < 8; ++j)
        {
            const float gc = fminf(gs[j], limit);
            const float uc = fminf(fmaxf(us[j], -limit), limit);
            const float a = silu_mul(gc, uc);
            x[8 * i + j] = h2f(f2h(a)) * ss[j];                 // fp16 rounding point of the reference
        }
    }
    had128_t16(x);
}

}  // namespace exl3
