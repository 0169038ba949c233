// Shared host/device helpers for the EXL3 grouped prefill library (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <atomic>
#include <string>

#include "../../include/exl3_grouped.h"

namespace exl3 {

// ------------------------------------------------------------------------------------------- host errors
// One message per calling thread; entry points return EXL3_OK / EXL3_ERR_ARG / EXL3_ERR_HIP and leave the
// text in here, where exl3_last_error() reads it.
std::string& last_error();

inline int fail(const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    last_error() = buf;
    return EXL3_ERR_ARG;
}

inline int hip_status(const char* what)
{
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
    {
        last_error() = std::string(what) + ": " + hipGetErrorString(e);
        return EXL3_ERR_HIP;
    }
    return EXL3_OK;
}

#define EXL3_CHECK(cond, ...) do { if (!(cond)) return ::exl3::fail(__VA_ARGS__); } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// CUs of the current device (256 if the query fails), cached per device; threads racing on the first query store the
// same value.
inline int device_cus()
{
    static std::atomic<int> cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n == 0)
    {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// The decode path's activation pass fused into its split-K gate|up GEMM (ATOMIC_F32 over both tensors, 64-row tiles;
// trellis_gemm.h, act_after_last_slice): arrive is int32 [max_blocks * N / 128], zero before the call; act is fp16
// T16 [a_rows rounded up to 16, N]; suh is suh_down with row e at suh + e * suh_stride (16-byte aligned).
// K stages of act a down workgroup with the activation pass inside holds in LDS (12 KB; trellis_gemm_actin_kernel).
constexpr int ACTIN_MAX_KB = 12;

struct ActFuse
{
    int* arrive;
    uint16_t* act;
    const uint16_t* suh;
    int64_t suh_stride;
    float limit;
    // not null: the pass runs inside the down GEMM instead (mode 1 on tiles of at most 16 rows), which reads these fp32
    // gate|up sums [rows, 2 I] and still stores act; arrive is then unused
    const float* gu_in = nullptr;
};

// exl3_grouped_gemm_split, plus the fused activation pass when `act` is not null and the clear of zero[0 ..
// zero_floats) as a side job of the same launch (trellis_gemm.hip). weights_nt: 64-row tiles load their trellis words
// non-temporal (the store modes' 64-row tables always do).
int grouped_gemm_split(const uint16_t* a, int64_t a_rows, int size_k, int a_layout, const uint16_t* packed_gate,
                       const uint16_t* packed_up, int64_t expert_stride_words, int tiles_k, int tiles_n, int bits,
                       const uint16_t* svh_gate, const uint16_t* svh_up, int64_t svh_stride,
                       const int32_t* block_expert, const int32_t* block_row0, int max_blocks, int tile_rows,
                       const int32_t* counts, const int32_t* expert_row0, int n_experts, const int64_t* token_sorted,
                       const uint16_t* route_weight, const int32_t* route_index, void* out, int64_t out_rows, int mode,
                       int k_split, const ActFuse* act, hipStream_t s, float* zero = nullptr,
                       int64_t zero_floats = 0, bool weights_nt = false);

// ------------------------------------------------------------------------------------------- device helpers
constexpr float HAD_SCALE = 0.088388347648f;     // 1/sqrt(128)
constexpr int MAX_EXPERTS = 1024;

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

// Lane exchange within 32-lane groups: value of lane (lane ^ M).
template <int M>
__device__ __forceinline__ float xor_lane(float v)
{
    const int i = __float_as_int(v);
    int r;
    if constexpr (M == 1)
        r = __builtin_amdgcn_update_dpp(0, i, 0xB1, 0xF, 0xF, false);       // quad_perm [1,0,3,2]
    else if constexpr (M == 2)
        r = __builtin_amdgcn_update_dpp(0, i, 0x4E, 0xF, 0xF, false);       // quad_perm [2,3,0,1]
    else
        r = __builtin_amdgcn_ds_swizzle(i, 0x1F | (M << 10));              // bitmask mode: xor M
    return __int_as_float(r);
}

// One Walsh-Hadamard butterfly stage across lanes: v' = v + partner on the lower lane, partner - v on the upper.
template <int M>
__device__ __forceinline__ float lane_butterfly(float v, int lane)
{
    const float p = xor_lane<M>(v);
    return (lane & M) ? (p - v) : (v + p);
}

// Butterflies across lanes l and l ^ 16 (rows of 16 lanes) or l ^ 32 (wave halves) for two registers at once, with
// the gfx950 row-swap permutes (no LDS traffic): afterwards the lower lane of each pair holds own + partner and the
// upper lane partner - own, for p and for q. The first swap gathers {p_lower, q_lower} / {p_upper, q_upper}, the
// second puts the sums and differences back.
__device__ __forceinline__ void pair_butterfly16(float& p, float& q)
{
    auto s1 = __builtin_amdgcn_permlane16_swap(__float_as_uint(p), __float_as_uint(q), false, false);
    const float a = __uint_as_float(s1[0]), b = __uint_as_float(s1[1]);
    auto s2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(a + b), __float_as_uint(a - b), false, false);
    p = __uint_as_float(s2[0]);
    q = __uint_as_float(s2[1]);
}
__device__ __forceinline__ void pair_butterfly32(float& p, float& q)
{
    auto s1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(p), __float_as_uint(q), false, false);
    const float a = __uint_as_float(s1[0]), b = __uint_as_float(s1[1]);
    auto s2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a + b), __float_as_uint(a - b), false, false);
    p = __uint_as_float(s2[0]);
    q = __uint_as_float(s2[1]);
}

// XCD-aware workgroup order: workgroups are handed to the 8 XCDs round robin by dispatch id, so dispatch id
// i runs on XCD i % 8. Map it to (group, slot) such that every slot of one group lands on the same XCD
// (they share an activation tile through that XCD's L2) and groups interleave over XCDs.
// Requires the grid to be padded to a multiple of 8 groups.
__device__ __forceinline__ void xcd_group_slot(int id, int slots, int& group, int& slot)
{
    const int xcd = id & 7;
    const int j = id >> 3;
    slot = j % slots;
    group = (j / slots) * 8 + xcd;
}

}  // namespace exl3
