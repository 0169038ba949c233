// Reading the router's outputs: expert ids (int64 or int32; out-of-range ids drop the route) and route weights
// (fp32, fp16 or bf16, rounded to fp16 as the reference's grouped path stores them). Shared by the route sort
// (route_sort.hip) and the decode path's fused preparation (moe_decode.hip).
#pragma once
#include "exl3_common.h"

namespace exl3 {

template <typename T>
__device__ __forceinline__ int load_id(const void* ids, int64_t i)
{
    const int64_t v = (int64_t) reinterpret_cast<const T*>(ids)[i];
    return (int) v == v ? (int) v : -1;
}

__device__ __forceinline__ int route_id(const void* ids, int ids_dtype, int64_t i, int n_experts)
{
    const int e = (ids_dtype == EXL3_DTYPE_I64) ? load_id<int64_t>(ids, i) : load_id<int32_t>(ids, i);
    return (e >= 0 && e < n_experts) ? e : -1;
}

__device__ __forceinline__ uint16_t route_weight_f16(const void* w, int dtype, int64_t i)
{
    float f;
    if (dtype == EXL3_DTYPE_F32) f = reinterpret_cast<const float*>(w)[i];
    else if (dtype == EXL3_DTYPE_F16) return reinterpret_cast<const uint16_t*>(w)[i];
    else f = __uint_as_float((uint32_t) reinterpret_cast<const uint16_t*>(w)[i] << 16);   // bf16
    return f2h(f);
}

}  // namespace exl3
