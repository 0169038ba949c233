// Row Hadamard passes of the grouped prefill:
//   row_had (kernel/exl3_grouped_prefill.cu:101-115): dst[r] = fp16(H128(src[tok_r or r] * suh[e_r]) / sqrt(128))
//   act_had (kernel/exl3_grouped_prefill.cu:118-141): act[r] = fp16(H128(fp16(silu(min(g,L)) * clamp(u,+-L)) * suh_down[e_r]) / sqrt(128))
// Both are HBM-bound. Row-major output: a lane owns 8 consecutive columns (one 16-byte load and store) of a
// 128-column block, 16 lanes own a block: 3 butterfly stages run in registers, 4 across lanes (DPP / ds_swizzle),
// fp32 inside; a wave covers 4 (row, block) pairs per step. T16 output (the layout the grouped GEMM reads): see
// the *_t16 kernels below.
#include "hadamard.h"

namespace exl3 {
namespace {

constexpr int HAD_THREADS = 256;

// A 16-byte streaming store: the T16 outputs are written once and read by the next launch in another order, long
// after a cache would have kept them; non-temporal stores keep them from evicting the gathered source rows.
__device__ __forceinline__ void store_nt(uint16_t* p, const uint4 v)
{
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(u4{v.x, v.y, v.z, v.w}, reinterpret_cast<u4*>(p));
}
constexpr int PAIRS_PER_WG = HAD_THREADS / 16;

template <bool GATHER>
__global__ __launch_bounds__(HAD_THREADS)
void row_had_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, const int64_t* __restrict__ token_sorted,
                    const int32_t* __restrict__ expert_of_row, const uint16_t* __restrict__ suh, int64_t suh_stride,
                    int64_t rows, int K)
{
    const int blocks = K / 128;
    const int64_t n_pairs = rows * blocks;
    const int lane = threadIdx.x & 63;
    const int sub = threadIdx.x >> 4;                        // pair slot in the workgroup
    const int col = 8 * (lane & 15);
    for (int64_t pr = (int64_t) blockIdx.x * PAIRS_PER_WG + sub; pr - sub < n_pairs;
         pr += (int64_t) gridDim.x * PAIRS_PER_WG)
    {
        const bool ok = pr < n_pairs;                        // lanes past the end still join the shuffles
        const int64_t prc = ok ? pr : n_pairs - 1;
        const int64_t r = prc / blocks;
        const int blk = (int) (prc - r * blocks);
        const int64_t srow = GATHER ? token_sorted[r] : r;
        const int e = expert_of_row ? expert_of_row[r] : 0;
        const uint4 xv = *reinterpret_cast<const uint4*>(src + srow * K + blk * 128 + col);
        const uint4 sv = *reinterpret_cast<const uint4*>(suh + (int64_t) e * suh_stride + blk * 128 + col);
        float x[8], s[8];
        unpack8(xv, x);
        unpack8(sv, s);
        #pragma unroll
        for (int i = 0; i < 8; ++i) x[i] *= s[i];
        had128_lane8(x, lane);
        if (ok) *reinterpret_cast<uint4*>(dst + r * K + blk * 128 + col) = pack8(x);
    }
}

__global__ __launch_bounds__(HAD_THREADS)
void act_had_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ act, const int32_t* __restrict__ expert_of_row,
                    const uint16_t* __restrict__ suh, int64_t suh_stride, int64_t rows, int I, float limit)
{
    const int blocks = I / 128;
    const int64_t n_pairs = rows * blocks;
    const int lane = threadIdx.x & 63;
    const int sub = threadIdx.x >> 4;
    const int col = 8 * (lane & 15);
    for (int64_t pr = (int64_t) blockIdx.x * PAIRS_PER_WG + sub; pr - sub < n_pairs;
         pr += (int64_t) gridDim.x * PAIRS_PER_WG)
    {
        const bool ok = pr < n_pairs;
        const int64_t prc = ok ? pr : n_pairs - 1;
        const int64_t r = prc / blocks;
        const int blk = (int) (prc - r * blocks);
        const int e = expert_of_row ? expert_of_row[r] : 0;
        const uint16_t* g = gu + r * (2 * (int64_t) I) + blk * 128 + col;
        const uint4 gv = *reinterpret_cast<const uint4*>(g);
        const uint4 uv = *reinterpret_cast<const uint4*>(g + I);
        const uint4 sv = *reinterpret_cast<const uint4*>(suh + (int64_t) e * suh_stride + blk * 128 + col);
        float x[8], u[8], s[8];
        unpack8(gv, x);
        unpack8(uv, u);
        unpack8(sv, s);
        #pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            const float gc = fminf(x[i], limit);
            const float uc = fminf(fmaxf(u[i], -limit), limit);
            const float a = silu_mul(gc, uc);
            x[i] = h2f(f2h(a)) * s[i];                        // fp16 rounding point of the reference
        }
        had128_lane8(x, lane);
        if (ok) *reinterpret_cast<uint4*>(act + r * I + blk * 128 + col) = pack8(x);
    }
}

// ---- T16-layout passes. A wave owns one 16-row group x one 128-column block: lane l holds row l & 15 and the 8-column
// chunks 4 i + (l >> 4) (i = 0..3). For each i the four lanes of a row then read 64 contiguous bytes of it, and the
// wave stores four whole, adjacent 256-byte T16 chunks (16 rows x 8 columns): 1 KB contiguous per store. Column bits
// 0-2 and 5-6 of the block are in the lane's registers (x[8 i + j]: 5 butterfly stages), bits 3 and 4 across lanes
// l ^ 16 and l ^ 32.
template <bool GATHER>
__global__ __launch_bounds__(HAD_THREADS)
void row_had_t16_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                        const int64_t* __restrict__ token_sorted, const int32_t* __restrict__ expert_of_row,
                        const uint16_t* __restrict__ suh, int64_t suh_stride, int64_t rows, int K)
{
    const int blocks = K / 128;
    const int64_t groups = (rows + 15) / 16;
    const int64_t n_items = groups * blocks;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rl = lane & 15, cq = lane >> 4;
    for (int64_t it = (int64_t) blockIdx.x * (HAD_THREADS / 64) + wave; it < n_items;
         it += (int64_t) gridDim.x * (HAD_THREADS / 64))                        // uniform per wave
    {
        const int64_t g = it / blocks;
        const int blk = (int) (it - g * blocks);
        const int64_t r = min(g * 16 + rl, rows - 1);          // rows past the end recompute the last row, unstored
        const int64_t srow = GATHER ? token_sorted[r] : r;
        const int e = expert_of_row ? expert_of_row[r] : 0;
        float x[32];
        #pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const int c = blk * 128 + 8 * (4 * i + cq);
            mul8_stage1(*reinterpret_cast<const uint4*>(src + srow * K + c),
                        *reinterpret_cast<const uint4*>(suh + (int64_t) e * suh_stride + c), x + 8 * i);
        }
        had128_t16_from2_unscaled(x);
        if (g * 16 + rl < rows)
            #pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const int64_t chunk = g * (K / 8) + blk * 16 + 4 * i + cq;
                store_nt(dst + chunk * 128 + rl * 8, pack8_scaled(x + 8 * i));
            }
    }
}

template <bool GU_F32, bool GU_T16 = false>
__global__ __launch_bounds__(HAD_THREADS)
void act_had_t16_kernel(const void* __restrict__ gu, uint16_t* __restrict__ act,
                        const int32_t* __restrict__ expert_of_row, const uint16_t* __restrict__ suh,
                        int64_t suh_stride, int64_t rows, int I, float limit)
{
    const int blocks = I / 128;
    const int64_t groups = (rows + 15) / 16;
    const int64_t n_items = groups * blocks;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rl = lane & 15, cq = lane >> 4;
    for (int64_t it = (int64_t) blockIdx.x * (HAD_THREADS / 64) + wave; it < n_items;
         it += (int64_t) gridDim.x * (HAD_THREADS / 64))
    {
        const int64_t g = it / blocks;
        const int blk = (int) (it - g * blocks);
        const int64_t r = min(g * 16 + rl, rows - 1);
        const int e = expert_of_row ? expert_of_row[r] : 0;
        float x[32];
        act_had_row<GU_F32, GU_T16>(gu, r, blk, cq, I, suh + (int64_t) e * suh_stride, limit, x);
        if (g * 16 + rl < rows)
            #pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                float o[8];
                #pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = x[8 * i + j];
                const int64_t chunk = g * (I / 8) + blk * 16 + 4 * i + cq;
                store_nt(act + chunk * 128 + rl * 8, pack8(o));
            }
    }
}

unsigned t16_grid(int64_t rows, int width)
{
    const int64_t items = (rows + 15) / 16 * (width / 128);
    const int64_t wgs = (items + HAD_THREADS / 64 - 1) / (HAD_THREADS / 64);
    return (unsigned) (wgs < 16384 ? wgs : 16384);
}

unsigned had_grid(int64_t n_pairs)
{
    const int64_t wgs = (n_pairs + PAIRS_PER_WG - 1) / PAIRS_PER_WG;
    return (unsigned) (wgs < 16384 ? wgs : 16384);
}

}  // namespace
}  // namespace exl3

using namespace exl3;

extern "C" int exl3_row_had_ex(const uint16_t* src, uint16_t* dst, const int64_t* token_sorted,
                               const int32_t* expert_of_row, const uint16_t* suh, int64_t suh_stride, int64_t suh_len,
                               int64_t rows, int K, int gather, int dst_layout, void* stream)
{
    EXL3_CHECK(K > 0 && K % 128 == 0 && suh_len == K, "K must be a multiple of 128 and match suh");
    EXL3_CHECK(rows >= 0, "bad row count");
    EXL3_CHECK(dst_layout == EXL3_LAYOUT_ROWS || dst_layout == EXL3_LAYOUT_T16, "unknown layout");
    if (rows == 0) return EXL3_OK;
    EXL3_CHECK(src && dst && suh && (!gather || token_sorted), "null pointer");
    EXL3_CHECK(((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(suh)) & 15) == 0
               && suh_stride % 8 == 0, "src/dst/suh must be 16-byte aligned");
    const unsigned grid = had_grid(rows * (K / 128));
    hipStream_t s = as_stream(stream);
    if (dst_layout == EXL3_LAYOUT_T16)
    {
        const unsigned g16 = t16_grid(rows, K);
        if (gather)
            row_had_t16_kernel<true><<<g16, HAD_THREADS, 0, s>>>(src, dst, token_sorted, expert_of_row, suh, suh_stride,
                                                                 rows, K);
        else
            row_had_t16_kernel<false><<<g16, HAD_THREADS, 0, s>>>(src, dst, nullptr, expert_of_row, suh, suh_stride,
                                                                  rows, K);
    }
    else if (gather)
        row_had_kernel<true><<<grid, HAD_THREADS, 0, s>>>(src, dst, token_sorted, expert_of_row, suh, suh_stride, rows, K);
    else
        row_had_kernel<false><<<grid, HAD_THREADS, 0, s>>>(src, dst, nullptr, expert_of_row, suh, suh_stride, rows, K);
    return hip_status("row_had");
}

extern "C" int exl3_row_had(const uint16_t* src, uint16_t* dst, const int64_t* token_sorted, const int32_t* expert_of_row,
                            const uint16_t* suh, int64_t suh_stride, int64_t suh_len, int64_t rows, int K, int gather,
                            void* stream)
{
    EXL3_CHECK(rows == 0 || expert_of_row, "null pointer");
    return exl3_row_had_ex(src, dst, token_sorted, expert_of_row, suh, suh_stride, suh_len, rows, K, gather,
                           EXL3_LAYOUT_ROWS, stream);
}

extern "C" int exl3_act_had_ex(const uint16_t* gu, int64_t gu_width, uint16_t* act, const int32_t* expert_of_row,
                               const uint16_t* suh_down, int64_t suh_stride, int64_t rows, int I, float limit,
                               int dst_layout, void* stream)
{
    EXL3_CHECK(I > 0 && gu_width == 2 * (int64_t) I && I % 128 == 0, "gate|up width must be 2I, I multiple of 128");
    EXL3_CHECK(rows >= 0, "bad row count");
    EXL3_CHECK(dst_layout == EXL3_LAYOUT_ROWS || dst_layout == EXL3_LAYOUT_T16, "unknown layout");
    if (rows == 0) return EXL3_OK;
    EXL3_CHECK(gu && act && suh_down, "null pointer");
    EXL3_CHECK(((reinterpret_cast<uintptr_t>(gu) | reinterpret_cast<uintptr_t>(act) | reinterpret_cast<uintptr_t>(suh_down)) & 15) == 0
               && suh_stride % 8 == 0, "gu/act/suh must be 16-byte aligned");
    if (dst_layout == EXL3_LAYOUT_T16)
        act_had_t16_kernel<false><<<t16_grid(rows, I), HAD_THREADS, 0, as_stream(stream)>>>(gu, act, expert_of_row,
                                                                                            suh_down, suh_stride, rows,
                                                                                            I, limit);
    else
        act_had_kernel<<<had_grid(rows * (I / 128)), HAD_THREADS, 0, as_stream(stream)>>>(gu, act, expert_of_row,
                                                                                          suh_down, suh_stride, rows, I,
                                                                                          limit);
    return hip_status("act_had");
}

extern "C" int exl3_act_had_f32(const float* gu, int64_t gu_width, uint16_t* act, const int32_t* expert_of_row,
                                const uint16_t* suh_down, int64_t suh_stride, int64_t rows, int I, float limit,
                                void* stream)
{
    EXL3_CHECK(I > 0 && gu_width == 2 * (int64_t) I && I % 128 == 0, "gate|up width must be 2I, I multiple of 128");
    EXL3_CHECK(rows >= 0, "bad row count");
    if (rows == 0) return EXL3_OK;
    EXL3_CHECK(gu && act && suh_down, "null pointer");
    EXL3_CHECK(((reinterpret_cast<uintptr_t>(gu) | reinterpret_cast<uintptr_t>(act) | reinterpret_cast<uintptr_t>(suh_down)) & 15) == 0
               && suh_stride % 8 == 0, "gu/act/suh must be 16-byte aligned");
    act_had_t16_kernel<true><<<t16_grid(rows, I), HAD_THREADS, 0, as_stream(stream)>>>(gu, act, expert_of_row, suh_down,
                                                                                       suh_stride, rows, I, limit);
    return hip_status("act_had_f32");
}

extern "C" int exl3_act_had_t16(const uint16_t* gu, int64_t gu_width, uint16_t* act, const int32_t* expert_of_row,
                                const uint16_t* suh_down, int64_t suh_stride, int64_t rows, int I, float limit,
                                void* stream)
{
    EXL3_CHECK(I > 0 && gu_width == 2 * (int64_t) I && I % 128 == 0, "gate|up width must be 2I, I multiple of 128");
    EXL3_CHECK(rows >= 0, "bad row count");
    if (rows == 0) return EXL3_OK;
    EXL3_CHECK(gu && act && suh_down, "null pointer");
    EXL3_CHECK(((reinterpret_cast<uintptr_t>(gu) | reinterpret_cast<uintptr_t>(act) | reinterpret_cast<uintptr_t>(suh_down)) & 15) == 0
               && suh_stride % 8 == 0, "gu/act/suh must be 16-byte aligned");
    act_had_t16_kernel<false, true><<<t16_grid(rows, I), HAD_THREADS, 0, as_stream(stream)>>>(gu, act, expert_of_row,
                                                                                              suh_down, suh_stride,
                                                                                              rows, I, limit);
    return hip_status("act_had_t16");
}

extern "C" int exl3_act_had(const uint16_t* gu, int64_t gu_width, uint16_t* act, const int32_t* expert_of_row,
                            const uint16_t* suh_down, int64_t suh_stride, int64_t rows, int I, float limit, void* stream)
{
    EXL3_CHECK(rows == 0 || expert_of_row, "null pointer");
    return exl3_act_had_ex(gu, gu_width, act, expert_of_row, suh_down, suh_stride, rows, I, limit, EXL3_LAYOUT_ROWS,
                           stream);
}
