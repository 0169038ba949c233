// Decode-path MoE: the whole routed-expert op for small batches (the `tokens <= cap` side of the reference's switch,
// kernel/exl3_grouped_runtime.py:93-98, where the overlay calls exllamav3's fused exl3_moe,
// kernel/tuned-fused-kernel-patch/exl3patch/exllamav3/exllamav3_ext/quant/exl3_moe.cu:133-345).
//
// Same stages and rounding points as the grouped prefill -- route sort, gather + input Hadamard, gate|up GEMM,
// activation + Hadamard, down GEMM with scatter -- on a fixed launch sequence whose grids depend on the sizes only:
//   * 64-row tiles on the thin GEMM kernel (16 rows per wave, a quarter of the accumulators, four workgroups per CU):
//     most waves of a small batch only decode, and the extra resident waves hide the trellis loads' latency.
//   * The row-tile table is bounded by min(E, R) + R / 64 entries (every expert with rows adds at most one partial
//     tile), so a batch of a few tokens launches a few dozen row tiles instead of one per expert.
//   * A batch of a few tokens has too few (row tile, column tile) pairs to fill the GPU, so both GEMMs split K into
//     slices (chosen from the sizes so that about two workgroups per CU are resident) and add their partial sums
//     with fp32 atomics: gate|up into an fp32 buffer (rounded to fp16 where act_had reads it, the reference's fp16
//     gu), down straight into the output rows.
//   * Everything lives in one caller-provided workspace; buffers that accumulate are cleared by a fill kernel (no
//     memset nodes), and nothing is read back to the host, so a caller may capture the call in a HIP graph.
#include <algorithm>
#include <mutex>

#include "exl3_common.h"
#include "hadamard.h"
#include "routes.h"

// Scratch of exl3_moe_decode_noalloc: the workspace of a decode call, for callers that cannot allocate. Every GPU
// the library runs on holds its own copy until the process ends.
constexpr int64_t DECODE_SCRATCH_BYTES = (int64_t) 32 << 20;
static __device__ __align__(256) unsigned char scratch[DECODE_SCRATCH_BYTES];

namespace exl3 {
namespace {

constexpr int DECODE_TILE_ROWS = 64;                 // the thin GEMM kernel: 16 rows per wave, four workgroups per CU
constexpr int SMALL_ROUTES = 2048;                   // routes exl3_route_prep_small sorts in one workgroup

__global__ __launch_bounds__(256)
void zero2_kernel(float4* __restrict__ a, int64_t na, float4* __restrict__ b, int64_t nb)
{
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < na + nb; i += (int64_t) gridDim.x * 256)
    {
        if (i < na) a[i] = z;
        else b[i - na] = z;
    }
}

int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

struct DecodeLayout
{
    int64_t sort_ws, token_sorted, weight_sorted, expert_of_row, counts, expert_row0, block_expert, block_row0, meta,
        h13, gu, act_arrive, act, total;
    int64_t gu_clear_floats;       // gu and the act arrival counts after it: one region the preparation clears
    int64_t sort_ws_bytes;
    int max_blocks;
};

DecodeLayout decode_layout(int64_t tokens, int topk, int n_experts, int hidden, int inter)
{
    const int64_t R = tokens * topk;
    const int64_t r16 = (R + 15) / 16 * 16;
    DecodeLayout L{};
    L.max_blocks = (int) (std::min<int64_t>(n_experts, R) + R / DECODE_TILE_ROWS);
    L.sort_ws_bytes = (int64_t) exl3_sort_routes_workspace_bytes(tokens, topk, n_experts);
    int64_t o = 0;
    auto take = [&](int64_t bytes) { const int64_t at = o; o += align256(bytes); return at; };
    L.sort_ws = take(L.sort_ws_bytes);
    L.token_sorted = take(R * 8);
    L.weight_sorted = take(R * 2);
    L.expert_of_row = take(R * 4);
    L.counts = take((int64_t) n_experts * 4);
    L.expert_row0 = take((int64_t) n_experts * 4);
    L.block_expert = take((int64_t) L.max_blocks * 4);
    L.block_row0 = take((int64_t) L.max_blocks * 4);
    L.meta = take(8);
    L.h13 = take(r16 * hidden * 2);
    const int64_t gu_bytes = R * 2 * (int64_t) inter * 4;                     // a multiple of 16
    const int64_t arrive_bytes = ((int64_t) L.max_blocks * (inter / 128) * 4 + 15) / 16 * 16;
    L.gu = take(gu_bytes + arrive_bytes);
    L.act_arrive = L.gu + gu_bytes;
    L.gu_clear_floats = (gu_bytes + arrive_bytes) / 4;
    L.act = take(r16 * inter * 2);
    L.total = o;
    return L;
}

#ifndef EXL3_DECODE_WG_PER_CU
#define EXL3_DECODE_WG_PER_CU 4
#endif

// Workgroups a launch should put on the device: four resident thin-kernel workgroups per CU.
int target_workgroups() { return EXL3_DECODE_WG_PER_CU * device_cus(); }

// K slices for a launch of `wgs` workgroups over `stages` 32-wide K stages. A slice holds an even number of stages
// (per = ceil(stages / s) rounded up to even; ceil(stages / per) slices, as exl3_grouped_gemm_split lays them out),
// and the dispatcher deals the workgroups out evenly over the CUs, so the launch lasts about as long as its busiest
// CU's ceil(workgroups / CUs) * per stages of decoding. Take the slice count with the fewest such stages among those
// whose workgroups fit one round of `target` resident ones (a partial second round would double the launch's time),
// the most workgroups among equals (more resident waves hide more latency). At one token on the 288-expert layer:
// 8 slices of 16 stages, 768 workgroups, 48 stages per CU (a plain fill of the round: 10 slices of 14 and 2, 960
// workgroups, 56 stages on the busiest CUs).
int k_split_for(int64_t wgs, int stages, int target)
{
    if (wgs <= 0) return 1;
    const int64_t cus = device_cus();
    int best = 1;
    int64_t best_cost = -1;
    for (int s = 1; s <= std::max(1, stages / 2); ++s)
    {
        const int per = ((stages + s - 1) / s + 1) / 2 * 2;
        const int64_t n = wgs * ((stages + per - 1) / per);
        if (s > 1 && n > target) break;
        const int64_t cost = (n + cus - 1) / cus * per;
        if (best_cost < 0 || cost <= best_cost)
        {
            best_cost = cost;
            best = s;
        }
    }
    return best;
}

// K slices for the down launch with the activation pass inside (trellis_gemm_actin_kernel): equal slices of whole
// 128-column act blocks, at most ACTIN_MAX_KB stages each, with the cost rule of k_split_for but the fewest
// workgroups among equals (at one token 2 slices of 12 stages ran 30.3-30.5 us per call in a step's graph, 3 slices
// of 8 stages 30.6-30.8: each slice adds its partial rows into the same output row, and the act work per slice is
// spread over the waves either way); 0 when no such split fits one round of `target` workgroups (the gate|up launch
// then keeps the pass).
// Whether the gate|up launch and the down launch with the activation pass inside load the trellis words
// non-temporal (each call reads each active expert's weights once). Measured per call in a step's graph (two
// alternating runs): one token 25.6-26.0 vs 26.7-26.8 us, 16 tokens 172-177 vs 183-184, 32 tokens 262-266 vs 276-277,
// 64 tokens 400 vs 403-405; at 2 and 4 tokens the non-temporal loads measured 2.8-3 us slower, at 8 and 128 even. The
// down launch after a separate activation pass (more than 16 routes) measured slower with them at every size.
bool decode_weights_nt(int64_t routes) { return routes <= 8 || routes >= 64; }

int k_split_actin(int64_t wgs, int stages, int target)
{
    if (wgs <= 0 || stages % 4 != 0) return 0;
    const int64_t cus = device_cus();
    int best = 0;
    int64_t best_cost = -1;
    for (int per = 4; per <= ACTIN_MAX_KB && per <= stages; per += 4)
    {
        if (stages % per != 0) continue;
        const int s = stages / per;
        const int64_t n = wgs * s;
        if (n > target) continue;
        const int64_t cost = (n + cus - 1) / cus * per;
        if (best_cost < 0 || cost <= best_cost)            // per rises: the last of equals has the fewest workgroups
        {
            best_cost = cost;
            best = s;
        }
    }
    return best;
}

// This device's address of `scratch`, looked up once per device with that device current. In host code the array's
// name is not a device address: every host use of the scratch (kernel arguments, fills, copies) takes this pointer.
int decode_scratch(void** ptr)
{
    constexpr int MAX_DEVICES = 64;
    static std::mutex mu;
    static void* addr[MAX_DEVICES] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
        return hip_status("moe_decode_noalloc: no current device");
    std::lock_guard<std::mutex> guard(mu);
    if (!addr[dev])
    {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
        {
            last_error() = std::string("moe_decode_noalloc: hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
            return EXL3_ERR_HIP;
        }
        addr[dev] = p;
    }
    *ptr = addr[dev];
    return EXL3_OK;
}

// ------------------------------------------------------------------------------------------- fused preparation
// Up to TINY_ROUTES routes are ranked by direct comparison: the stable sort by expert puts route i at row
// #{valid j : e_j < e_i} + #{j < i : e_j == e_i}, which every workgroup can compute from the ids alone. So the
// gathered input Hadamard need not wait for the sort: one launch does it all, with the rows and tables identical to
// exl3_route_prep_small's and h13 identical to row_had's.
constexpr int TINY_ROUTES = 128;
constexpr int PREP_THREADS = 256;

// Workgroup 0: the sorted routes (token, fp16 weight, expert; rows past the valid ones zeroed), counts and
// expert_row0 of every expert, the 64-row tile table (entries past the last tile -1) and meta = {tiles, rows}.
// Workgroups 1 .. n_had: h13 (T16 layout, width `hidden`) = fp16(H128(x[token] * suh[e]) / sqrt(128)) at each
// route's row; a wave takes 16 routes x one 128-column block per step. The remaining workgroups clear two fp32
// buffers (float4 counts na, nb).
__global__ __launch_bounds__(PREP_THREADS)
void decode_prep_tiny_kernel(const uint16_t* __restrict__ x, int hidden, const void* __restrict__ ids, int ids_dtype,
                             const void* __restrict__ weights, int w_dtype, int R, int topk, int n_experts,
                             const uint16_t* __restrict__ suh, int64_t suh_stride, int max_tiles, int n_had,
                             int64_t* __restrict__ token_sorted, uint16_t* __restrict__ weight_sorted,
                             int32_t* __restrict__ expert_of_row, int32_t* __restrict__ counts,
                             int32_t* __restrict__ expert_row0, int32_t* __restrict__ tile_expert,
                             int32_t* __restrict__ tile_row0, int32_t* __restrict__ meta, uint16_t* __restrict__ h13,
                             float4* __restrict__ zero_a, int64_t na, float4* __restrict__ zero_b, int64_t nb)
{
    const int t = threadIdx.x;
    if ((int) blockIdx.x > n_had)
    {
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
        const int64_t wgs = gridDim.x - 1 - n_had;
        for (int64_t i = (int64_t) (blockIdx.x - 1 - n_had) * PREP_THREADS + t; i < na + nb; i += wgs * PREP_THREADS)
        {
            if (i < na) zero_a[i] = z;
            else zero_b[i - na] = z;
        }
        return;
    }
    // route j's expert (-1: dropped or past R), in int4 steps; its row; its expert's tile count if j is the expert's
    // first route (else 0)
    __shared__ __align__(16) int s_e[TINY_ROUTES];
    __shared__ __align__(16) int s_nt[TINY_ROUTES];
    __shared__ int s_rank[TINY_ROUTES];
    if (t < TINY_ROUTES) s_e[t] = t < R ? route_id(ids, ids_dtype, t, n_experts) : -1;
    __syncthreads();
    const int R4 = (R + 3) / 4;
    const int4* e4 = reinterpret_cast<const int4*>(s_e);
    int n_rows = 0;                                     // valid routes (every thread)
    if (t < TINY_ROUTES)
    {
        const int e = s_e[t];
        int before = 0, same_before = 0, same = 0;
        for (int q = 0; q < R4; ++q)
        {
            const int4 f4 = e4[q];
            const int f[4] = {f4.x, f4.y, f4.z, f4.w};
            #pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                n_rows += f[k] >= 0;
                before += f[k] >= 0 && f[k] < e;
                same_before += f[k] == e && 4 * q + k < t;
                same += f[k] == e;
            }
        }
        s_rank[t] = e >= 0 ? before + same_before : -1;
        s_nt[t] = e >= 0 && same_before == 0 ? (same + DECODE_TILE_ROWS - 1) / DECODE_TILE_ROWS : 0;
    }
    else
        for (int q = 0; q < R4; ++q)
        {
            const int4 f4 = e4[q];
            n_rows += (f4.x >= 0) + (f4.y >= 0) + (f4.z >= 0) + (f4.w >= 0);
        }
    __syncthreads();

    if (blockIdx.x == 0)
    {
        if (t < R)
        {
            const int r = s_rank[t];
            if (r >= 0)
            {
                token_sorted[r] = t / topk;
                weight_sorted[r] = route_weight_f16(weights, w_dtype, t);
                expert_of_row[r] = s_e[t];
            }
            if (t >= n_rows)                            // rows past the valid ones (dropped routes)
            {
                token_sorted[t] = 0;
                weight_sorted[t] = 0;
                expert_of_row[t] = 0;
            }
        }
        for (int e = t; e < n_experts; e += PREP_THREADS)
        {
            int c = 0, below = 0;
            for (int q = 0; q < R4; ++q)
            {
                const int4 f4 = e4[q];
                const int f[4] = {f4.x, f4.y, f4.z, f4.w};
                #pragma unroll
                for (int k = 0; k < 4; ++k)
                {
                    c += f[k] == e;
                    below += f[k] >= 0 && f[k] < e;
                }
            }
            counts[e] = c;
            expert_row0[e] = below;
        }
        // tiles of 64 rows, experts in order: expert e's first tile follows those of every smaller active expert
        const int e = t < TINY_ROUTES ? s_e[t] : -1;
        const int4* nt4 = reinterpret_cast<const int4*>(s_nt);
        int tile0 = 0, n_tiles = 0;
        for (int q = 0; q < R4; ++q)
        {
            const int4 f4 = e4[q], n4 = nt4[q];
            n_tiles += n4.x + n4.y + n4.z + n4.w;
            tile0 += (f4.x < e ? n4.x : 0) + (f4.y < e ? n4.y : 0) + (f4.z < e ? n4.z : 0) + (f4.w < e ? n4.w : 0);
        }
        if (t < R)
            for (int q = 0; q < s_nt[t]; ++q)
                if (tile0 + q < max_tiles)
                {
                    tile_expert[tile0 + q] = e;
                    tile_row0[tile0 + q] = s_rank[t] + q * DECODE_TILE_ROWS;
                }
        for (int b = n_tiles + t; b < max_tiles; b += PREP_THREADS) tile_expert[b] = -1;
        if (t == 0) { meta[0] = n_tiles; meta[1] = n_rows; }
        return;
    }

    // the input Hadamard of every route, at its sorted row
    const int lane = t & 63, wave = t >> 6, rl = lane & 15, cq = lane >> 4;
    const int blocks = hidden / 128;
    const int n_items = (R + 15) / 16 * blocks;
    for (int it = (blockIdx.x - 1) * (PREP_THREADS / 64) + wave; it < n_items; it += n_had * (PREP_THREADS / 64))
    {
        const int g = it / blocks, blk = it - g * blocks;
        const int i = g * 16 + rl;
        const int r = i < R ? s_rank[i] : -1;
        const int ic = r >= 0 ? i : 0;                  // lanes without a route still join the lane butterflies
        const int e = max(s_e[ic], 0);
        const int64_t tok = ic / topk;
        float v[32];
        #pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            const int c = blk * 128 + 8 * (4 * k + cq);
            mul8_stage1(*reinterpret_cast<const uint4*>(x + tok * hidden + c),
                        *reinterpret_cast<const uint4*>(suh + (int64_t) e * suh_stride + c), v + 8 * k);
        }
        had128_t16_from2_unscaled(v);
        if (r >= 0)
            #pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                const int64_t chunk = (int64_t) (r >> 4) * (hidden / 8) + blk * 16 + 4 * k + cq;
                *reinterpret_cast<uint4*>(h13 + chunk * 128 + (r & 15) * 8) = pack8_scaled(v + 8 * k);
            }
    }
}

}  // namespace
}  // namespace exl3

using namespace exl3;

extern "C" int64_t exl3_moe_decode_workspace_bytes(int64_t tokens, int topk, int n_experts, int hidden, int inter)
{
    if (tokens < 0 || topk <= 0 || n_experts <= 0 || n_experts > MAX_EXPERTS || hidden <= 0 || inter <= 0) return -1;
    return decode_layout(tokens, topk, n_experts, hidden, inter).total;
}

extern "C" int exl3_moe_decode(const uint16_t* x, int64_t tokens, int hidden, const void* topk_ids, int ids_dtype,
                               const void* topk_weights, int weights_dtype, int topk, int n_experts, int inter,
                               int bits, const uint16_t* packed_gate, const uint16_t* packed_up,
                               int64_t w13_expert_stride_words, const uint16_t* suh_gate, int64_t suh13_stride,
                               const uint16_t* svh_gate, const uint16_t* svh_up, int64_t svh13_stride,
                               const uint16_t* packed_down, int64_t w2_expert_stride_words, const uint16_t* suh_down,
                               int64_t suh2_stride, const uint16_t* svh_down, int64_t svh2_stride, float limit,
                               float* out, void* workspace, int64_t workspace_bytes, void* stream)
{
    EXL3_CHECK(tokens >= 0 && topk > 0, "bad routing shape");
    EXL3_CHECK(hidden > 0 && hidden % 128 == 0 && inter > 0 && inter % 128 == 0,
               "hidden and intermediate sizes must be multiples of 128");
    EXL3_CHECK(n_experts > 0 && n_experts <= MAX_EXPERTS, "too many experts");
    EXL3_CHECK(bits >= 2 && bits <= 4, "unsupported bits %d (2, 3 or 4)", bits);
    EXL3_CHECK(tokens * topk < ((int64_t) 1 << 31), "too many routes");
    if (tokens == 0) return EXL3_OK;
    EXL3_CHECK(x && topk_ids && topk_weights && packed_gate && packed_up && suh_gate && svh_gate && svh_up &&
               packed_down && suh_down && svh_down && out && workspace, "null pointer");
    EXL3_CHECK((reinterpret_cast<uintptr_t>(out) & 15) == 0 && (reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
               "out must be 16-byte and the workspace 256-byte aligned");
    const DecodeLayout L = decode_layout(tokens, topk, n_experts, hidden, inter);
    EXL3_CHECK(workspace_bytes >= L.total, "decode workspace too small (%lld < %lld bytes)",
               (long long) workspace_bytes, (long long) L.total);
    hipStream_t s = as_stream(stream);
    char* ws = reinterpret_cast<char*>(workspace);
    auto at = [&](int64_t off) { return reinterpret_cast<void*>(ws + off); };
    const int64_t R = tokens * topk;
    auto* token_sorted = reinterpret_cast<int64_t*>(at(L.token_sorted));
    auto* weight_sorted = reinterpret_cast<uint16_t*>(at(L.weight_sorted));
    auto* expert_of_row = reinterpret_cast<int32_t*>(at(L.expert_of_row));
    auto* counts = reinterpret_cast<int32_t*>(at(L.counts));
    auto* expert_row0 = reinterpret_cast<int32_t*>(at(L.expert_row0));
    auto* block_expert = reinterpret_cast<int32_t*>(at(L.block_expert));
    auto* block_row0 = reinterpret_cast<int32_t*>(at(L.block_row0));
    auto* meta = reinterpret_cast<int32_t*>(at(L.meta));
    auto* h13 = reinterpret_cast<uint16_t*>(at(L.h13));
    auto* gu = reinterpret_cast<float*>(at(L.gu));
    auto* act_arrive = reinterpret_cast<int*>(at(L.act_arrive));
    auto* act = reinterpret_cast<uint16_t*>(at(L.act));

    // accumulation targets, cleared by the preparation: out [tokens, hidden] and gu [R, 2 inter] followed by the
    // activation pass's arrival counts, both whole float4s
    const int64_t n_out = tokens * hidden, n_gu = L.gu_clear_floats;
    int rc;
    if (R <= TINY_ROUTES)
    {
        // sort, tile table, both clears and the input Hadamard in one launch
        EXL3_CHECK(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(suh_gate)) & 15) == 0 &&
                   suh13_stride % 8 == 0, "x and suh must be 16-byte aligned");
        const int n_had = ((int) ((R + 15) / 16) * (hidden / 128) + PREP_THREADS / 64 - 1) / (PREP_THREADS / 64);
        const int64_t n4 = n_out / 4 + n_gu / 4;
        const int64_t zwgs = std::min<int64_t>((n4 + PREP_THREADS - 1) / PREP_THREADS, 1024);
        decode_prep_tiny_kernel<<<(unsigned) (1 + n_had + zwgs), PREP_THREADS, 0, s>>>(
            x, hidden, topk_ids, ids_dtype, topk_weights, weights_dtype, (int) R, topk, n_experts, suh_gate,
            suh13_stride, L.max_blocks, n_had, token_sorted, weight_sorted, expert_of_row, counts, expert_row0,
            block_expert, block_row0, meta, h13, reinterpret_cast<float4*>(out), n_out / 4,
            reinterpret_cast<float4*>(gu), n_gu / 4);
        rc = hip_status("moe_decode prep");
        if (rc) return rc;
    }
    else if (R <= SMALL_ROUTES)
    {
        // sort, tile table and both clears in one launch
        rc = exl3_route_prep_small(topk_ids, ids_dtype, topk_weights, weights_dtype, tokens, topk, n_experts,
                                   DECODE_TILE_ROWS, L.max_blocks, token_sorted, weight_sorted, expert_of_row, counts,
                                   expert_row0, block_expert, block_row0, meta, out, n_out, gu, n_gu, stream);
        if (rc) return rc;
    }
    else
    {
        const int64_t zgrid = std::min<int64_t>((n_out / 4 + n_gu / 4 + 255) / 256, 2048);
        zero2_kernel<<<(unsigned) zgrid, 256, 0, s>>>(reinterpret_cast<float4*>(out), n_out / 4,
                                                      reinterpret_cast<float4*>(gu), n_gu / 4);
        rc = hip_status("moe_decode zero");
        if (rc) return rc;
        rc = exl3_sort_routes(topk_ids, ids_dtype, topk_weights, weights_dtype, tokens, topk, n_experts, token_sorted,
                              weight_sorted, expert_of_row, nullptr, counts, expert_row0, at(L.sort_ws),
                              (size_t) L.sort_ws_bytes, stream);
        if (rc) return rc;
        rc = exl3_build_tiles(counts, n_experts, DECODE_TILE_ROWS, L.max_blocks, block_expert, block_row0, meta,
                              stream);
        if (rc) return rc;
    }
    if (R > TINY_ROUTES)
    {
        rc = exl3_row_had_ex(x, h13, token_sorted, expert_of_row, suh_gate, suh13_stride, hidden, R, hidden, 1,
                             EXL3_LAYOUT_T16, stream);
        if (rc) return rc;
    }
    const int target = target_workgroups();
    const int gu_split = k_split_for((int64_t) L.max_blocks * 2 * (inter / 128), hidden / 32, target);
    // With at most 16 routes every tile holds at most 16 rows (whatever the ids), and where the down launch can take K
    // slices of whole act blocks the activation pass runs inside it (each down workgroup computes its own slice of act
    // from the gate|up sums, behind its first trellis loads); otherwise the last gate|up workgroup of each (row tile,
    // 128-column block) computes that block of act from the finished sums. Either way the pass needs no launch of its
    // own.
    const int actin_split = R <= 16 ? k_split_actin((int64_t) L.max_blocks * (hidden / 128), inter / 32, target) : 0;
    const bool nt = decode_weights_nt(R);
    const ActFuse fuse{act_arrive, act, suh_down, suh2_stride, limit};
    rc = grouped_gemm_split(h13, R, hidden, EXL3_LAYOUT_T16, packed_gate, packed_up, w13_expert_stride_words,
                            hidden / 16, inter / 16, bits, svh_gate, svh_up, svh13_stride, block_expert, block_row0,
                            L.max_blocks, DECODE_TILE_ROWS, counts, expert_row0, n_experts, token_sorted, weight_sorted,
                            nullptr, gu, R, EXL3_GEMM_ATOMIC_F32, gu_split, actin_split ? nullptr : &fuse, s, nullptr, 0,
                            nt);
    if (rc) return rc;
    if (actin_split)
    {
        const ActFuse in{nullptr, act, suh_down, suh2_stride, limit, gu};
        return grouped_gemm_split(act, R, inter, EXL3_LAYOUT_T16, packed_down, nullptr, w2_expert_stride_words,
                                  inter / 16, hidden / 16, bits, svh_down, nullptr, svh2_stride, block_expert,
                                  block_row0, L.max_blocks, DECODE_TILE_ROWS, counts, expert_row0, n_experts,
                                  token_sorted, weight_sorted, nullptr, out, tokens, EXL3_GEMM_SCATTER_F32, actin_split,
                                  &in, s, nullptr, 0, nt);
    }
    const int down_split = k_split_for((int64_t) L.max_blocks * (hidden / 128), inter / 32, target);
    return exl3_grouped_gemm_split(act, R, inter, EXL3_LAYOUT_T16, packed_down, nullptr, w2_expert_stride_words,
                                   inter / 16, hidden / 16, bits, svh_down, nullptr, svh2_stride, block_expert,
                                   block_row0, L.max_blocks, DECODE_TILE_ROWS, counts, expert_row0, n_experts,
                                   token_sorted, weight_sorted, nullptr, out, tokens, EXL3_GEMM_SCATTER_F32,
                                   down_split, stream);
}

extern "C" int exl3_moe_decode_noalloc(const uint16_t* x, int64_t tokens, int hidden, const void* topk_ids,
                                       int ids_dtype, const void* topk_weights, int weights_dtype, int topk,
                                       int n_experts, int inter, int bits, const uint16_t* packed_gate,
                                       const uint16_t* packed_up, int64_t w13_expert_stride_words,
                                       const uint16_t* suh_gate, int64_t suh13_stride, const uint16_t* svh_gate,
                                       const uint16_t* svh_up, int64_t svh13_stride, const uint16_t* packed_down,
                                       int64_t w2_expert_stride_words, const uint16_t* suh_down, int64_t suh2_stride,
                                       const uint16_t* svh_down, int64_t svh2_stride, float limit, float* out,
                                       void* stream)
{
    EXL3_CHECK(tokens >= 0 && topk > 0, "bad routing shape");
    const int64_t need = exl3_moe_decode_workspace_bytes(tokens, topk, n_experts, hidden, inter);
    EXL3_CHECK(need >= 0, "bad decode sizes");
    EXL3_CHECK(need <= DECODE_SCRATCH_BYTES,
               "moe_decode_noalloc: this call needs %lld bytes of workspace, more than its fixed scratch of %lld bytes "
               "(use exl3_moe_decode with a caller workspace)", (long long) need, (long long) DECODE_SCRATCH_BYTES);
    if (tokens == 0) return EXL3_OK;
    void* ws = nullptr;
    const int rc = decode_scratch(&ws);
    if (rc) return rc;
    return exl3_moe_decode(x, tokens, hidden, topk_ids, ids_dtype, topk_weights, weights_dtype, topk, n_experts, inter,
                           bits, packed_gate, packed_up, w13_expert_stride_words, suh_gate, suh13_stride, svh_gate,
                           svh_up, svh13_stride, packed_down, w2_expert_stride_words, suh_down, suh2_stride, svh_down,
                           svh2_stride, limit, out, ws, DECODE_SCRATCH_BYTES, stream);
}
