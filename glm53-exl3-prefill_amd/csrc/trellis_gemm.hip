// Entry points of the weight-stationary trellis GEMMs (kernels in trellis_gemm.h): the grouped gate|up / down stages
// of the EXL3 MoE prefill (kernel/exl3_grouped_prefill.cu:148-279 and :324-378), the single-expert fat GEMM
// (kernel/exl3_fat_gemm_v2.cu:236-333), the dense EXL3 linear, reconstruct and the decoder probe.
#include "trellis_gemm.h"

#include <algorithm>

namespace exl3 {
namespace {

// out[t, :] = sum_j partial[t*topk + j, :] in order j = 0 .. topk-1 (deterministic), skipping routes whose id is
// outside [0, n_experts) (their partial rows were never written). A workgroup per token (grid-strided): the token's
// route ids are read once; each thread loads its columns of all topk rows before adding them (a skipped route's row is
// loaded and discarded by a select, so no load waits behind a branch). TOPK > 0 fixes topk at compile time. The
// common case (topk 8, rows of a multiple of 1024 floats) runs combine_routes_cols_kernel, the same sum in the same
// order.
constexpr int COMBINE_THREADS = 256;
constexpr int COMBINE_MAX_TOPK = 32;

// fp32 -> bf16 bits, round to nearest even, every NaN -> 0x7FC0: torch's float -> bfloat16 conversion.
__device__ __forceinline__ uint32_t f2bf(float f)
{
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Four consecutive outputs (float4 index i4) in the output's dtype: fp32, or rounded once to bf16 / fp16 (RNE), which
// is what casting the fp32 sums afterwards gives.
template <int OUT>
__device__ __forceinline__ void store_out4(void* out, int64_t i4, const float4& v)
{
    if constexpr (OUT == EXL3_DTYPE_F32)
        reinterpret_cast<float4*>(out)[i4] = v;
    else if constexpr (OUT == EXL3_DTYPE_BF16)
        reinterpret_cast<uint2*>(out)[i4] = make_uint2(f2bf(v.x) | f2bf(v.y) << 16, f2bf(v.z) | f2bf(v.w) << 16);
    else
        reinterpret_cast<uint2*>(out)[i4] = make_uint2((uint32_t) f2h(v.x) | (uint32_t) f2h(v.y) << 16,
                                                       (uint32_t) f2h(v.z) | (uint32_t) f2h(v.w) << 16);
}

template <int TOPK, int OUT>
__global__ __launch_bounds__(COMBINE_THREADS)
void combine_routes_kernel(const float4* __restrict__ partial, void* __restrict__ out, const void* __restrict__ ids,
                           int ids_dtype, int n_experts, int64_t tokens, int topk_rt, int64_t n4)
{
    const int topk = TOPK > 0 ? TOPK : topk_rt;
    for (int64_t t = blockIdx.x; t < tokens; t += gridDim.x)
    {
        uint32_t live = 0;                              // bit j: route j of the token contributes
        for (int j = 0; j < topk; ++j)
        {
            const int64_t i = t * topk + j;
            int64_t e = 0;
            if (ids)
                e = ids_dtype == EXL3_DTYPE_I64 ? reinterpret_cast<const int64_t*>(ids)[i]
                                                : reinterpret_cast<const int32_t*>(ids)[i];
            if (e >= 0 && e < n_experts) live |= 1u << j;
        }
        const float4* rows = partial + t * topk * n4;
        for (int64_t c = threadIdx.x; c < n4; c += COMBINE_THREADS)
        {
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (TOPK > 0)
            {
                float4 v[TOPK];
                #pragma unroll
                for (int j = 0; j < TOPK; ++j) v[j] = rows[j * n4 + c];
                #pragma unroll
                for (int j = 0; j < TOPK; ++j)
                {
                    const bool on = live >> j & 1;
                    acc.x += on ? v[j].x : 0.f; acc.y += on ? v[j].y : 0.f;
                    acc.z += on ? v[j].z : 0.f; acc.w += on ? v[j].w : 0.f;
                }
            }
            else
                for (int j = 0; j < topk; ++j)
                {
                    if (!(live >> j & 1)) continue;
                    const float4 v = rows[j * n4 + c];
                    acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
                }
            store_out4<OUT>(out, t * n4 + c, acc);
        }
    }
}

// The same sum for topk = TOPK when the row width is a multiple of COMBINE_THREADS float4s: one workgroup per (token,
// COMBINE_THREADS float4 columns), so the token is uniform and its ids arrive through scalar loads issued after the
// lane's TOPK row loads (rows read once: non-temporal). Grid = tokens x n4 / COMBINE_THREADS (fits 31 bits).
template <int TOPK, int OUT>
__global__ __launch_bounds__(COMBINE_THREADS)
void combine_routes_cols_kernel(const float4* __restrict__ partial, void* __restrict__ out,
                                const void* __restrict__ ids, int ids_dtype, int n_experts, int64_t n4)
{
    typedef float fv4 __attribute__((ext_vector_type(4)));
    const uint32_t blocks_per_token = (uint32_t) (n4 / COMBINE_THREADS);
    const uint32_t tb = blockIdx.x / blocks_per_token;
    const int64_t t = tb;
    const int64_t c = (int64_t) (blockIdx.x - tb * blocks_per_token) * COMBINE_THREADS + threadIdx.x;
    const float4* rows = partial + t * TOPK * n4 + c;
    fv4 v[TOPK];
    #pragma unroll
    for (int j = 0; j < TOPK; ++j) v[j] = __builtin_nontemporal_load(reinterpret_cast<const fv4*>(rows + j * n4));
    uint32_t live = (1u << TOPK) - 1;
    if (ids && ids_dtype == EXL3_DTYPE_I64)
    {
        const int64_t* q = reinterpret_cast<const int64_t*>(ids) + t * TOPK;
        live = 0;
        #pragma unroll
        for (int j = 0; j < TOPK; ++j) live |= (q[j] >= 0 && q[j] < n_experts) ? 1u << j : 0u;
    }
    else if (ids)
    {
        const int32_t* q = reinterpret_cast<const int32_t*>(ids) + t * TOPK;
        live = 0;
        #pragma unroll
        for (int j = 0; j < TOPK; ++j) live |= (q[j] >= 0 && q[j] < n_experts) ? 1u << j : 0u;
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    #pragma unroll
    for (int j = 0; j < TOPK; ++j)
    {
        const bool on = live >> j & 1;
        acc.x += on ? v[j][0] : 0.f; acc.y += on ? v[j][1] : 0.f;
        acc.z += on ? v[j][2] : 0.f; acc.w += on ? v[j][3] : 0.f;
    }
    store_out4<OUT>(out, t * n4 + c, acc);
}

// ------------------------------------------------------------------------------------------- reconstruct
// packed [tiles_k, tiles_n, 16 bits] -> out fp16 [16 tiles_k, 16 tiles_n]; 8 lanes per tile as in the GEMM.
template <int BITS>
__global__ __launch_bounds__(256)
void reconstruct_kernel(uint16_t* __restrict__ out, const uint32_t* __restrict__ packed, int tiles_k, int tiles_n)
{
    constexpr int NDW = 8 * BITS;
    const int64_t gid = (int64_t) blockIdx.x * 256 + threadIdx.x;
    const int64_t tile = gid >> 3;
    if (tile >= (int64_t) tiles_k * tiles_n) return;
    const int j = (int) (gid & 7);
    const uint32_t* t = packed + tile * NDW;
    uint32_t r[BITS + 1];
    #pragma unroll
    for (int i = 0; i <= BITS; ++i) r[i] = t[(BITS * j - 1 + i + NDW) % NDW];
    const int tk = (int) (tile / tiles_n), tn = (int) (tile % tiles_n);
    const int64_t ncols = (int64_t) tiles_n * 16;
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int b0 = 8 * i * BITS + BITS - 16;
        const int rel = (b0 >= 0 ? b0 / 32 : -1) + 1;
        const int off = b0 - 32 * (rel - 1);
        const Chunk4 c = decode_chunk<BITS>(r[rel], r[rel + 1 <= BITS ? rel + 1 : BITS], off);
        // chunk 4j+i: k0 = 2i, columns j and j+8
        #pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            const int k = 2 * i + 8 * (q & 1);
            const int n = j + 8 * (q >> 1);
            uint16_t* o = out + (int64_t) (tk * 16 + k) * ncols + tn * 16 + n;
            o[0] = (uint16_t) (c.w[q] & 0xFFFF);
            o[ncols] = (uint16_t) (c.w[q] >> 16);
        }
    }
}

// Each thread decodes two dwords (four states); n2 = number of dwords.
__global__ void decode_states_kernel(const uint32_t* __restrict__ states, uint32_t* __restrict__ out, int64_t n2)
{
    const int64_t i = 2 * ((int64_t) blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= n2) return;
    const uint32_t ra = states[i], rb = (i + 1 < n2) ? states[i + 1] : 0u;
    uint32_t wa, wb;
    decode_state_pairs(ra, rb, wa, wb);
    out[i] = wa;
    if (i + 1 < n2) out[i + 1] = wb;
}

template <int MODE, bool DENSE>
int launch_bits(int bits, const GemmParams& p, hipStream_t s)
{
    switch (bits)
    {
        case 2: return launch_gemm_b2(MODE, DENSE, p, s);
        case 3: return launch_gemm_b3(MODE, DENSE, p, s);
        case 4: return DENSE ? launch_gemm_b4d(MODE, p, s) : launch_gemm_b4g(MODE, p, s);
        default: return fail("unsupported bits %d (2, 3 or 4)", bits);
    }
}

int launch_actin_bits(int bits, const GemmParams& p, hipStream_t s)
{
    switch (bits)
    {
        case 2: return launch_gemm_actin_b2(p, s);
        case 3: return launch_gemm_actin_b3(p, s);
        case 4: return launch_gemm_actin_b4(p, s);
        default: return fail("unsupported bits %d (2, 3 or 4)", bits);
    }
}

// The K-pair schedule (trellis_gemm_kpair_kernel): a dense store on 256-row tiles with both K halves of a tile in one
// 8-wave workgroup.
template <int MODE>
int launch_kpair_bits(int bits, GemmParams p, hipStream_t s)
{
    p.tile_rows = 256;
    p.n_groups = (int) ((p.m + 255) / 256);
    p.k_split = 0;
    switch (bits)
    {
        case 2: return launch_gemm_kpair_b2(MODE, p, s);
        case 3: return launch_gemm_kpair_b3(MODE, p, s);
        case 4: return launch_gemm_kpair_b4(MODE, p, s);
        default: return fail("unsupported bits %d (2, 3 or 4)", bits);
    }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace
}  // namespace exl3

using namespace exl3;

namespace exl3 {
int grouped_gemm_split(const uint16_t* a, int64_t a_rows, int size_k, int a_layout, const uint16_t* packed_gate,
                       const uint16_t* packed_up, int64_t expert_stride_words, int tiles_k, int tiles_n, int bits,
                       const uint16_t* svh_gate, const uint16_t* svh_up, int64_t svh_stride,
                       const int32_t* block_expert, const int32_t* block_row0, int max_blocks, int tile_rows,
                       const int32_t* counts, const int32_t* expert_row0, int n_experts, const int64_t* token_sorted,
                       const uint16_t* route_weight, const int32_t* route_index, void* out, int64_t out_rows, int mode,
                       int k_split, const ActFuse* act, hipStream_t s, float* zero, int64_t zero_floats,
                       bool weights_nt)
{
    EXL3_CHECK(tile_rows == 64 || tile_rows == 128 || tile_rows == 256 || tile_rows == 512,
               "tile_rows must be 64, 128, 256 or 512");
    EXL3_CHECK(a_layout == EXL3_LAYOUT_ROWS || a_layout == EXL3_LAYOUT_T16, "unknown layout");
    EXL3_CHECK(bits >= 2 && bits <= 4, "unsupported bits %d (2, 3 or 4)", bits);
    EXL3_CHECK(size_k == tiles_k * 16 && size_k % 64 == 0 && size_k > 0, "K mismatch");
    const int size_n_each = tiles_n * 16;
    EXL3_CHECK(size_n_each % TILE_N == 0 && size_n_each > 0, "N must be a multiple of 128");
    EXL3_CHECK(n_experts > 0 && n_experts <= MAX_EXPERTS, "too many experts");
    EXL3_CHECK(max_blocks >= 0 && a_rows >= 0, "bad sizes");
    EXL3_CHECK((packed_up == nullptr) == (svh_up == nullptr), "gate/up strides must match");
    EXL3_CHECK(expert_stride_words >= (int64_t) tiles_k * tiles_n * 16 * bits || n_experts == 1,
               "packed [E, tiles_k, tiles_n, 16*bits] with contiguous inner dims (expert stride may be larger: [E,2,...] views)");
    EXL3_CHECK(svh_stride >= size_n_each || n_experts == 1, "svh N mismatch");
    EXL3_CHECK(a && packed_gate && svh_gate && block_expert && block_row0 && counts && expert_row0 && out,
               "null pointer");
    EXL3_CHECK(aligned16(a) && (size_k * 2) % 16 == 0, "a must be 16-byte aligned");
    EXL3_CHECK(((reinterpret_cast<uintptr_t>(packed_gate) | reinterpret_cast<uintptr_t>(packed_up)) & 7) == 0 &&
               expert_stride_words % 4 == 0, "trellis tensors must be 8-byte aligned");
    EXL3_CHECK(((reinterpret_cast<uintptr_t>(svh_gate) | reinterpret_cast<uintptr_t>(svh_up)) & 7) == 0 &&
               svh_stride % 4 == 0, "svh must be 8-byte aligned");
    const int n_tensors = packed_up ? 2 : 1;
    GemmParams p{};
    p.a = a; p.a_rows = a_rows; p.size_k = size_k; p.a_t16 = a_layout == EXL3_LAYOUT_T16;
    p.packed0 = packed_gate; p.packed1 = packed_up; p.expert_stride_words = expert_stride_words;
    p.tiles_n = tiles_n; p.svh0 = svh_gate; p.svh1 = svh_up; p.svh_stride = svh_stride;
    p.block_expert = block_expert; p.block_row0 = block_row0; p.counts = counts; p.expert_row0 = expert_row0;
    p.tile_rows = tile_rows; p.n_groups = max_blocks; p.n_tiles_each = size_n_each / TILE_N;
    p.n_slots = n_tensors * p.n_tiles_each;
    p.token = token_sorted; p.route_weight = route_weight; p.route_index = route_index; p.out = out;
    // K slices of an even number of stages each (the main loop runs stages in pairs)
    const int total_kb = size_k / TILE_K;
    EXL3_CHECK(k_split >= 1 && k_split <= total_kb / 2, "k_split must be in [1, K / 64]");
    EXL3_CHECK(k_split == 1 || mode == EXL3_GEMM_SCATTER_F32 || mode == EXL3_GEMM_ATOMIC_F32,
               "k_split > 1 needs an accumulating mode (1: fp32 atomic scatter, 3: fp32 atomic rows)");
    p.kb_per_split = ((total_kb + k_split - 1) / k_split + 1) / 2 * 2;
    p.k_split = (total_kb + p.kb_per_split - 1) / p.kb_per_split;
    EXL3_CHECK(zero_floats >= 0 && zero_floats % 4 == 0 && (zero_floats == 0 || zero) && aligned16(zero),
               "zero must be 16-byte aligned, a multiple of 4 floats");
    EXL3_CHECK(zero_floats == 0 || max_blocks > 0, "the clear runs on the GEMM's workgroups: max_blocks must be > 0");
    p.zero = reinterpret_cast<float4*>(zero);
    p.zero4 = zero_floats / 4;
    // Thin tables (64-row tiles: each expert's small last tile) in the store modes, the prefill's thin launches, read
    // each tail expert's weights once: loaded non-temporal, they leave the caches to the data that is read again
    // (headline 2.083-2.096 vs 2.097-2.108 ms per layer over six alternating runs, most of it in the combine that
    // follows). The decode path chooses per call (weights_nt).
    p.weights_nt = (weights_nt || (tile_rows == 64 && (mode == EXL3_GEMM_STORE_F16 || mode == EXL3_GEMM_STORE_F16_T16 ||
                                                       mode == EXL3_GEMM_STORE_ROUTE_F32))) ? 1 : 0;
    if (act && act->gu_in)
    {
        EXL3_CHECK(mode == EXL3_GEMM_SCATTER_F32 && n_tensors == 1 && tile_rows == 64 && a_layout == EXL3_LAYOUT_T16,
                   "internal: the activation pass inside the down GEMM runs on mode 1 with 64-row tiles");
        EXL3_CHECK(total_kb % 4 == 0 && p.kb_per_split % 4 == 0 && p.kb_per_split <= ACTIN_MAX_KB,
                   "internal: the down GEMM's K slices must be whole 128-column act blocks of at most %d stages",
                   ACTIN_MAX_KB);
        EXL3_CHECK(act->suh && act->act && aligned16(act->suh) && act->suh_stride % 8 == 0 && aligned16(act->gu_in) &&
                   aligned16(act->act), "suh_down, act and the gate|up sums must be 16-byte aligned");
        p.act_gu = act->gu_in;
        p.act_out = act->act;
        p.act_suh = act->suh;
        p.act_suh_stride = act->suh_stride;
        p.act_limit = act->limit;
    }
    else if (act)
    {
        EXL3_CHECK(mode == EXL3_GEMM_ATOMIC_F32 && n_tensors == 2 && tile_rows == 64,
                   "internal: the fused activation pass runs on mode 3 over gate|up with 64-row tiles");
        EXL3_CHECK(act->arrive && act->act && act->suh, "null pointer");
        EXL3_CHECK(aligned16(act->act) && aligned16(act->suh) && act->suh_stride % 8 == 0,
                   "act and suh_down must be 16-byte aligned");
        p.act_arrive = act->arrive;
        p.act_out = act->act;
        p.act_suh = act->suh;
        p.act_suh_stride = act->suh_stride;
        p.act_limit = act->limit;
    }
    int rc;
    if (mode == EXL3_GEMM_STORE_F16 || mode == EXL3_GEMM_STORE_F16_T16)
    {
        p.out_ld = (int64_t) n_tensors * size_n_each;
        p.out_t16 = mode == EXL3_GEMM_STORE_F16_T16;
        EXL3_CHECK(p.out_t16 ? out_rows >= (a_rows + 15) / 16 * 16 : out_rows >= a_rows,
                   "mode 0: out fp16 [rows, n_tensors*N] (mode 4: T16, rows rounded up to 16)");
        EXL3_CHECK((reinterpret_cast<uintptr_t>(out) & 7) == 0, "out must be 8-byte aligned");
        rc = launch_bits<MODE_STORE_F16, false>(bits, p, s);
    }
    else if (mode == EXL3_GEMM_SCATTER_F32)
    {
        EXL3_CHECK(n_tensors == 1, "mode 1: out fp32 [T, N], single tensor");
        EXL3_CHECK(token_sorted && route_weight, "routing dtypes");
        p.out_ld = size_n_each;
        rc = p.act_gu ? launch_actin_bits(bits, p, s) : launch_bits<MODE_SCATTER_F32, false>(bits, p, s);
    }
    else if (mode == EXL3_GEMM_STORE_ROUTE_F32)
    {
        EXL3_CHECK(n_tensors == 1, "mode 2: out fp32 [routes, N], single tensor");
        EXL3_CHECK(route_index && route_weight, "mode 2 needs route_index and route_weight");
        EXL3_CHECK(aligned16(out), "out must be 16-byte aligned");
        p.out_ld = size_n_each;
        rc = launch_bits<MODE_STORE_ROUTE_F32, false>(bits, p, s);
    }
    else if (mode == EXL3_GEMM_ATOMIC_F32)
    {
        EXL3_CHECK(out_rows >= a_rows, "mode 3: out fp32 [rows, n_tensors*N]");
        EXL3_CHECK(tile_rows <= 256, "mode 3 takes row tiles of 64, 128 or 256 rows");
        EXL3_CHECK((reinterpret_cast<uintptr_t>(out) & 3) == 0, "out must be 4-byte aligned");
        p.out_ld = (int64_t) n_tensors * size_n_each;
        rc = launch_bits<MODE_ATOMIC_F32, false>(bits, p, s);
    }
    else
        return fail("mode must be 0 (fp16 store), 1 (fp32 atomic scatter), 2 (fp32 per-route store), 3 (fp32 atomic "
                    "rows) or 4 (fp16 store, T16 layout)");
    if (rc != EXL3_OK) return rc;
    return hip_status("grouped_gemm");
}
}  // namespace exl3

extern "C" int exl3_grouped_gemm_split(const uint16_t* a, int64_t a_rows, int size_k, int a_layout,
                                       const uint16_t* packed_gate, const uint16_t* packed_up,
                                       int64_t expert_stride_words, int tiles_k, int tiles_n, int bits,
                                       const uint16_t* svh_gate, const uint16_t* svh_up, int64_t svh_stride,
                                       const int32_t* block_expert, const int32_t* block_row0, int max_blocks,
                                       int tile_rows, const int32_t* counts, const int32_t* expert_row0,
                                       int n_experts, const int64_t* token_sorted, const uint16_t* route_weight,
                                       const int32_t* route_index, void* out, int64_t out_rows, int mode,
                                       int k_split, void* stream)
{
    return grouped_gemm_split(a, a_rows, size_k, a_layout, packed_gate, packed_up, expert_stride_words, tiles_k,
                              tiles_n, bits, svh_gate, svh_up, svh_stride, block_expert, block_row0, max_blocks,
                              tile_rows, counts, expert_row0, n_experts, token_sorted, route_weight, route_index, out,
                              out_rows, mode, k_split, nullptr, as_stream(stream));
}

extern "C" int exl3_grouped_gemm_clear(const uint16_t* a, int64_t a_rows, int size_k, int a_layout,
                                       const uint16_t* packed_gate, const uint16_t* packed_up,
                                       int64_t expert_stride_words, int tiles_k, int tiles_n, int bits,
                                       const uint16_t* svh_gate, const uint16_t* svh_up, int64_t svh_stride,
                                       const int32_t* block_expert, const int32_t* block_row0, int max_blocks,
                                       int tile_rows, const int32_t* counts, const int32_t* expert_row0,
                                       int n_experts, const int64_t* token_sorted, const uint16_t* route_weight,
                                       const int32_t* route_index, void* out, int64_t out_rows, int mode,
                                       int k_split, float* zero, int64_t zero_floats, void* stream)
{
    return grouped_gemm_split(a, a_rows, size_k, a_layout, packed_gate, packed_up, expert_stride_words, tiles_k,
                              tiles_n, bits, svh_gate, svh_up, svh_stride, block_expert, block_row0, max_blocks,
                              tile_rows, counts, expert_row0, n_experts, token_sorted, route_weight, route_index, out,
                              out_rows, mode, k_split, nullptr, as_stream(stream), zero, zero_floats);
}

extern "C" int exl3_grouped_gemm_ex(const uint16_t* a, int64_t a_rows, int size_k, int a_layout,
                                    const uint16_t* packed_gate, const uint16_t* packed_up,
                                    int64_t expert_stride_words, int tiles_k, int tiles_n, int bits,
                                    const uint16_t* svh_gate, const uint16_t* svh_up, int64_t svh_stride,
                                    const int32_t* block_expert, const int32_t* block_row0, int max_blocks,
                                    int tile_rows, const int32_t* counts, const int32_t* expert_row0,
                                    int n_experts, const int64_t* token_sorted, const uint16_t* route_weight,
                                    const int32_t* route_index, void* out, int64_t out_rows, int mode,
                                    void* stream)
{
    return exl3_grouped_gemm_split(a, a_rows, size_k, a_layout, packed_gate, packed_up, expert_stride_words, tiles_k,
                                   tiles_n, bits, svh_gate, svh_up, svh_stride, block_expert, block_row0, max_blocks,
                                   tile_rows, counts, expert_row0, n_experts, token_sorted, route_weight, route_index,
                                   out, out_rows, mode, 1, stream);
}

extern "C" int exl3_grouped_gemm(const uint16_t* a, int64_t a_rows, int size_k,
                                 const uint16_t* packed_gate, const uint16_t* packed_up, int64_t expert_stride_words,
                                 int tiles_k, int tiles_n, int bits,
                                 const uint16_t* svh_gate, const uint16_t* svh_up, int64_t svh_stride,
                                 const int32_t* block_expert, const int32_t* block_row0, int max_blocks,
                                 const int32_t* counts, const int32_t* expert_row0, int n_experts,
                                 const int64_t* token_sorted, const uint16_t* route_weight, const int32_t* route_index,
                                 void* out, int64_t out_rows, int mode, void* stream)
{
    return exl3_grouped_gemm_ex(a, a_rows, size_k, EXL3_LAYOUT_ROWS, packed_gate, packed_up, expert_stride_words,
                                tiles_k, tiles_n, bits, svh_gate, svh_up, svh_stride, block_expert, block_row0,
                                max_blocks, 128, counts, expert_row0, n_experts, token_sorted, route_weight,
                                route_index, out, out_rows, mode, stream);
}

namespace {

int fat_common(const uint16_t* a, int64_t m, int size_k, const uint16_t* packed, int tiles_k, int tiles_n,
               int packed_words, const float* out, const uint16_t* svh, int64_t svh_len, int bits, int mcg, int mul1,
               int variant)
{
    EXL3_CHECK(a && packed && out && svh, "tensors must be CUDA");
    EXL3_CHECK(bits >= 2 && bits <= 4 && mcg && !mul1, "only K2/K3/K4 MCG tensors");
    EXL3_CHECK(size_k == tiles_k * 16, "a K dimension does not match packed tensor");
    EXL3_CHECK(svh_len == (int64_t) tiles_n * 16, "svh N dimension does not match packed tensor");
    EXL3_CHECK(svh_len % TILE_N == 0, "N must be divisible by 128");
    EXL3_CHECK(packed_words == 16 * bits, "packed block width must be 16*K int16 words");
    EXL3_CHECK(size_k % 64 == 0, "K must be divisible by 64");
    EXL3_CHECK(variant >= 0 && variant <= 3, "unknown variant");
    EXL3_CHECK(m >= 0 && m < ((int64_t) 1 << 31), "bad row count");
    EXL3_CHECK(aligned16(a) && aligned16(out) && (reinterpret_cast<uintptr_t>(svh) & 7) == 0 &&
               (reinterpret_cast<uintptr_t>(packed) & 7) == 0, "tensors must be contiguous and aligned");
    return EXL3_OK;
}

// Single-expert row tiles. A single expert's matrix is short next to the device: 256-row tiles of a 2048 x 4096 x 4096
// GEMM are 256 workgroups for 256 CUs. 64-row tiles on the thin kernel (four workgroups per CU) decode each weight
// once per 64 rows instead of 256 but spread the work over four times the workgroups, which wins up to 256 rows, and
// up to 2048 rows when K is short (K < 2048: fewer stages to decode per tile). Larger matrices take 512-row tiles on
// the 8-wave kernel. Measured per call (gate|up M x 4096 x 2048, down M x 1024 x 4096, M = 128 .. 2048).
int dense_tile_rows(int64_t m, int size_k)
{
    if (m <= 256 || (m <= 2048 && size_k < 2048)) return 64;
    return 512;
}

// The fat GEMM's `variant` (the reference's four smem/pipeline variants, kernel/exl3_fat_gemm_v2.cu:285-295) selects
// the row-tile schedule here: 1 (the reference's production variant, K64 / 2 stages) the shape-tuned policy above,
// 0 64-row tiles on the thin kernel, 2 256-row tiles on the 4-wave kernel, 3 512-row tiles on the 8-wave kernel. A
// long-K store that would leave CUs idle runs as two K slices, or on the K-pair schedule, under every variant
// (dense_split_pays, dense_kpair_pays), so all four give bit-identical results: each row's sum over K runs in the same
// order whatever the tile height.
int variant_tile_rows(int variant, int64_t m, int size_k)
{
    switch (variant)
    {
        case 0: return 64;
        case 2: return 256;
        case 3: return 512;
        default: return dense_tile_rows(m, size_k);
    }
}

// LDS bytes per workgroup of the kernels a variant can launch (the largest: the scatter form stages output rows).
int64_t variant_lds_bytes(int variant)
{
    const int64_t four = std::max<int64_t>(LDS_MAIN_BYTES, lds_scatter_bytes<4>());   // 64- and 256-row kernels
    const int64_t eight = std::max<int64_t>(LDS_MAIN_BYTES, lds_scatter_bytes<8>());  // 512-row kernel
    switch (variant)
    {
        case 0: case 2: return four;
        case 1: case 3: return eight;          // variant 1 picks 64- or 512-row tiles by shape
        default: return -1;
    }
}

__global__ __launch_bounds__(256)
void zero_f32x4_kernel(float4* __restrict__ p, int64_t n4)
{
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t) gridDim.x * 256) p[i] = z;
}

// A single-expert fp32 GEMM with a long K whose 256-row tiles would give at most one workgroup per CU (two fit) runs
// as two K slices (on 64-row tiles up to 1024 rows, 256-row tiles above) instead: the output is zeroed and each slice
// adds its H128-transformed partial product with fp32 atomics. Two additions onto zero commute exactly, so the result
// is still the same on every run. With K < 2048 the zero fill and the second epilogue cost more than the slices gain
// (measured at K = 1024).
bool dense_split_pays(int64_t m, int n_slots, int size_k)
{
    return (m + 255) / 256 * n_slots <= device_cus() && size_k >= 2048;
}

// Such a GEMM whose 256-row tiles still cover at least 70% of the CUs runs the K-pair schedule instead: both K halves
// of a tile in one 8-wave workgroup, deterministic plain stores (no zero fill, no atomics). Config 2 (4096 x 4096 x
// 1536, 192 tiles): 0.086 vs 0.107 ms for the two slices; at 128 tiles (2048 x 4096 x 2048) the slices stay ahead
// (0.073 vs 0.080 ms): the K-pair workgroups leave half the CUs idle.
bool dense_kpair_pays(int64_t m, int n_slots, int size_k)
{
    return dense_split_pays(m, n_slots, size_k) && (m + 255) / 256 * n_slots * 10 >= 7 * device_cus();
}

template <int MODE>
int launch_dense_split2(GemmParams p, int bits, float* out, int64_t out_floats, hipStream_t s, int variant = 1)
{
    const int total_kb = p.size_k / TILE_K;
    // thin tiles here too, up to 1024 rows (measured); a fixed-schedule variant keeps its tiles (at most 256 rows:
    // the slices add with the 4-wave kernels)
    p.tile_rows = variant == 1 ? (p.m <= 1024 ? 64 : 256) : std::min(p.tile_rows, 256);
    p.n_groups = (int) ((p.m + p.tile_rows - 1) / p.tile_rows);
    p.kb_per_split = ((total_kb + 1) / 2 + 1) / 2 * 2;        // even: both slices have an even number of stages
    p.k_split = (total_kb + p.kb_per_split - 1) / p.kb_per_split;
    const int64_t n4 = out_floats / 4;
    if (n4 > 0)
    {
        const int64_t zgrid = std::min<int64_t>((n4 + 255) / 256, 4096);
        zero_f32x4_kernel<<<(unsigned) zgrid, 256, 0, s>>>(reinterpret_cast<float4*>(out), n4);
    }
    return launch_bits<MODE, true>(bits, p, s);
}

}  // namespace

extern "C" int exl3_fat_gemm(const uint16_t* a, int64_t m, int size_k, const uint16_t* packed, int tiles_k, int tiles_n,
                             int packed_words, float* out, int64_t out_rows, const uint16_t* svh, int64_t svh_len,
                             int bits, int mcg, int mul1, int variant, void* stream)
{
    int rc = fat_common(a, m, size_k, packed, tiles_k, tiles_n, packed_words, out, svh, svh_len, bits, mcg, mul1, variant);
    if (rc) return rc;
    EXL3_CHECK(out_rows == m, "out shape must be [M, N]");
    GemmParams p{};
    p.a = a; p.a_rows = m; p.size_k = size_k; p.packed0 = packed; p.tiles_n = tiles_n;
    p.svh0 = svh; p.tile_rows = variant_tile_rows(variant, m, size_k);
    p.n_groups = (int) ((m + p.tile_rows - 1) / p.tile_rows);
    p.n_tiles_each = (int) (svh_len / TILE_N);
    p.n_slots = p.n_tiles_each; p.m = m; p.out = out; p.out_ld = svh_len;
    if (dense_kpair_pays(m, p.n_slots, size_k))
        rc = launch_kpair_bits<MODE_STORE_F32>(bits, p, as_stream(stream));
    else
        rc = dense_split_pays(m, p.n_slots, size_k)
                 ? launch_dense_split2<MODE_ATOMIC_F32>(p, bits, out, m * svh_len, as_stream(stream), variant)
                 : launch_bits<MODE_STORE_F32, true>(bits, p, as_stream(stream));
    if (rc) return rc;
    return hip_status("fat_gemm_v2");
}

extern "C" int exl3_fat_gemm_scatter(const uint16_t* a, int64_t m, int size_k, const uint16_t* packed, int tiles_k,
                                     int tiles_n, int packed_words, float* out, int64_t out_rows, const uint16_t* svh,
                                     int64_t svh_len, const int64_t* token_idx, const uint16_t* route_weight,
                                     int bits, int mcg, int mul1, int variant, void* stream)
{
    int rc = fat_common(a, m, size_k, packed, tiles_k, tiles_n, packed_words, out, svh, svh_len, bits, mcg, mul1, variant);
    if (rc) return rc;
    EXL3_CHECK(token_idx && route_weight, "routing tensors");
    EXL3_CHECK(out_rows >= 0, "bad out rows");
    GemmParams p{};
    p.a = a; p.a_rows = m; p.size_k = size_k; p.packed0 = packed; p.tiles_n = tiles_n;
    p.svh0 = svh; p.tile_rows = variant_tile_rows(variant, m, size_k);
    p.n_groups = (int) ((m + p.tile_rows - 1) / p.tile_rows);
    p.n_tiles_each = (int) (svh_len / TILE_N);
    p.n_slots = p.n_tiles_each; p.m = m; p.out = out; p.out_ld = svh_len;
    p.token = token_idx; p.route_weight = route_weight;
    rc = launch_bits<MODE_SCATTER_F32, true>(bits, p, as_stream(stream));
    if (rc) return rc;
    return hip_status("fat_gemm_v2_scatter");
}

extern "C" int64_t exl3_linear_workspace_bytes(int64_t m, int k)
{
    if (m < 0 || k <= 0) return -1;
    return (m + 15) / 16 * 16 * (int64_t) k * 2;
}

extern "C" int exl3_linear(const uint16_t* x, int64_t m, int k, const uint16_t* packed, int tiles_k, int tiles_n,
                           int bits, const uint16_t* suh, const uint16_t* svh, uint16_t* work, void* out, int out_dtype,
                           void* stream)
{
    EXL3_CHECK(bits >= 2 && bits <= 4, "unsupported bits %d (2, 3 or 4)", bits);
    EXL3_CHECK(k == tiles_k * 16 && k % 128 == 0 && k > 0, "K must be a multiple of 128 and match the packed tensor");
    EXL3_CHECK(tiles_n > 0 && (tiles_n * 16) % TILE_N == 0, "N must be a multiple of 128");
    EXL3_CHECK(m >= 0 && m < ((int64_t) 1 << 31), "bad row count");
    EXL3_CHECK(out_dtype == EXL3_DTYPE_F32 || out_dtype == EXL3_DTYPE_F16, "out must be fp32 or fp16");
    if (m == 0) return EXL3_OK;
    EXL3_CHECK(x && packed && suh && svh && work && out, "null pointer");
    EXL3_CHECK(aligned16(x) && aligned16(work) && aligned16(suh) && aligned16(out) &&
               (reinterpret_cast<uintptr_t>(svh) & 7) == 0 && (reinterpret_cast<uintptr_t>(packed) & 7) == 0,
               "tensors must be contiguous and aligned");
    hipStream_t s = as_stream(stream);
    int rc = exl3_row_had_ex(x, work, nullptr, nullptr, suh, 0, k, m, k, 0, EXL3_LAYOUT_T16, stream);
    if (rc) return rc;
    const int n = tiles_n * 16;
    GemmParams p{};
    p.a = work; p.a_rows = m; p.a_t16 = 1; p.size_k = k; p.packed0 = packed; p.tiles_n = tiles_n;
    p.svh0 = svh; p.tile_rows = dense_tile_rows(m, k); p.n_groups = (int) ((m + p.tile_rows - 1) / p.tile_rows);
    p.n_tiles_each = n / TILE_N; p.n_slots = p.n_tiles_each; p.m = m; p.out = out; p.out_ld = n;
    if (dense_kpair_pays(m, p.n_slots, k))
        rc = out_dtype == EXL3_DTYPE_F32 ? launch_kpair_bits<MODE_STORE_F32>(bits, p, s)
                                         : launch_kpair_bits<MODE_STORE_F16>(bits, p, s);
    else if (out_dtype == EXL3_DTYPE_F32 && dense_split_pays(m, p.n_slots, k))
        rc = launch_dense_split2<MODE_ATOMIC_F32>(p, bits, reinterpret_cast<float*>(out), m * n, s);
    else
        rc = out_dtype == EXL3_DTYPE_F32 ? launch_bits<MODE_STORE_F32, true>(bits, p, s)
                                         : launch_bits<MODE_STORE_F16, true>(bits, p, s);
    if (rc) return rc;
    return hip_status("linear");
}

namespace exl3 {
namespace {
template <int OUT>
void launch_combine(const float4* p4, void* out, const void* topk_ids, int ids_dtype, int n_experts, int64_t tokens,
                    int topk, int64_t n4, hipStream_t s)
{
    const int64_t blocks = std::min<int64_t>(tokens, 65536), col_blocks = tokens * (n4 / COMBINE_THREADS);
    if (topk == 8 && n4 % COMBINE_THREADS == 0 && col_blocks <= 0x7FFFFFFF)
        combine_routes_cols_kernel<8, OUT><<<(unsigned) col_blocks, COMBINE_THREADS, 0, s>>>(
            p4, out, topk_ids, ids_dtype, n_experts, n4);
    else if (topk == 8)
        combine_routes_kernel<8, OUT><<<(unsigned) blocks, COMBINE_THREADS, 0, s>>>(
            p4, out, topk_ids, ids_dtype, n_experts, tokens, topk, n4);
    else
        combine_routes_kernel<0, OUT><<<(unsigned) blocks, COMBINE_THREADS, 0, s>>>(
            p4, out, topk_ids, ids_dtype, n_experts, tokens, topk, n4);
}
}  // namespace
}  // namespace exl3

extern "C" int exl3_combine_routes_dt(const float* partial, void* out, int out_dtype, const void* topk_ids,
                                      int ids_dtype, int n_experts, int64_t tokens, int topk, int64_t n, void* stream)
{
    EXL3_CHECK(tokens >= 0 && topk > 0 && n > 0 && n % 4 == 0, "combine: bad shape");
    EXL3_CHECK(!topk_ids || ids_dtype == EXL3_DTYPE_I64 || ids_dtype == EXL3_DTYPE_I32, "topk_ids must be int64 or int32");
    EXL3_CHECK(out_dtype == EXL3_DTYPE_F32 || out_dtype == EXL3_DTYPE_BF16 || out_dtype == EXL3_DTYPE_F16,
               "combine: out must be fp32, bf16 or fp16");
    if (tokens == 0) return EXL3_OK;
    EXL3_CHECK(partial && out, "null pointer");
    EXL3_CHECK(aligned16(partial) && (reinterpret_cast<uintptr_t>(out) & (out_dtype == EXL3_DTYPE_F32 ? 15 : 7)) == 0,
               "partial must be 16-byte aligned, out 16-byte (fp32) or 8-byte (bf16 / fp16) aligned");
    EXL3_CHECK(topk <= COMBINE_MAX_TOPK, "combine: topk above %d", COMBINE_MAX_TOPK);
    const auto* p4 = reinterpret_cast<const float4*>(partial);
    const hipStream_t s = as_stream(stream);
    if (out_dtype == EXL3_DTYPE_F32)
        launch_combine<EXL3_DTYPE_F32>(p4, out, topk_ids, ids_dtype, n_experts, tokens, topk, n / 4, s);
    else if (out_dtype == EXL3_DTYPE_BF16)
        launch_combine<EXL3_DTYPE_BF16>(p4, out, topk_ids, ids_dtype, n_experts, tokens, topk, n / 4, s);
    else
        launch_combine<EXL3_DTYPE_F16>(p4, out, topk_ids, ids_dtype, n_experts, tokens, topk, n / 4, s);
    return hip_status("combine_routes");
}

extern "C" int exl3_combine_routes(const float* partial, float* out, const void* topk_ids, int ids_dtype, int n_experts,
                                   int64_t tokens, int topk, int64_t n, void* stream)
{
    return exl3_combine_routes_dt(partial, out, EXL3_DTYPE_F32, topk_ids, ids_dtype, n_experts, tokens, topk, n, stream);
}

extern "C" int64_t exl3_smem_bytes(int64_t variant)
{
    if (variant < 0 || variant > 3) return -1;
    return variant_lds_bytes((int) variant);
}

extern "C" int exl3_reconstruct(uint16_t* out, const uint16_t* packed, int tiles_k, int tiles_n, int bits, int mcg,
                                int mul1, void* stream)
{
    EXL3_CHECK(bits >= 2 && bits <= 4 && mcg && !mul1, "only K2/K3/K4 MCG tensors");
    EXL3_CHECK(tiles_k >= 0 && tiles_n >= 0, "bad shape");
    EXL3_CHECK(out && packed, "null pointer");
    EXL3_CHECK((reinterpret_cast<uintptr_t>(packed) & 3) == 0, "packed must be 4-byte aligned");
    const int64_t lanes = (int64_t) tiles_k * tiles_n * 8;
    if (lanes == 0) return EXL3_OK;
    const unsigned grid = (unsigned) ((lanes + 255) / 256);
    hipStream_t s = as_stream(stream);
    const uint32_t* pk = reinterpret_cast<const uint32_t*>(packed);
    switch (bits)
    {
        case 2: reconstruct_kernel<2><<<grid, 256, 0, s>>>(out, pk, tiles_k, tiles_n); break;
        case 3: reconstruct_kernel<3><<<grid, 256, 0, s>>>(out, pk, tiles_k, tiles_n); break;
        default: reconstruct_kernel<4><<<grid, 256, 0, s>>>(out, pk, tiles_k, tiles_n); break;
    }
    return hip_status("reconstruct");
}

extern "C" int exl3_decode_states(const uint16_t* states, uint16_t* out, int64_t n, void* stream)
{
    EXL3_CHECK(n >= 0 && n % 2 == 0, "n must be even");
    EXL3_CHECK(n == 0 || (states && out), "null pointer");
    EXL3_CHECK(((reinterpret_cast<uintptr_t>(states) | reinterpret_cast<uintptr_t>(out)) & 3) == 0,
               "states/out must be 4-byte aligned");
    const int64_t n2 = n / 2;
    if (n2 == 0) return EXL3_OK;
    decode_states_kernel<<<(unsigned) ((n2 + 511) / 512), 256, 0, as_stream(stream)>>>(
        reinterpret_cast<const uint32_t*>(states), reinterpret_cast<uint32_t*>(out), n2);
    return hip_status("decode_states");
}
