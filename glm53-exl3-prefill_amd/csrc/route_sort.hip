// Route sort and block table.
//
// sort_routes replaces the torch glue of grouped_prefill (kernel/exl3_grouped_runtime.py:59-68: stable
// argsort, repeat_interleave, gathers, scatter_add_, cumsum) with a stable counting sort in three launches:
//   1. hist:    one workgroup per CHUNK of routes counts experts in LDS -> hist[chunk][e]
//   2. offsets: one workgroup turns hist into counts[e], expert_row0[e] and per-chunk write cursors
//   3. scatter: each chunk re-walks its routes in index order; ranks among equal ids inside a wave come from
//      a ballot match over the id bits, across the chunk's waves from per-wave counts in LDS, so the write
//      order is exactly the stable order.
// The prefill path runs passes 2 and 3 and its tile tables as one launch (sort_scatter_tiles_kernel): every scatter
// workgroup derives its own cursors from the histograms.
// build_blocks restates kernel/exl3_grouped_prefill.cu:63-96 with a parallel scan instead of the serial one.
// route_topk is the router glue in front of the sort (GLM-5.3-Flash's noaux_tc top-k): one wave per token.
#include "routes.h"

#include <math.h>

#include <algorithm>

namespace exl3 {
namespace {

constexpr int SORT_THREADS = 256;
constexpr int SORT_WAVES = SORT_THREADS / 64;
constexpr int ROUTES_PER_THREAD = 8;
constexpr int CHUNK = SORT_THREADS * ROUTES_PER_THREAD;    // routes per workgroup in passes 1 and 3
#ifndef EXL3_PREP_CLEAR_WGS
#define EXL3_PREP_CLEAR_WGS 8192
#endif
constexpr int PREP_CLEAR_WGS = EXL3_PREP_CLEAR_WGS;         // workgroups clearing the output beside the scatter

__global__ __launch_bounds__(SORT_THREADS)
void sort_hist_kernel(const void* __restrict__ ids, int ids_dtype, int64_t R, int n_experts,
                      int32_t* __restrict__ hist, int32_t* __restrict__ bad_per_chunk)
{
    __shared__ int32_t s_hist[MAX_EXPERTS];
    const int t = threadIdx.x;
    for (int e = t; e < n_experts; e += SORT_THREADS) s_hist[e] = 0;
    __syncthreads();
    const int64_t base = (int64_t) blockIdx.x * CHUNK;
    int bad = 0;
    int ev[ROUTES_PER_THREAD];
    #pragma unroll
    for (int k = 0; k < ROUTES_PER_THREAD; ++k)
    {
        const int64_t i = base + k * SORT_THREADS + t;
        ev[k] = (i < R) ? route_id(ids, ids_dtype, i, n_experts) : -2;
    }
    #pragma unroll
    for (int k = 0; k < ROUTES_PER_THREAD; ++k)
    {
        if (ev[k] >= 0) atomicAdd(&s_hist[ev[k]], 1);
        else if (ev[k] == -1) ++bad;
    }
    __syncthreads();
    for (int e = t; e < n_experts; e += SORT_THREADS) hist[(int64_t) blockIdx.x * n_experts + e] = s_hist[e];
    __shared__ int32_t s_bad;
    if (t == 0) s_bad = 0;
    __syncthreads();
    if (bad) atomicAdd(&s_bad, bad);
    __syncthreads();
    if (t == 0) bad_per_chunk[blockIdx.x] = s_bad;
}

// Single workgroup of 1024 threads; thread e owns expert e.
__global__ __launch_bounds__(1024)
void sort_offsets_kernel(int32_t* __restrict__ hist, const int32_t* __restrict__ bad_per_chunk, int n_chunks,
                         int n_experts, int32_t* __restrict__ counts, int32_t* __restrict__ expert_row0,
                         int32_t* __restrict__ dropped)
{
    __shared__ int32_t s_scan[1024];
    const int e = threadIdx.x;
    if (e == 0)
    {
        int d = 0;
        for (int b = 0; b < n_chunks; ++b) d += bad_per_chunk[b];
        *dropped = d;
    }
    // 8 independent loads per step: one loop-carried load per chunk would serialise n_chunks memory latencies
    int c = 0;
    if (e < n_experts)
    {
        int part[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int b = 0;
        for (; b + 8 <= n_chunks; b += 8)
            #pragma unroll
            for (int i = 0; i < 8; ++i) part[i] += hist[(int64_t) (b + i) * n_experts + e];
        for (; b < n_chunks; ++b) part[0] += hist[(int64_t) b * n_experts + e];
        #pragma unroll
        for (int i = 0; i < 8; ++i) c += part[i];
    }
    s_scan[e] = (e < n_experts) ? c : 0;
    __syncthreads();
    // Hillis-Steele inclusive scan over 1024 entries
    for (int d = 1; d < 1024; d <<= 1)
    {
        const int v = (e >= d) ? s_scan[e - d] : 0;
        __syncthreads();
        s_scan[e] += v;
        __syncthreads();
    }
    if (e < n_experts)
    {
        const int row0 = s_scan[e] - c;
        counts[e] = c;
        expert_row0[e] = row0;
        int cur = row0;
        int b = 0;
        for (; b + 8 <= n_chunks; b += 8)
        {
            int h[8];
            #pragma unroll
            for (int i = 0; i < 8; ++i) h[i] = hist[(int64_t) (b + i) * n_experts + e];
            #pragma unroll
            for (int i = 0; i < 8; ++i)
            {
                hist[(int64_t) (b + i) * n_experts + e] = cur;   // becomes chunk b + i's first row for expert e
                cur += h[i];
            }
        }
        for (; b < n_chunks; ++b)
        {
            const int h = hist[(int64_t) b * n_experts + e];
            hist[(int64_t) b * n_experts + e] = cur;
            cur += h;
        }
    }
}

// Bitmask of the lanes of this wave whose key equals ours (only among lanes with valid keys).
__device__ __forceinline__ uint64_t match_lanes(int key, bool valid)
{
    uint64_t peers = __ballot(valid);
    #pragma unroll
    for (int bit = 0; bit < 10; ++bit)            // keys < 1024
    {
        const bool b = (key >> bit) & 1;
        const uint64_t m = __ballot(b);
        peers &= b ? m : ~m;
    }
    return peers;
}

// Writes the routes of chunk [base, base + CHUNK) to their sorted rows, in index order: s_cursor[e] holds the chunk's
// first row for expert e (advanced here), s_wave_cnt is zero on entry and on exit. Called by all SORT_THREADS
// threads of the workgroup.
__device__ __forceinline__ void scatter_chunk(const void* __restrict__ ids, int ids_dtype,
                                              const void* __restrict__ weights, int w_dtype, int64_t R, int topk,
                                              int n_experts, int64_t base, int32_t* s_cursor,
                                              int32_t (*s_wave_cnt)[MAX_EXPERTS], int64_t* __restrict__ token_sorted,
                                              uint16_t* __restrict__ weight_sorted,
                                              int32_t* __restrict__ expert_of_row, int32_t* __restrict__ route_index)
{
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    // all of this thread's ids and weights up front: one round of memory latency instead of one per step
    int ev[ROUTES_PER_THREAD];
    uint16_t wv[ROUTES_PER_THREAD];
    #pragma unroll
    for (int k = 0; k < ROUTES_PER_THREAD; ++k)
    {
        const int64_t i = base + k * SORT_THREADS + t;
        ev[k] = (i < R) ? route_id(ids, ids_dtype, i, n_experts) : -1;
        wv[k] = (i < R) ? route_weight_f16(weights, w_dtype, i) : 0;
    }
    #pragma unroll
    for (int k = 0; k < ROUTES_PER_THREAD; ++k)
    {
        const int64_t i = base + k * SORT_THREADS + t;
        const int e = ev[k];
        const bool valid = e >= 0;
        const uint64_t peers = match_lanes(valid ? e : 0, valid);
        const int rank = __popcll(peers & below);
        const bool leader = valid && rank == 0;
        if (leader) s_wave_cnt[wave][e] = __popcll(peers);
        __syncthreads();
        if (valid)
        {
            int row = s_cursor[e] + rank;
            for (int w = 0; w < wave; ++w) row += s_wave_cnt[w][e];
            token_sorted[row] = i / topk;
            weight_sorted[row] = wv[k];
            expert_of_row[row] = e;
            if (route_index) route_index[row] = (int32_t) i;
        }
        __syncthreads();
        if (leader)
        {
            atomicAdd(&s_cursor[e], __popcll(peers));
            s_wave_cnt[wave][e] = 0;
        }
        __syncthreads();
    }
}

// Rows past sum(counts) (only present when routes were dropped): token 0, weight 0, expert 0, route 0. Disjoint from
// the rows the scatter writes, so every workgroup of the scatter launch takes a grid-strided share.
__device__ __forceinline__ void fill_tail(const int32_t* __restrict__ counts, const int32_t* __restrict__ expert_row0,
                                          int n_experts, int64_t R, int64_t* __restrict__ token_sorted,
                                          uint16_t* __restrict__ weight_sorted, int32_t* __restrict__ expert_of_row,
                                          int32_t* __restrict__ route_index)
{
    const int64_t n_rows = (int64_t) expert_row0[n_experts - 1] + counts[n_experts - 1];
    for (int64_t r = n_rows + (int64_t) blockIdx.x * blockDim.x + threadIdx.x; r < R; r += (int64_t) gridDim.x * blockDim.x)
    {
        token_sorted[r] = 0;
        weight_sorted[r] = 0;
        expert_of_row[r] = 0;
        if (route_index) route_index[r] = 0;
    }
}

__global__ __launch_bounds__(SORT_THREADS)
void sort_scatter_kernel(const void* __restrict__ ids, int ids_dtype, const void* __restrict__ weights, int w_dtype,
                         int64_t R, int topk, int n_experts, const int32_t* __restrict__ cursor0,
                         const int32_t* __restrict__ counts, const int32_t* __restrict__ expert_row0,
                         int64_t* __restrict__ token_sorted, uint16_t* __restrict__ weight_sorted,
                         int32_t* __restrict__ expert_of_row, int32_t* __restrict__ route_index)
{
    __shared__ int32_t s_cursor[MAX_EXPERTS];
    __shared__ int32_t s_wave_cnt[SORT_WAVES][MAX_EXPERTS];
    const int t = threadIdx.x;
    for (int e = t; e < n_experts; e += SORT_THREADS)
    {
        s_cursor[e] = cursor0[(int64_t) blockIdx.x * n_experts + e];
        for (int w = 0; w < SORT_WAVES; ++w) s_wave_cnt[w][e] = 0;
    }
    __syncthreads();
    scatter_chunk(ids, ids_dtype, weights, w_dtype, R, topk, n_experts, (int64_t) blockIdx.x * CHUNK, s_cursor,
                  s_wave_cnt, token_sorted, weight_sorted, expert_of_row, route_index);
    fill_tail(counts, expert_row0, n_experts, R, token_sorted, weight_sorted, expert_of_row, route_index);
}

// The prefill path's pass 2 and tile tables in one launch, after sort_hist_kernel (no offsets launch). Workgroup c <
// n_chunks scatters chunk c: it sums the per-chunk histograms itself -- every expert's total over all chunks and over
// the chunks before c -- and scans the totals into expert_row0, which gives the cursors sort_offsets_kernel would
// have handed it, then writes the chunk's rows (scatter_chunk) and its share of the tail rows. Workgroup n_chunks
// writes counts, expert_row0, the dropped count and the two tables of build_tiles_split_kernel (meta = {full tiles,
// rows, thin tiles}); the rest clear the caller's fp32 buffer. No workgroup waits for another. Thread t owns experts
// 4t .. 4t + 3.
__global__ __launch_bounds__(SORT_THREADS)
void sort_scatter_tiles_kernel(const void* __restrict__ ids, int ids_dtype, const void* __restrict__ weights,
                               int w_dtype, int64_t R, int topk, int n_experts, int n_chunks,
                               const int32_t* __restrict__ hist, const int32_t* __restrict__ bad_per_chunk,
                               int32_t* __restrict__ dropped, int64_t* __restrict__ token_sorted,
                               uint16_t* __restrict__ weight_sorted, int32_t* __restrict__ expert_of_row,
                               int32_t* __restrict__ route_index, int32_t* __restrict__ counts,
                               int32_t* __restrict__ expert_row0, int tile_rows, int thin_rows, int max_full,
                               int max_thin, int32_t* __restrict__ full_expert, int32_t* __restrict__ full_row0,
                               int32_t* __restrict__ thin_expert, int32_t* __restrict__ thin_row0,
                               int32_t* __restrict__ meta, float4* __restrict__ zero, int64_t zero4)
{
    static_assert(4 * SORT_THREADS >= MAX_EXPERTS, "four experts per thread");
    const int t = threadIdx.x;
    const int wg = blockIdx.x;
    if (wg > n_chunks)                                    // clear the caller's fp32 buffer
    {
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
        const int64_t step = (int64_t) (gridDim.x - n_chunks - 1) * SORT_THREADS;
        for (int64_t i = (int64_t) (wg - n_chunks - 1) * SORT_THREADS + t; i < zero4; i += step) zero[i] = z;
        return;
    }
    // totals over all chunks and over the chunks before this one (the tables workgroup: wg == n_chunks, all of them);
    // 16 chunks per step, the thread's four experts in one 16-byte load per chunk when rows are 16-byte multiples
    int tot[4] = {0, 0, 0, 0}, pre[4] = {0, 0, 0, 0};
    const bool vec = (n_experts & 3) == 0;
    for (int c0 = 0; c0 < n_chunks; c0 += 16)
    {
        int4 h[16];
        #pragma unroll
        for (int i = 0; i < 16; ++i)
        {
            const int c = c0 + i, e = 4 * t;
            const int32_t* row = hist + (int64_t) c * n_experts;
            if (c >= n_chunks || e >= n_experts) h[i] = make_int4(0, 0, 0, 0);
            else if (vec) h[i] = *reinterpret_cast<const int4*>(row + e);
            else h[i] = make_int4(row[e], e + 1 < n_experts ? row[e + 1] : 0, e + 2 < n_experts ? row[e + 2] : 0,
                                  e + 3 < n_experts ? row[e + 3] : 0);
        }
        #pragma unroll
        for (int i = 0; i < 16; ++i)
        {
            const int m = (c0 + i < wg) ? -1 : 0;          // chunks before this one count towards its cursors
            tot[0] += h[i].x; tot[1] += h[i].y; tot[2] += h[i].z; tot[3] += h[i].w;
            pre[0] += h[i].x & m; pre[1] += h[i].y & m; pre[2] += h[i].z & m; pre[3] += h[i].w & m;
        }
    }
    int nfull[4], nthin[4];
    #pragma unroll
    for (int j = 0; j < 4; ++j)
    {
        const int rem = tot[j] % tile_rows;
        nthin[j] = (rem > 0 && rem <= thin_rows) ? 1 : 0;
        nfull[j] = tot[j] / tile_rows + ((rem > thin_rows) ? 1 : 0);
    }
    const int my_rows = tot[0] + tot[1] + tot[2] + tot[3];
    const int my_full = nfull[0] + nfull[1] + nfull[2] + nfull[3];
    const int my_thin = nthin[0] + nthin[1] + nthin[2] + nthin[3];
    __shared__ int32_t s_rows[SORT_THREADS], s_full[SORT_THREADS], s_thin[SORT_THREADS];
    s_rows[t] = my_rows;
    s_full[t] = my_full;
    s_thin[t] = my_thin;
    __syncthreads();
    for (int d = 1; d < SORT_THREADS; d <<= 1)            // inclusive scans over the threads
    {
        const int vr = (t >= d) ? s_rows[t - d] : 0;
        const int vf = (t >= d) ? s_full[t - d] : 0;
        const int vt = (t >= d) ? s_thin[t - d] : 0;
        __syncthreads();
        s_rows[t] += vr;
        s_full[t] += vf;
        s_thin[t] += vt;
        __syncthreads();
    }
    int row0 = s_rows[t] - my_rows;
    const int64_t n_rows = s_rows[SORT_THREADS - 1];
    if (wg == n_chunks)
    {
        int f0 = s_full[t] - my_full, t0 = s_thin[t] - my_thin;
        #pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const int e = 4 * t + j;
            if (e < n_experts)
            {
                counts[e] = tot[j];
                expert_row0[e] = row0;
                for (int i = 0; i < nfull[j]; ++i)
                    if (f0 + i < max_full) { full_expert[f0 + i] = e; full_row0[f0 + i] = row0 + i * tile_rows; }
                if (nthin[j] && t0 < max_thin)
                {
                    thin_expert[t0] = e;
                    thin_row0[t0] = row0 + (tot[j] / tile_rows) * tile_rows;
                }
            }
            row0 += tot[j];
            f0 += nfull[j];
            t0 += nthin[j];
        }
        const int n_full = s_full[SORT_THREADS - 1], n_thin = s_thin[SORT_THREADS - 1];
        if (t == 0)
        {
            meta[0] = n_full;
            meta[1] = (int) n_rows;
            meta[2] = n_thin;
            int d = 0;
            for (int c = 0; c < n_chunks; ++c) d += bad_per_chunk[c];
            *dropped = d;
        }
        for (int b = n_full + t; b < max_full; b += SORT_THREADS) full_expert[b] = -1;
        for (int b = n_thin + t; b < max_thin; b += SORT_THREADS) thin_expert[b] = -1;
        return;
    }
    __shared__ int32_t s_cursor[MAX_EXPERTS];
    __shared__ int32_t s_wave_cnt[SORT_WAVES][MAX_EXPERTS];
    #pragma unroll
    for (int j = 0; j < 4; ++j)
    {
        const int e = 4 * t + j;
        if (e < n_experts)
        {
            s_cursor[e] = row0 + pre[j];
            for (int w = 0; w < SORT_WAVES; ++w) s_wave_cnt[w][e] = 0;
        }
        row0 += tot[j];
    }
    __syncthreads();
    scatter_chunk(ids, ids_dtype, weights, w_dtype, R, topk, n_experts, (int64_t) wg * CHUNK, s_cursor, s_wave_cnt,
                  token_sorted, weight_sorted, expert_of_row, route_index);
    // rows past the routed ones (dropped routes): token 0, weight 0, expert 0, route 0, as fill_tail writes them
    for (int64_t r = n_rows + (int64_t) wg * SORT_THREADS + t; r < R; r += (int64_t) n_chunks * SORT_THREADS)
    {
        token_sorted[r] = 0;
        weight_sorted[r] = 0;
        expert_of_row[r] = 0;
        if (route_index) route_index[r] = 0;
    }
}

// The decode path's route preparation in one launch, for R <= CHUNK routes. Workgroup 0 sorts: expert histogram in
// LDS, exclusive scans of rows and tiles over the experts (thread t owns experts 4t .. 4t + 3), counts / expert_row0,
// the tile table of build_blocks_kernel, the tail rows of fill_tail, then the stable scatter of
// sort_scatter_kernel from the scanned cursors -- the same rows the three-pass sort writes. Workgroups 1.. clear two
// fp32 buffers (float4 counts na, nb).
__global__ __launch_bounds__(SORT_THREADS)
void route_prep_small_kernel(const void* __restrict__ ids, int ids_dtype, const void* __restrict__ weights,
                             int w_dtype, int64_t R, int topk, int n_experts, int tile_rows, int max_tiles,
                             int64_t* __restrict__ token_sorted, uint16_t* __restrict__ weight_sorted,
                             int32_t* __restrict__ expert_of_row, int32_t* __restrict__ counts,
                             int32_t* __restrict__ expert_row0, int32_t* __restrict__ tile_expert,
                             int32_t* __restrict__ tile_row0, int32_t* __restrict__ meta, float4* __restrict__ zero_a,
                             int64_t na, float4* __restrict__ zero_b, int64_t nb)
{
    const int t = threadIdx.x;
    if (blockIdx.x > 0)
    {
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int64_t i = (int64_t) (blockIdx.x - 1) * SORT_THREADS + t; i < na + nb;
             i += (int64_t) (gridDim.x - 1) * SORT_THREADS)
        {
            if (i < na) zero_a[i] = z;
            else zero_b[i - na] = z;
        }
        return;
    }
    static_assert(MAX_EXPERTS == 4 * SORT_THREADS, "four experts per thread in the scans");
    __shared__ int32_t s_cursor[MAX_EXPERTS];
    __shared__ int32_t s_wave_cnt[SORT_WAVES][MAX_EXPERTS];
    __shared__ int32_t s_rows[SORT_THREADS], s_tiles[SORT_THREADS];
    for (int e = t; e < MAX_EXPERTS; e += SORT_THREADS)
    {
        s_cursor[e] = 0;
        for (int w = 0; w < SORT_WAVES; ++w) s_wave_cnt[w][e] = 0;
    }
    __syncthreads();
    int ev[ROUTES_PER_THREAD];
    #pragma unroll
    for (int k = 0; k < ROUTES_PER_THREAD; ++k)
    {
        const int64_t i = (int64_t) k * SORT_THREADS + t;
        ev[k] = (i < R) ? route_id(ids, ids_dtype, i, n_experts) : -1;
    }
    #pragma unroll
    for (int k = 0; k < ROUTES_PER_THREAD; ++k)
        if (ev[k] >= 0) atomicAdd(&s_cursor[ev[k]], 1);
    __syncthreads();
    int c[4], nbk[4], my_rows = 0, my_tiles = 0;
    #pragma unroll
    for (int j = 0; j < 4; ++j)
    {
        c[j] = s_cursor[4 * t + j];                     // zero past n_experts
        nbk[j] = (c[j] + tile_rows - 1) / tile_rows;
        my_rows += c[j];
        my_tiles += nbk[j];
    }
    s_rows[t] = my_rows;
    s_tiles[t] = my_tiles;
    __syncthreads();
    for (int d = 1; d < SORT_THREADS; d <<= 1)         // inclusive scans over the threads
    {
        const int vr = (t >= d) ? s_rows[t - d] : 0;
        const int vt = (t >= d) ? s_tiles[t - d] : 0;
        __syncthreads();
        s_rows[t] += vr;
        s_tiles[t] += vt;
        __syncthreads();
    }
    int row = s_rows[t] - my_rows, tile = s_tiles[t] - my_tiles;
    const int n_rows = s_rows[SORT_THREADS - 1], n_tiles = s_tiles[SORT_THREADS - 1];
    #pragma unroll
    for (int j = 0; j < 4; ++j)
    {
        const int e = 4 * t + j;
        if (e < n_experts)
        {
            counts[e] = c[j];
            expert_row0[e] = row;
            for (int q = 0; q < nbk[j]; ++q)
                if (tile + q < max_tiles) { tile_expert[tile + q] = e; tile_row0[tile + q] = row + q * tile_rows; }
        }
        s_cursor[e] = row;                              // every slot was read into c[] before the scans' barriers
        row += c[j];
        tile += nbk[j];
    }
    if (t == 0) { meta[0] = n_tiles; meta[1] = n_rows; }
    for (int b = n_tiles + t; b < max_tiles; b += SORT_THREADS) tile_expert[b] = -1;
    for (int64_t r = n_rows + t; r < R; r += SORT_THREADS)
    {
        token_sorted[r] = 0;
        weight_sorted[r] = 0;
        expert_of_row[r] = 0;
    }
    __syncthreads();
    scatter_chunk(ids, ids_dtype, weights, w_dtype, R, topk, n_experts, 0, s_cursor, s_wave_cnt, token_sorted,
                  weight_sorted, expert_of_row, nullptr);
}

// Per-expert row tiles of `tile_rows` rows (128 for the reference's block table).
__global__ __launch_bounds__(1024)
void build_blocks_kernel(const int32_t* __restrict__ counts, int n_experts, int tile_rows, int max_blocks,
                         int32_t* __restrict__ block_expert, int32_t* __restrict__ block_row0,
                         int32_t* __restrict__ meta)
{
    __shared__ int32_t s_rows[1024];
    __shared__ int32_t s_blks[1024];
    const int e = threadIdx.x;
    const int c = (e < n_experts) ? counts[e] : 0;
    const int nb = (c + tile_rows - 1) / tile_rows;
    s_rows[e] = c;
    s_blks[e] = nb;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1)
    {
        const int vr = (e >= d) ? s_rows[e - d] : 0;
        const int vb = (e >= d) ? s_blks[e - d] : 0;
        __syncthreads();
        s_rows[e] += vr;
        s_blks[e] += vb;
        __syncthreads();
    }
    const int row0 = s_rows[e] - c;
    const int blk0 = s_blks[e] - nb;
    if (e < n_experts)
        for (int i = 0; i < nb; ++i)
        {
            const int b = blk0 + i;
            if (b < max_blocks) { block_expert[b] = e; block_row0[b] = row0 + i * tile_rows; }
        }
    const int n_blocks = s_blks[1023];
    if (e == 0) { meta[0] = n_blocks; meta[1] = s_rows[1023]; }
    for (int b = n_blocks + e; b < max_blocks; b += 1024) block_expert[b] = -1;
}

// Two tables over the same rows: `tile_rows`-row tiles, except that an expert's last tile goes to a second table of
// `thin_rows`-row tiles when it holds at most thin_rows rows (the thin GEMM kernel runs those at twice the occupancy).
// meta = {full tiles, rows, thin tiles}. Single workgroup of 1024 threads; thread e owns expert e.
__global__ __launch_bounds__(1024)
void build_tiles_split_kernel(const int32_t* __restrict__ counts, int n_experts, int tile_rows, int thin_rows,
                              int max_full, int max_thin, int32_t* __restrict__ full_expert,
                              int32_t* __restrict__ full_row0, int32_t* __restrict__ thin_expert,
                              int32_t* __restrict__ thin_row0, int32_t* __restrict__ meta,
                              float4* __restrict__ zero, int64_t zero4)
{
    if (blockIdx.x > 0)                                   // workgroups 1..: clear the caller's fp32 buffer
    {
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int64_t i = (int64_t) (blockIdx.x - 1) * 1024 + threadIdx.x; i < zero4; i += (int64_t) (gridDim.x - 1) * 1024)
            zero[i] = z;
        return;
    }
    __shared__ int32_t s_rows[1024];
    __shared__ int32_t s_full[1024];
    __shared__ int32_t s_thin[1024];
    const int e = threadIdx.x;
    const int c = (e < n_experts) ? counts[e] : 0;
    const int rem = c % tile_rows;
    const int nthin = (rem > 0 && rem <= thin_rows) ? 1 : 0;
    const int nfull = c / tile_rows + ((rem > thin_rows) ? 1 : 0);
    s_rows[e] = c;
    s_full[e] = nfull;
    s_thin[e] = nthin;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1)
    {
        const int vr = (e >= d) ? s_rows[e - d] : 0;
        const int vf = (e >= d) ? s_full[e - d] : 0;
        const int vt = (e >= d) ? s_thin[e - d] : 0;
        __syncthreads();
        s_rows[e] += vr;
        s_full[e] += vf;
        s_thin[e] += vt;
        __syncthreads();
    }
    const int row0 = s_rows[e] - c;
    const int f0 = s_full[e] - nfull, t0 = s_thin[e] - nthin;
    if (e < n_experts)
    {
        for (int i = 0; i < nfull; ++i)
            if (f0 + i < max_full) { full_expert[f0 + i] = e; full_row0[f0 + i] = row0 + i * tile_rows; }
        if (nthin && t0 < max_thin) { thin_expert[t0] = e; thin_row0[t0] = row0 + (c / tile_rows) * tile_rows; }
    }
    const int n_full = s_full[1023], n_thin = s_thin[1023];
    if (e == 0) { meta[0] = n_full; meta[1] = s_rows[1023]; meta[2] = n_thin; }
    for (int b = n_full + e; b < max_full; b += 1024) full_expert[b] = -1;
    for (int b = n_thin + e; b < max_thin; b += 1024) thin_expert[b] = -1;
}

// ------------------------------------------------------------------------------------------- router top-k
constexpr int ROUTER_VPL = MAX_EXPERTS / 64;           // scores per lane (expert e = lane + 64 i)
constexpr int ROUTER_MAX_TOPK = 16;

__device__ __forceinline__ float load_logit(const void* p, int dtype, int64_t i)
{
    if (dtype == EXL3_DTYPE_F32) return reinterpret_cast<const float*>(p)[i];
    if (dtype == EXL3_DTYPE_F16) return h2f(reinterpret_cast<const uint16_t*>(p)[i]);
    return __uint_as_float((uint32_t) reinterpret_cast<const uint16_t*>(p)[i] << 16);    // bf16
}

// Per token t (one wave): s_e = sigmoid(logit_e) in fp32; the k experts with the largest s_e + bias_e (ties: lower
// expert id) in decreasing order; weight_j = s_(j) / sum_j s_(j) * scale (renorm; the sum runs in selection order) or
// s_(j) * scale. NaN scores are never chosen; if fewer than k finite candidates exist the rest get id -1, weight 0.
__global__ __launch_bounds__(256)
void route_topk_kernel(const void* __restrict__ logits, int logits_dtype, int64_t ld, const float* __restrict__ bias,
                       int64_t tokens, int E, int k, int renorm, float scale, void* __restrict__ ids, int ids_dtype,
                       float* __restrict__ weights)
{
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    for (int64_t t = (int64_t) blockIdx.x * 4 + wv; t < tokens; t += (int64_t) gridDim.x * 4)
    {
        float sel[ROUTER_VPL], sc[ROUTER_VPL];
        #pragma unroll
        for (int i = 0; i < ROUTER_VPL; ++i)
        {
            const int e = lane + 64 * i;
            sel[i] = -INFINITY;
            sc[i] = 0.0f;
            if (e < E)
            {
                const float s = 1.0f / (1.0f + expf(-load_logit(logits, logits_dtype, t * ld + e)));
                sc[i] = s;
                sel[i] = s + (bias ? bias[e] : 0.0f);
            }
        }
        int my_id = -1;
        float my_score = 0.0f, sum = 0.0f;
        for (int j = 0; j < k; ++j)
        {
            float best = -INFINITY, bsc = 0.0f;
            int be = 0x7FFFFFFF;
            #pragma unroll
            for (int i = 0; i < ROUTER_VPL; ++i)
                if (sel[i] > best) { best = sel[i]; bsc = sc[i]; be = lane + 64 * i; }
            #pragma unroll
            for (int off = 32; off >= 1; off >>= 1)
            {
                const float ob = __shfl_xor(best, off);
                const int oe = __shfl_xor(be, off);
                const float os = __shfl_xor(bsc, off);
                if (ob > best || (ob == best && oe < be)) { best = ob; be = oe; bsc = os; }
            }
            if (best == -INFINITY) { be = -1; bsc = 0.0f; }      // no finite candidate left
            else if ((be & 63) == lane)
            {
                #pragma unroll
                for (int i = 0; i < ROUTER_VPL; ++i)
                    if (i == (be >> 6)) sel[i] = -INFINITY;
            }
            if (lane == j) { my_id = be; my_score = bsc; }
            sum += bsc;
        }
        if (lane < k)
        {
            const float w = renorm ? (sum > 0.0f ? my_score / sum * scale : 0.0f) : my_score * scale;
            const int64_t o = t * k + lane;
            if (ids_dtype == EXL3_DTYPE_I64) reinterpret_cast<int64_t*>(ids)[o] = my_id;
            else reinterpret_cast<int32_t*>(ids)[o] = my_id;
            weights[o] = w;
        }
    }
}

}  // namespace
}  // namespace exl3

using namespace exl3;

extern "C" size_t exl3_sort_routes_workspace_bytes(int64_t tokens, int topk, int n_experts)
{
    if (tokens < 0 || topk <= 0 || n_experts <= 0) return 0;
    const int64_t R = tokens * topk;
    const int64_t n_chunks = (R + CHUNK - 1) / CHUNK;
    return (size_t) (256 + 4 * n_chunks * n_experts + 4 * n_chunks);
}

extern "C" int exl3_sort_routes(const void* topk_ids, int ids_dtype, const void* topk_weights, int weights_dtype,
                                int64_t tokens, int topk, int n_experts,
                                int64_t* token_sorted, uint16_t* weight_sorted, int32_t* expert_of_row,
                                int32_t* route_index, int32_t* counts, int32_t* expert_row0,
                                void* workspace, size_t workspace_bytes, void* stream)
{
    EXL3_CHECK(ids_dtype == EXL3_DTYPE_I64 || ids_dtype == EXL3_DTYPE_I32, "topk_ids must be int64 or int32");
    EXL3_CHECK(weights_dtype == EXL3_DTYPE_F32 || weights_dtype == EXL3_DTYPE_F16 || weights_dtype == EXL3_DTYPE_BF16,
               "topk_weights must be float32, float16 or bfloat16");
    EXL3_CHECK(tokens >= 0 && topk > 0, "bad routing shape");
    EXL3_CHECK(n_experts > 0 && n_experts <= MAX_EXPERTS, "too many experts");
    const int64_t R = tokens * topk;
    EXL3_CHECK(R < (int64_t) 1 << 31, "too many routes");
    const size_t need = exl3_sort_routes_workspace_bytes(tokens, topk, n_experts);
    EXL3_CHECK(workspace != nullptr && workspace_bytes >= need, "sort workspace too small (%zu < %zu bytes)",
               workspace_bytes, need);
    EXL3_CHECK(counts && expert_row0, "null output pointer");
    EXL3_CHECK(R == 0 || (topk_ids && topk_weights && token_sorted && weight_sorted && expert_of_row),
               "null pointer");
    hipStream_t s = as_stream(stream);
    int32_t* dropped = reinterpret_cast<int32_t*>(workspace);
    int32_t* hist = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(workspace) + 256);
    const int n_chunks = (int) ((R + CHUNK - 1) / CHUNK);
    int32_t* bad = hist + (int64_t) n_chunks * n_experts;
    if (n_chunks > 0)
        sort_hist_kernel<<<n_chunks, SORT_THREADS, 0, s>>>(topk_ids, ids_dtype, R, n_experts, hist, bad);
    sort_offsets_kernel<<<1, 1024, 0, s>>>(hist, bad, n_chunks, n_experts, counts, expert_row0, dropped);
    if (n_chunks > 0)
    {
        sort_scatter_kernel<<<n_chunks, SORT_THREADS, 0, s>>>(topk_ids, ids_dtype, topk_weights, weights_dtype, R, topk,
                                                              n_experts, hist, counts, expert_row0, token_sorted,
                                                              weight_sorted, expert_of_row, route_index);
    }
    return hip_status("sort_routes");
}

extern "C" int exl3_route_prep_small(const void* topk_ids, int ids_dtype, const void* topk_weights, int weights_dtype,
                                     int64_t tokens, int topk, int n_experts, int tile_rows, int max_tiles,
                                     int64_t* token_sorted, uint16_t* weight_sorted, int32_t* expert_of_row,
                                     int32_t* counts, int32_t* expert_row0, int32_t* tile_expert, int32_t* tile_row0,
                                     int32_t* meta, float* zero_a, int64_t zero_a_floats, float* zero_b,
                                     int64_t zero_b_floats, void* stream)
{
    EXL3_CHECK(ids_dtype == EXL3_DTYPE_I64 || ids_dtype == EXL3_DTYPE_I32, "topk_ids must be int64 or int32");
    EXL3_CHECK(weights_dtype == EXL3_DTYPE_F32 || weights_dtype == EXL3_DTYPE_F16 || weights_dtype == EXL3_DTYPE_BF16,
               "topk_weights must be float32, float16 or bfloat16");
    EXL3_CHECK(tokens >= 0 && topk > 0, "bad routing shape");
    EXL3_CHECK(n_experts > 0 && n_experts <= MAX_EXPERTS, "too many experts");
    EXL3_CHECK(tokens * topk <= CHUNK, "route_prep_small takes at most %d routes", CHUNK);
    EXL3_CHECK(tile_rows == 64 || tile_rows == 128 || tile_rows == 256 || tile_rows == 512,
               "tile_rows must be 64, 128, 256 or 512");
    EXL3_CHECK(max_tiles >= 0 && zero_a_floats >= 0 && zero_b_floats >= 0 && zero_a_floats % 4 == 0 &&
               zero_b_floats % 4 == 0, "bad sizes (zero-fill lengths are whole float4s)");
    const int64_t R = tokens * topk;
    EXL3_CHECK(counts && expert_row0 && meta && (max_tiles == 0 || (tile_expert && tile_row0)), "null pointer");
    EXL3_CHECK(R == 0 || (topk_ids && topk_weights && token_sorted && weight_sorted && expert_of_row), "null pointer");
    EXL3_CHECK((zero_a_floats == 0 || zero_a) && (zero_b_floats == 0 || zero_b) &&
               ((reinterpret_cast<uintptr_t>(zero_a) | reinterpret_cast<uintptr_t>(zero_b)) & 15) == 0,
               "zero-fill buffers must be 16-byte aligned");
    const int64_t n4 = zero_a_floats / 4 + zero_b_floats / 4;
    const int64_t zwgs = std::min<int64_t>((n4 + SORT_THREADS - 1) / SORT_THREADS, 1024);
    route_prep_small_kernel<<<(unsigned) (1 + zwgs), SORT_THREADS, 0, as_stream(stream)>>>(
        topk_ids, ids_dtype, topk_weights, weights_dtype, R, topk, n_experts, tile_rows, max_tiles, token_sorted,
        weight_sorted, expert_of_row, counts, expert_row0, tile_expert, tile_row0, meta,
        reinterpret_cast<float4*>(zero_a), zero_a_floats / 4, reinterpret_cast<float4*>(zero_b), zero_b_floats / 4);
    return hip_status("route_prep_small");
}

extern "C" int exl3_build_tiles(const int32_t* counts, int n_experts, int tile_rows, int max_tiles,
                                int32_t* tile_expert, int32_t* tile_row0, int32_t* meta, void* stream)
{
    EXL3_CHECK(n_experts >= 0 && n_experts <= MAX_EXPERTS, "too many experts");
    EXL3_CHECK(tile_rows == 64 || tile_rows == 128 || tile_rows == 256 || tile_rows == 512,
               "tile_rows must be 64, 128, 256 or 512");
    EXL3_CHECK(max_tiles >= 0, "bad max_blocks");
    EXL3_CHECK(counts && meta && (max_tiles == 0 || (tile_expert && tile_row0)), "null pointer");
    build_blocks_kernel<<<1, 1024, 0, as_stream(stream)>>>(counts, n_experts, tile_rows, max_tiles, tile_expert,
                                                           tile_row0, meta);
    return hip_status("build_blocks");
}

extern "C" int exl3_build_tiles_split(const int32_t* counts, int n_experts, int tile_rows, int thin_rows,
                                      int max_full, int max_thin, int32_t* full_expert, int32_t* full_row0,
                                      int32_t* thin_expert, int32_t* thin_row0, int32_t* meta, float* zero,
                                      int64_t zero_floats, void* stream)
{
    EXL3_CHECK(n_experts >= 0 && n_experts <= MAX_EXPERTS, "too many experts");
    EXL3_CHECK((tile_rows == 128 || tile_rows == 256 || tile_rows == 512) && thin_rows == 64,
               "tile_rows must be 128, 256 or 512 and thin_rows 64");
    EXL3_CHECK(max_full >= 0 && max_thin >= 0, "bad table sizes");
    EXL3_CHECK(counts && meta && (max_full == 0 || (full_expert && full_row0)) &&
               (max_thin == 0 || (thin_expert && thin_row0)), "null pointer");
    EXL3_CHECK(zero_floats >= 0 && zero_floats % 4 == 0 && (zero_floats == 0 || zero) &&
               (reinterpret_cast<uintptr_t>(zero) & 15) == 0, "zero must be 16-byte aligned, a multiple of 4 floats");
    const int64_t zero4 = zero_floats / 4;
    const int64_t zwgs = zero4 > 0 ? std::min<int64_t>((zero4 + 1023) / 1024, 2048) : 0;
    build_tiles_split_kernel<<<(unsigned) (1 + zwgs), 1024, 0, as_stream(stream)>>>(
        counts, n_experts, tile_rows, thin_rows, max_full, max_thin, full_expert, full_row0, thin_expert, thin_row0,
        meta, reinterpret_cast<float4*>(zero), zero4);
    return hip_status("build_tiles_split");
}

extern "C" int exl3_sort_routes_split_tiles(const void* topk_ids, int ids_dtype, const void* topk_weights,
                                            int weights_dtype, int64_t tokens, int topk, int n_experts,
                                            int64_t* token_sorted, uint16_t* weight_sorted, int32_t* expert_of_row,
                                            int32_t* route_index, int32_t* counts, int32_t* expert_row0,
                                            void* workspace, size_t workspace_bytes, int tile_rows, int thin_rows,
                                            int max_full, int max_thin, int32_t* full_expert, int32_t* full_row0,
                                            int32_t* thin_expert, int32_t* thin_row0, int32_t* meta, float* zero,
                                            int64_t zero_floats, void* stream)
{
    EXL3_CHECK(ids_dtype == EXL3_DTYPE_I64 || ids_dtype == EXL3_DTYPE_I32, "topk_ids must be int64 or int32");
    EXL3_CHECK(weights_dtype == EXL3_DTYPE_F32 || weights_dtype == EXL3_DTYPE_F16 || weights_dtype == EXL3_DTYPE_BF16,
               "topk_weights must be float32, float16 or bfloat16");
    EXL3_CHECK(tokens >= 0 && topk > 0, "bad routing shape");
    EXL3_CHECK(n_experts > 0 && n_experts <= MAX_EXPERTS, "too many experts");
    const int64_t R = tokens * topk;
    EXL3_CHECK(R < (int64_t) 1 << 31, "too many routes");
    const size_t need = exl3_sort_routes_workspace_bytes(tokens, topk, n_experts);
    EXL3_CHECK(workspace != nullptr && workspace_bytes >= need, "sort workspace too small (%zu < %zu bytes)",
               workspace_bytes, need);
    EXL3_CHECK(counts && expert_row0, "null output pointer");
    EXL3_CHECK(R == 0 || (topk_ids && topk_weights && token_sorted && weight_sorted && expert_of_row),
               "null pointer");
    EXL3_CHECK((reinterpret_cast<uintptr_t>(workspace) & 15) == 0, "sort workspace must be 16-byte aligned");
    EXL3_CHECK((tile_rows == 128 || tile_rows == 256 || tile_rows == 512) && thin_rows == 64,
               "tile_rows must be 128, 256 or 512 and thin_rows 64");
    EXL3_CHECK(max_full >= 0 && max_thin >= 0, "bad table sizes");
    EXL3_CHECK(meta && (max_full == 0 || (full_expert && full_row0)) && (max_thin == 0 || (thin_expert && thin_row0)),
               "null pointer");
    EXL3_CHECK(zero_floats >= 0 && zero_floats % 4 == 0 && (zero_floats == 0 || zero) &&
               (reinterpret_cast<uintptr_t>(zero) & 15) == 0, "zero must be 16-byte aligned, a multiple of 4 floats");
    hipStream_t s = as_stream(stream);
    int32_t* dropped = reinterpret_cast<int32_t*>(workspace);
    int32_t* hist = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(workspace) + 256);
    const int n_chunks = (int) ((R + CHUNK - 1) / CHUNK);
    int32_t* bad = hist + (int64_t) n_chunks * n_experts;
    if (n_chunks > 0)
        sort_hist_kernel<<<n_chunks, SORT_THREADS, 0, s>>>(topk_ids, ids_dtype, R, n_experts, hist, bad);
    const int64_t zero4 = zero_floats / 4;
    const int64_t zwgs = zero4 > 0 ? std::min<int64_t>((zero4 + SORT_THREADS - 1) / SORT_THREADS, PREP_CLEAR_WGS) : 0;
    sort_scatter_tiles_kernel<<<(unsigned) (n_chunks + 1 + zwgs), SORT_THREADS, 0, s>>>(
        topk_ids, ids_dtype, topk_weights, weights_dtype, R, topk, n_experts, n_chunks, hist, bad, dropped,
        token_sorted, weight_sorted, expert_of_row, route_index, counts, expert_row0, tile_rows, thin_rows, max_full,
        max_thin, full_expert, full_row0, thin_expert, thin_row0, meta, reinterpret_cast<float4*>(zero), zero4);
    return hip_status("sort_routes_split_tiles");
}

extern "C" int exl3_build_blocks(const int32_t* counts, int n_experts, int max_blocks,
                                 int32_t* block_expert, int32_t* block_row0, int32_t* meta, void* stream)
{
    return exl3_build_tiles(counts, n_experts, 128, max_blocks, block_expert, block_row0, meta, stream);
}

extern "C" int exl3_route_topk(const void* logits, int logits_dtype, int64_t logits_ld, const float* bias,
                               int64_t tokens, int n_experts, int topk, int renorm, float scale, void* topk_ids,
                               int ids_dtype, float* topk_weights, void* stream)
{
    EXL3_CHECK(n_experts > 0 && n_experts <= MAX_EXPERTS, "too many experts");
    EXL3_CHECK(topk > 0 && topk <= ROUTER_MAX_TOPK && topk <= n_experts, "topk must be in [1, min(16, n_experts)]");
    EXL3_CHECK(logits_dtype == EXL3_DTYPE_F32 || logits_dtype == EXL3_DTYPE_F16 || logits_dtype == EXL3_DTYPE_BF16,
               "logits must be fp32, fp16 or bf16");
    EXL3_CHECK(ids_dtype == EXL3_DTYPE_I64 || ids_dtype == EXL3_DTYPE_I32, "topk_ids must be int64 or int32");
    EXL3_CHECK(tokens >= 0 && logits_ld >= n_experts, "bad sizes");
    if (tokens == 0) return EXL3_OK;
    EXL3_CHECK(logits && topk_ids && topk_weights, "null pointer");
    const int64_t blocks = (tokens + 3) / 4;
    route_topk_kernel<<<(unsigned) (blocks < 65536 ? blocks : 65536), 256, 0, as_stream(stream)>>>(
        logits, logits_dtype, logits_ld, bias, tokens, n_experts, topk, renorm, scale, topk_ids, ids_dtype,
        topk_weights);
    return hip_status("route_topk");
}
