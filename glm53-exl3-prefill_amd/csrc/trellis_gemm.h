// Weight-stationary trellis GEMM kernels for gfx950: the grouped gate|up / down stages of the EXL3 MoE prefill
// (kernel/exl3_grouped_prefill.cu:148-279) and the single-expert fat GEMM (kernel/exl3_fat_gemm_v2.cu:72-234).
//
// Workgroup = 4 waves, tile = up to 256 rows x 128 output columns (one H128 block), K stage = 32.
//   * Each stage's 16 trellis tiles (32 x 128 weights) are decoded ONCE per workgroup -- a 16-lane row per tile, every
//     lane decoding two 8-weight chunks from one coalesced load of its own stream words -- into a k-contiguous [n][k]
//     fp16 tile in LDS, and reused by all four waves for every row of the tile. A row tile covers `tile_rows` (128 or
//     256) rows of one expert, so each decoded weight feeds up to 256 rows of MFMA work.
//   * Each wave owns 64 rows x 128 columns and runs v_mfma_f32_16x16x32_f16 with the DECODED WEIGHTS as the first
//     operand and the activations as the second (out^T in the accumulators: a lane owns one row and 32 columns). The
//     activation operand of one MFMA is 16 rows x 64 contiguous bytes, so each activation load instruction touches 16
//     cache-line halves -- the vector memory pipeline (TA/TD), not HBM, is what the loads are sized for.
//   * Pipeline of stage s: barrier; read stage s's weight fragments from LDS; decode stage s+1 (VALU) while stage s's
//     MFMAs run; write stage s+1 into the other LDS buffer; issue loads for later stages. Raw trellis words are
//     prefetched RAW_DEPTH stages ahead and activations ACT_DEPTH stages ahead, straight into VGPRs. One barrier per
//     stage guards the double-buffered decoded tile.
//   * A wave with <= 16 valid rows multiplies one 16-row group, a wave with none only decodes (thin experts).
//   * Epilogue: H128 with 5 butterfly stages in registers and 2 across lanes, x svh / sqrt(128), fp16 store, fp32
//     store, fp32 per-route store, or fp32 atomics staged through LDS so each atomic instruction covers 64 consecutive
//     floats of one output row.
//   * Workgroups are laid out XCD-aware: the column tiles of one row tile share an XCD (and its L2).
//   * Optionally (the decode path's split-K gate|up on 64-row tiles) the workgroup that adds the last K slice of a
//     (row tile, 128-column block) pair of gate and up computes that block of the activation (act_had) itself.
//   * Activations and trellis words are read through buffer resources: fixed per-lane offsets plus a scalar stage
//     offset, and zero instead of a fault outside the operand.
// Variants of the same kernel: 16 rows per wave (64-row tiles, four workgroups per CU) for small tiles, and 8 waves
// (512-row tiles, one workgroup per CU, each wave decoding one chunk per lane) for 512-row tiles and large dense GEMMs.
#pragma once
#include "exl3_common.h"
#include "hadamard.h"
#include "trellis_decode.h"

#include <algorithm>
#include <type_traits>

namespace exl3 {


typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int TILE_N = 128;
constexpr int TILE_K = 32;
#ifndef EXL3_LDS_ROW_PAD
#define EXL3_LDS_ROW_PAD 8
#endif
#ifndef EXL3_LDS_BLK_PAD
#define EXL3_LDS_BLK_PAD 64
#endif
constexpr int LDS_ROW = TILE_K + EXL3_LDS_ROW_PAD;  // halves per n-row of the decoded tile (80 B)
constexpr int LDS_BLK = 16 * LDS_ROW + EXL3_LDS_BLK_PAD;   // halves per 16-row block: the pad puts neighbouring
                                                    // tiles' decode stores 32 banks apart
constexpr int LDS_TILE = 8 * LDS_BLK;               // halves per decoded stage (128 n-rows)
constexpr int SC_ROW = TILE_N + 4;                  // floats per staged output row of the scatter epilogue
constexpr int LDS_MAIN_BYTES = 2 * LDS_TILE * 2;
#ifndef EXL3_RAW_DEPTH
#define EXL3_RAW_DEPTH 4
#endif
#ifndef EXL3_ACT_DEPTH
#define EXL3_ACT_DEPTH 2
#endif
constexpr int RAW_DEPTH = EXL3_RAW_DEPTH;           // raw trellis words in flight (stages)
constexpr int ACT_DEPTH = EXL3_ACT_DEPTH;           // activation tiles in flight (stages)
constexpr int UNROLL = 4;                           // stages per loop trip: register buffers keep static names
static_assert(UNROLL % 2 == 0 && UNROLL % RAW_DEPTH == 0 && UNROLL % ACT_DEPTH == 0, "static buffer rotation");

// STORE_F16: fp16 rows (gate|up). SCATTER_F32: fp32 atomic add into out[token[r]]. STORE_F32: fp32 rows (fat GEMM).
// STORE_ROUTE_F32: fp32 rows at out[route_index[r]] (per-route partials for the deterministic combine).
// ATOMIC_F32: fp32 atomic add into out[r] (gate|up partial sums of a split-K launch).
enum { MODE_STORE_F16 = 0, MODE_SCATTER_F32 = 1, MODE_STORE_F32 = 2, MODE_STORE_ROUTE_F32 = 3, MODE_ATOMIC_F32 = 4 };
// Modes whose epilogue stages rows through LDS and adds them to the output with atomics.
constexpr bool atomic_mode(int mode) { return mode == MODE_SCATTER_F32 || mode == MODE_ATOMIC_F32; }

struct GemmParams
{
    const uint16_t* a;             // [a_rows, size_k] fp16, row-major or T16 (a_t16)
    int64_t a_rows;
    int a_t16;
    int size_k;
    const uint16_t* packed0;       // trellis of tensor 0 (gate / single tensor)
    const uint16_t* packed1;       // trellis of tensor 1 (up), may be null
    int64_t expert_stride_words;   // uint16 words between experts
    int tiles_n;                   // 16-col trellis tiles per tensor
    const uint16_t* svh0;
    const uint16_t* svh1;
    int64_t svh_stride;
    const int32_t* block_expert;   // grouped schedule: row tiles of `tile_rows` rows
    const int32_t* block_row0;
    const int32_t* counts;
    const int32_t* expert_row0;
    int tile_rows;                 // rows per row tile (grouped: 128, 256 or 512; dense: 64 x waves)
    int n_groups;                  // row tiles (grouped: table entries; dense: ceil(m / tile_rows))
    int n_slots;                   // 128-col tiles over all tensors
    int n_tiles_each;              // 128-col tiles per tensor
    int k_split;                   // K slices per output tile (0 or 1: none); slices add into the output atomically
    int kb_per_split;              // TILE_K stages per slice (even)
    int64_t m;                     // dense rows
    const int64_t* token;          // scatter destination row per sorted row
    const uint16_t* route_weight;  // fp16 per sorted row
    const int32_t* route_index;    // STORE_ROUTE_F32 destination row per sorted row
    void* out;
    int64_t out_ld;                // elements per output row
    int out_t16;                   // STORE_F16: out in the T16 layout (16-row x 8-column blocks), width out_ld
    // act_had fused into ATOMIC_F32 gate|up on 64-row tiles (act_arrive null: not fused)
    int* act_arrive;               // arrivals per (row tile, 128-column block), zero before the launch
    uint16_t* act_out;             // act fp16, T16 layout, width n_tiles_each * 128
    const uint16_t* act_suh;       // suh_down, row e at act_suh + e * act_suh_stride
    int64_t act_suh_stride;
    float act_limit;
    // SCATTER_F32 thin tiles of the decode path (trellis_gemm_actin_kernel): the fp32 gate|up sums [rows, 2 I] from
    // which each workgroup computes its own K slice of act into LDS (act_suh / act_suh_stride / act_limit as above)
    const float* act_gu;
    // grouped 64-row tiles that read each expert's weights once (the prefill's thin launches, the decode path) load the
    // trellis words non-temporal
    int weights_nt;
    // a side job of the launch: clear zero[0 .. zero4) (float4s), a buffer a later launch accumulates into
    float4* zero;
    int64_t zero4;
};

// A wave's epilogue inputs, staged in LDS while its main loop's pipeline fills (their global loads then overlap the
// first trellis and activation loads instead of each opening a step of the epilogue): the svh of the tile's 128 output
// columns and, for the route modes, every row slot's route weight and destination row (slot 16 mb + tok of the wave's
// group mb; rows past the tile's last clamped to it, as the epilogue clamps them).
struct EpiLds
{
    uint32_t svh[64];              // 128 fp16
    float rw[64];
    int64_t dest[64];
};
constexpr bool route_mode(int mode) { return mode == MODE_SCATTER_F32 || mode == MODE_STORE_ROUTE_F32; }

// In-place Walsh-Hadamard transform of 32 values (Sylvester order over the index bits).
__device__ __forceinline__ void fwht32(float (&x)[32])
{
    #pragma unroll
    for (int len = 1; len < 32; len <<= 1)
        #pragma unroll
        for (int i = 0; i < 32; ++i)
            if (!(i & len))
            {
                const float a = x[i], b = x[i + len];
                x[i] = a + b;
                x[i + len] = a - b;
            }
}

// Raw stream dwords a lane holds per stage. K=4 / K=2: the lane's own 2 / 1 dwords of the tile (one coalesced load
// per 16-lane row) -- the 16-bit look-back of its first chunk is the previous lane's last dword (DPP rotate);
// K=3: the three dwords its two windows touch, loaded directly.
template <int BITS> constexpr int raw_words() { return BITS == 4 ? 2 : (BITS == 2 ? 1 : 3); }

// Value of `v` in the previous lane of this lane's 16-lane row (lane 0 of the row gets lane 15's).
__device__ __forceinline__ uint32_t prev_in_row(uint32_t v)
{
    return (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, 0x121, 0xF, 0xF, false);     // row_ror:1
}

// Raw buffer resource over [base, base + bytes): loads through it take a per-lane 32-bit offset and a uniform scalar
// offset, and return zero (instead of faulting) outside the range. Word 3 selects 32-bit data for untyped access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int64_t bytes)
{
    const int n = (int) (bytes < 0 ? 0 : (bytes > 0x7FFFFFFF ? 0x7FFFFFFF : bytes));
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short) 0, n, 0x00020000);
}

// f(integral_constant<int, I>) for I = 0 .. N-1, unrolled at compile time.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for_from(F&& f)
{
    if constexpr (I < N)
    {
        f(std::integral_constant<int, I>{});
        static_for_from<I + 1, N>(f);
    }
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) { static_for_from<0, N>(f); }

// ------------------------------------------------------------------------------------------- workgroup tile
// The rows (of one expert), tensor and 128-column tile one workgroup computes.
struct Tile
{
    int e, row0, rows_valid, which, nt;
    int kb0, num_kb;               // the workgroup's K slice: TILE_K stages kb0 .. kb0 + num_kb - 1
    const uint32_t* packed;        // the tensor's trellis for expert e
    const uint16_t* svh;           // svh of the tile's 128 output columns
};

// `slot` runs over n_slots x k_split: the column tile, then the K slice.
template <bool DENSE>
__device__ __forceinline__ bool resolve_tile(const GemmParams& p, int group, int slot, Tile& t)
{
    if (group >= p.n_groups) return false;
    const int total_kb = p.size_k / TILE_K;
    t.kb0 = 0;
    t.num_kb = total_kb;
    if (p.k_split > 1)
    {
        const int ks = slot / p.n_slots;
        slot -= ks * p.n_slots;
        t.kb0 = ks * p.kb_per_split;
        t.num_kb = min(p.kb_per_split, total_kb - t.kb0);
        if (t.num_kb <= 0) return false;
    }
    if constexpr (DENSE)
    {
        t.e = 0;
        t.row0 = group * p.tile_rows;
        t.rows_valid = (int) min((int64_t) p.tile_rows, p.m - t.row0);
    }
    else
    {
        t.e = p.block_expert[group];
        if (t.e < 0) return false;
        t.row0 = p.block_row0[group];
        t.rows_valid = min(p.tile_rows, p.expert_row0[t.e] + p.counts[t.e] - t.row0);
    }
    if (t.rows_valid <= 0) return false;
    t.which = slot >= p.n_tiles_each ? 1 : 0;
    t.nt = slot - t.which * p.n_tiles_each;
    t.packed = reinterpret_cast<const uint32_t*>((t.which ? p.packed1 : p.packed0) +
                                                 (int64_t) t.e * p.expert_stride_words);
    t.svh = (t.which ? p.svh1 : p.svh0) + (int64_t) t.e * p.svh_stride + t.nt * TILE_N;
    return true;
}

// ------------------------------------------------------------------------------------------- decoding share
// Wave dw's (0..3) share of decoding each stage. A stage holds 16 trellis tiles (kt, nt8) = (k-tile 0..1, n-tile
// 0..7); wave dw decodes the four tiles kt = dw >> 1, nt8 = 4 (dw & 1) .. + 3 (512 contiguous bytes at 4 bpw), one
// 16-lane row per tile. Lane j16 of a row decodes chunks 2 j16 and 2 j16 + 1 (positions 16 j16 .. + 15): tile column
// a = j16 >> 1 and a + 8, rows 4 b .. 4 b + 3 and 8 + 4 b .. with b = j16 & 1.
template <int N> struct Chunks { Chunk4 c[N]; };

// NT: the raw words are loaded non-temporal (64-row tiles that read each weight once: the prefill's thin launches and
// the decode path).
template <int BITS, bool NT = false>
struct Decoder
{
    static constexpr int AUX = NT ? 2 : 0;                // buffer-load cache policy: 2 = non-temporal
    static constexpr int NDW = 8 * BITS;                  // dwords per tile
    static constexpr int NR = raw_words<BITS>();
    using Out = Chunks<2>;
    __amdgpu_buffer_rsrc_t raw;    // based at the wave's first tile of stage 0
    int stage_bytes, last_kb, tb, wcol0, wcol1;
    uint32_t off[NR];              // per-lane byte offsets of the raw words

    // cols: the thin tiles' column split -- wave dw decodes both k-tiles of n-tiles 2 dw and 2 dw + 1 (the weights of
    // its own 32 output columns; k-tile lane >> 5, n-tile 2 dw + ((lane >> 4) & 1)) instead of the four n-tiles above.
    __device__ __forceinline__ Decoder(const GemmParams& p, const Tile& t, int dw, int lane, int num_kb,
                                       bool cols = false)
    {
        const int j16 = lane & 15;
        const int ta = j16 >> 1;
        tb = j16 & 1;
        const int kt = cols ? (lane >> 5) : (dw >> 1);
        const int nt8 = cols ? 2 * dw + ((lane >> 4) & 1) : 4 * (dw & 1) + (lane >> 4);
        stage_bytes = 2 * p.tiles_n * NDW * 4;
        const int64_t first = cols ? ((int64_t) (2 * t.kb0) * p.tiles_n + t.nt * 8 + 2 * dw) * NDW
                                   : ((int64_t) (2 * t.kb0 + kt) * p.tiles_n + t.nt * 8 + 4 * (dw & 1)) * NDW;
        raw = buffer_rsrc(t.packed + first, ((int64_t) (p.size_k >> 4) * p.tiles_n * NDW - first) * 4);
        last_kb = num_kb - 1;
        const int tile_off = cols ? (kt * p.tiles_n + ((lane >> 4) & 1)) * NDW : (lane >> 4) * NDW;
        if constexpr (BITS == 3)
        {
            const int d0 = (16 * j16 * BITS + BITS - 16) >> 5;  // dword of the first window bit (may be -1)
            #pragma unroll
            for (int i = 0; i < NR; ++i) off[i] = 4 * (tile_off + (d0 + i + NDW) % NDW);
        }
        else
        {
            #pragma unroll
            for (int i = 0; i < NR; ++i) off[i] = 4 * (tile_off + NR * j16 + i);
        }
        wcol0 = nt8 * LDS_BLK + ta * LDS_ROW + kt * 16 + 4 * tb;         // column a, rows 4 b ..
        wcol1 = wcol0 + 8 * LDS_ROW;                                    // column a + 8
    }
    // Raw words of stage kb (clamped to the last stage, so callers may run ahead of the end).
    __device__ __forceinline__ void load(int kb, uint32_t (&r)[NR]) const
    {
        const int so = min(kb, last_kb) * stage_bytes;
        if constexpr (BITS == 4)
        {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(raw, off[0], so, AUX);
            r[0] = v[0];
            r[1] = v[1];
        }
        else
        {
            #pragma unroll
            for (int i = 0; i < NR; ++i) r[i] = __builtin_amdgcn_raw_buffer_load_b32(raw, off[i], so, AUX);
        }
    }
    __device__ __forceinline__ void decode(const uint32_t (&r)[NR], Out& o) const
    {
        Chunk4& c0 = o.c[0];
        Chunk4& c1 = o.c[1];
        if constexpr (BITS == 4)
        {
            const uint32_t prev = prev_in_row(r[1]);
            c0 = decode_chunk<4>(prev, r[0], 20);
            c1 = decode_chunk<4>(r[0], r[1], 20);
        }
        else if constexpr (BITS == 2)
        {
            const uint32_t prev = prev_in_row(r[0]);
            c0 = decode_chunk<2>(prev, r[0], 18);
            c1 = decode_chunk<2>(r[0], r[0], 2);              // window ends inside r[0]
        }
        else
        {
            // chunk pair j16: windows start 19 / 43 bits (j16 even) or 3 / 27 bits (odd) into dw_off[0]. Even lanes
            // shift their words down by 16 bits first, so both kinds decode at the compile-time offsets 3 and 27:
            // constant shifts of a 64-bit window compile to 32-bit funnel shifts, while per-lane 64-bit shift amounts
            // feeding the decoder's asm gave wrong results at random.
            const uint32_t x0 = tb ? r[0] : __builtin_amdgcn_alignbit(r[1], r[0], 16);
            const uint32_t x1 = tb ? r[1] : __builtin_amdgcn_alignbit(r[2], r[1], 16);
            c0 = decode_chunk<3>(x0, x1, 3);
            c1 = decode_chunk<3>(x0, x1, 27);
        }
    }
    __device__ __forceinline__ void store(const Out& o, uint16_t* lds) const
    {
        const Chunk4& c0 = o.c[0];
        const Chunk4& c1 = o.c[1];
        *reinterpret_cast<uint2*>(lds + wcol0) = make_uint2(c0.w[0], c1.w[0]);
        *reinterpret_cast<uint2*>(lds + wcol0 + 8) = make_uint2(c0.w[1], c1.w[1]);
        *reinterpret_cast<uint2*>(lds + wcol1) = make_uint2(c0.w[2], c1.w[2]);
        *reinterpret_cast<uint2*>(lds + wcol1 + 8) = make_uint2(c0.w[3], c1.w[3]);
    }
};

// Wave dw's (0..7) share of decoding each stage in an 8-wave workgroup: the two tiles kt = dw >> 2,
// nt8 = 2 (dw & 3) .. + 1, one 32-lane half per tile. Lane c (0..31) of a half decodes chunk c (positions 8c .. 8c + 7):
// tile column c >> 2 and (c >> 2) + 8, rows 2 (c & 3), + 1, + 8, + 9. Its window bits [8cK + K - 16, 8cK + 8K) sit in
// the two tile dwords lo = floor(b / 32), hi = lo + 1 (mod 8K, the stream is tail-biting) starting `shift` bits into
// lo; 16 + 7K <= 44 bits and shift <= 27 for K <= 4, so two dwords always hold them.
template <int BITS>
struct Decoder1
{
    static constexpr int NDW = 8 * BITS;
    static constexpr int NR = 2;
    using Out = Chunks<1>;
    __amdgpu_buffer_rsrc_t raw;    // based at the wave's first tile of stage 0
    int stage_bytes, last_kb, shift, wcol0, wcol1;
    uint32_t lo_off, hi_off;       // per-lane byte offsets of the two raw words

    __device__ __forceinline__ Decoder1(const GemmParams& p, const Tile& t, int dw, int lane, int num_kb)
    {
        const int c = lane & 31;
        const int kt = dw >> 2;
        const int nt8 = 2 * (dw & 3) + (lane >> 5);
        stage_bytes = 2 * p.tiles_n * NDW * 4;
        const int64_t first = ((int64_t) (2 * t.kb0 + kt) * p.tiles_n + t.nt * 8 + 2 * (dw & 3)) * NDW;
        raw = buffer_rsrc(t.packed + first, ((int64_t) (p.size_k >> 4) * p.tiles_n * NDW - first) * 4);
        last_kb = num_kb - 1;
        const int b0 = 8 * c * BITS + BITS - 16;              // first window bit, >= -15
        const int d0 = b0 >= 0 ? (b0 >> 5) : -1;
        shift = b0 - 32 * d0;
        lo_off = 4 * ((lane >> 5) * NDW + (d0 + NDW) % NDW);
        hi_off = 4 * ((lane >> 5) * NDW + (d0 + 1) % NDW);
        wcol0 = nt8 * LDS_BLK + (c >> 2) * LDS_ROW + kt * 16 + 2 * (c & 3);
        wcol1 = wcol0 + 8 * LDS_ROW;
    }
    __device__ __forceinline__ void load(int kb, uint32_t (&r)[NR]) const
    {
        const int so = min(kb, last_kb) * stage_bytes;
        r[0] = __builtin_amdgcn_raw_buffer_load_b32(raw, lo_off, so, 0);
        r[1] = __builtin_amdgcn_raw_buffer_load_b32(raw, hi_off, so, 0);
    }
    __device__ __forceinline__ void decode(const uint32_t (&r)[NR], Out& o) const
    {
        if constexpr (BITS == 4)
            o.c[0] = decode_chunk<4>(r[0], r[1], 20);             // shift is 20 for every chunk
        else
        {
            // Realign with 32-bit funnel shifts (per-lane 64-bit shift amounts feeding the decoder's asm gave wrong
            // results at random), then decode at the compile-time offset 0.
            const uint32_t x0 = __builtin_amdgcn_alignbit(r[1], r[0], shift);
            const uint32_t x1 = r[1] >> shift;
            o.c[0] = decode_chunk<BITS>(x0, x1, 0);
        }
    }
    __device__ __forceinline__ void store(const Out& o, uint16_t* lds) const
    {
        const Chunk4& c = o.c[0];
        *reinterpret_cast<uint32_t*>(lds + wcol0) = c.w[0];
        *reinterpret_cast<uint32_t*>(lds + wcol0 + 8) = c.w[1];
        *reinterpret_cast<uint32_t*>(lds + wcol1) = c.w[2];
        *reinterpret_cast<uint32_t*>(lds + wcol1 + 8) = c.w[3];
    }
};

// ------------------------------------------------------------------------------------------- multiplying share
// Wave mw's (0..3) share of the MFMA work: tile rows [64 mw, 64 mw + 64) in four groups of 16 (mb).
// v_mfma_f32_16x16x32_f16 with the decoded weights as the first operand (16 columns x 32 k) and the activations as the
// second (32 k x 16 rows): lane l supplies row / column l & 15 and k 8 (l >> 4) .. + 7 of both, and receives row
// (token) l & 15, columns 4 (l >> 4) .. + 3 of the 16 x 16 output. Row-major A: an activation load is 16 rows x 16
// bytes per lane (one lane per cycle in the address unit); T16 A: 256 contiguous bytes per 16-row group.
// Activations are read through a buffer resource based at the tile's first row: per-lane offsets are fixed, the
// stage advance is a scalar offset, so a load needs no vector address arithmetic.
struct Mma
{
    __amdgpu_buffer_rsrc_t a_rsrc;
    uint32_t a_off[4];
    int a_step, wread, last_kb;

    // rpw: rows per wave (contiguous groups), or gstride > 0: the wave's groups are mw, mw + gstride, ...
    __device__ __forceinline__ Mma(const GemmParams& p, const Tile& t, int mw, int lane, int num_kb, int rpw,
                                   int gstride = 0)
    {
        const int tok = lane & 15, kq = lane >> 4;
        a_step = p.a_t16 ? 4 * 128 * 2 : TILE_K * 2;          // bytes per stage
        const int g0 = t.row0 >> 4;
        const int64_t base_el = (p.a_t16 ? (int64_t) g0 * (p.size_k >> 3) * 128 : (int64_t) t.row0 * p.size_k) +
                                (int64_t) t.kb0 * (a_step / 2);       // the slice's first stage
        const int64_t total_el = (p.a_t16 ? (p.a_rows + 15) / 16 * 16 : p.a_rows) * p.size_k;
        a_rsrc = buffer_rsrc(p.a + base_el, (total_el - base_el) * 2);
        #pragma unroll
        for (int mb = 0; mb < 4; ++mb)
        {
            const int row = t.row0 + min((gstride ? 16 * (mw + gstride * mb) : rpw * mw + 16 * mb) + tok,
                                         t.rows_valid - 1);
            a_off[mb] = p.a_t16 ? (uint32_t) ((((row >> 4) - g0) * (p.size_k >> 3) + kq) * 256 + (row & 15) * 16)
                                : (uint32_t) ((row - t.row0) * p.size_k * 2 + 16 * kq);
        }
        wread = tok * LDS_ROW + 8 * kq;
        last_kb = num_kb - 1;
    }
    template <int MBA, int N>
    __device__ __forceinline__ void load_act(int kb, half8_t (&a)[N]) const
    {
        static_assert(MBA <= N, "activation groups");
        const int so = min(kb, last_kb) * a_step;
        #pragma unroll
        for (int mb = 0; mb < MBA; ++mb)
            a[mb] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_off[mb], so, 0));
    }
    __device__ __forceinline__ void read_w(const uint16_t* lds, half8_t (&w)[8]) const
    {
        #pragma unroll
        for (int nb = 0; nb < 8; ++nb) w[nb] = *reinterpret_cast<const half8_t*>(lds + nb * LDS_BLK + wread);
    }
    // The wave's own two column blocks 2 w, 2 w + 1 of the decoded stage (thin tiles' column split).
    __device__ __forceinline__ void read_w2(const uint16_t* lds, int w, half8_t (&f)[2]) const
    {
        f[0] = *reinterpret_cast<const half8_t*>(lds + (2 * w) * LDS_BLK + wread);
        f[1] = *reinterpret_cast<const half8_t*>(lds + (2 * w + 1) * LDS_BLK + wread);
    }
    template <int MBA>
    __device__ __forceinline__ static void mfma2(const half8_t (&f)[2], const half8_t (&a)[4], floatx4 (&acc)[4][2])
    {
        #pragma unroll
        for (int nb = 0; nb < 2; ++nb)
            #pragma unroll
            for (int mb = 0; mb < MBA; ++mb)
                acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f[nb], a[mb], acc[mb][nb], 0, 0, 0);
    }
    template <int MBA, int MBN>
    __device__ __forceinline__ static void mfma(const half8_t (&w)[8], const half8_t (&a)[MBN], floatx4 (&acc)[MBN][8])
    {
        static_assert(MBA <= MBN, "row groups");
        #pragma unroll
        for (int nb = 0; nb < 8; ++nb)
            #pragma unroll
            for (int mb = 0; mb < MBA; ++mb)
                acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[nb], a[mb], acc[mb][nb], 0, 0, 0);
    }
};

// ------------------------------------------------------------------------------------------- epilogue
// pa = {fp16(a0 * s0), fp16(a1 * s1)}, pb = {fp16(b0 * t0), fp16(b1 * t1)}: each exact product rounded once, straight
// to fp16, packed in place. (The reference rounds the product in fp32 first and then to fp16,
// kernel/exl3_grouped_prefill.cu:54-56,273: the two differ by one fp16 step where the fp32 rounding crosses an fp16
// rounding boundary, about one element in 2^13.) A high half is written two instructions after the low half it keeps (gfx950 forwards a
// partial register write stale to the next instruction), and an s_nop guards the last one for the code after.
__device__ __forceinline__ void f16_products_4(float a0, float a1, float b0, float b1, float s0, float s1, float t0,
                                               float t1, uint32_t& pa, uint32_t& pb)
{
    asm("v_fma_mixlo_f16 %0, %2, %6, 0\n\t"
        "v_fma_mixlo_f16 %1, %4, %8, 0\n\t"
        "v_fma_mixhi_f16 %0, %3, %7, 0\n\t"
        "v_fma_mixhi_f16 %1, %5, %9, 0\n\t"
        "s_nop 1"
        : "=&v"(pa), "=&v"(pb) : "v"(a0), "v"(a1), "v"(b0), "v"(b1), "v"(s0), "v"(s1), "v"(t0), "v"(t1));
}

// Per 16-row group of multiplying wave mw (16 MBN rows per wave): H128 over the 128 columns of each row (lane l holds columns
// 16 nb + 4 (l >> 4) + r: 5 butterfly stages in registers, column bit 2 across lanes l ^ 16, bit 3 across l ^ 32),
// scale by svh / sqrt(128) (and the route weight), then store / scatter. The scatter stages each group through LDS
// (`stage`: 16 rows x SC_ROW floats of this wave) so that every atomic instruction covers 64 consecutive floats of
// one output row.
// GSTRIDE > 0: the wave's groups are interleaved over the tile (group mb of wave mw is the tile's 16-row group
// mw + GSTRIDE mb); 0: they are contiguous (rows 16 MBN mw + 16 mb ..).
// epi: the wave's inputs staged in LDS (EpiLds), or null to read them from global memory here.
template <int MODE, int MBN, int GSTRIDE = 0>
__device__ __forceinline__ void epilogue(const GemmParams& p, const Tile& t, int mw, int lane, floatx4 (&acc)[MBN][8],
                                         float* stage, const EpiLds* epi = nullptr)
{
    const int tok = lane & 15, kq = lane >> 4;
    auto group_row0 = [&](int mb) { return GSTRIDE ? 16 * (mw + GSTRIDE * mb) : 16 * MBN * mw + 16 * mb; };
    const int out_col0 = t.which * p.n_tiles_each * TILE_N + t.nt * TILE_N;
    float sv[32];
    #pragma unroll
    for (int nb = 0; nb < 8; ++nb)
    {
        const uint2 v = epi ? *reinterpret_cast<const uint2*>(epi->svh + 8 * nb + 2 * kq)
                            : *reinterpret_cast<const uint2*>(t.svh + 16 * nb + 4 * kq);
        sv[4 * nb + 0] = h2f(v.x & 0xFFFF) * HAD_SCALE;
        sv[4 * nb + 1] = h2f(v.x >> 16) * HAD_SCALE;
        sv[4 * nb + 2] = h2f(v.y & 0xFFFF) * HAD_SCALE;
        sv[4 * nb + 3] = h2f(v.y >> 16) * HAD_SCALE;
    }
    #pragma unroll
    for (int mb = 0; mb < MBN; ++mb)
    {
        const int grow0 = group_row0(mb);                       // the group's first row within the tile
        if (grow0 >= t.rows_valid) break;                       // uniform over the wave
        float x[32];
        #pragma unroll
        for (int nb = 0; nb < 8; ++nb)
            #pragma unroll
            for (int r = 0; r < 4; ++r) x[4 * nb + r] = acc[mb][nb][r];
        fwht32(x);
        #pragma unroll
        for (int i = 0; i < 32; i += 2) pair_butterfly16(x[i], x[i + 1]);
        #pragma unroll
        for (int i = 0; i < 32; i += 2) pair_butterfly32(x[i], x[i + 1]);

        const int r_local = grow0 + tok;                        // this lane's row within the tile
        const bool row_ok = r_local < t.rows_valid;
        const int64_t srow = (int64_t) t.row0 + min(r_local, t.rows_valid - 1);
        float rw = 1.0f;
        int64_t orow = srow;
        if constexpr (route_mode(MODE))
        {
            if (epi)
            {
                rw = epi->rw[16 * mb + tok];
                orow = epi->dest[16 * mb + tok];
            }
            else
            {
                rw = h2f(p.route_weight[srow]);
                orow = (MODE == MODE_SCATTER_F32) ? p.token[srow] : (int64_t) p.route_index[srow];
            }
        }
        #pragma unroll
        for (int nb = 0; nb < 8; ++nb)
        {
            const int col = 16 * nb + 4 * kq;                   // first of this lane's 4 consecutive columns
            float v[4];
            #pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = x[4 * nb + r] * sv[4 * nb + r] * rw;
            if constexpr (atomic_mode(MODE))
            {
                *reinterpret_cast<float4*>(stage + tok * SC_ROW + col) = make_float4(v[0], v[1], v[2], v[3]);
                continue;
            }
            if (!row_ok) continue;
            if constexpr (MODE == MODE_STORE_F16)
            {
                const int64_t c = out_col0 + col;              // a multiple of 4: one half of an 8-column block
                uint16_t* o = reinterpret_cast<uint16_t*>(p.out) +
                              (p.out_t16 ? ((((orow >> 4) * (p.out_ld >> 3) + (c >> 3)) * 16 + (orow & 15)) * 8 + (c & 7))
                                         : orow * p.out_ld + c);
                uint2 pk;                                       // fp16(x * svh / sqrt(128)), single-rounded
                f16_products_4(x[4 * nb], x[4 * nb + 1], x[4 * nb + 2], x[4 * nb + 3], sv[4 * nb], sv[4 * nb + 1],
                               sv[4 * nb + 2], sv[4 * nb + 3], pk.x, pk.y);
                *reinterpret_cast<uint2*>(o) = pk;
            }
            else
            {
                float* o = reinterpret_cast<float*>(p.out) + orow * p.out_ld + out_col0 + col;
                *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
        if constexpr (atomic_mode(MODE))
        {
            // LDS accesses of one wave complete in order: the reads below see the writes above, and the next
            // group's writes land after these reads. Lane t (< 16) holds row t's destination row (token, or the
            // sorted row itself in ATOMIC_F32).
            const int nrows = min(16, t.rows_valid - grow0);
            const uint32_t tok_lo = (uint32_t) orow, tok_hi = (uint32_t) ((uint64_t) orow >> 32);
            float* outp = reinterpret_cast<float*>(p.out) + out_col0 + lane;
            for (int tr = 0; tr < nrows; ++tr)
            {
                const int64_t trow = (int64_t) (((uint64_t) __builtin_amdgcn_readlane(tok_hi, tr) << 32) |
                                                __builtin_amdgcn_readlane(tok_lo, tr));
                const float v0 = stage[tr * SC_ROW + lane];
                const float v1 = stage[tr * SC_ROW + 64 + lane];
                float* o = outp + trow * p.out_ld;
                unsafeAtomicAdd(o, v0);
                unsafeAtomicAdd(o + 64, v1);
            }
        }
    }
}

// Epilogue inputs of a one-row tile in the atomic modes, loaded before the main loop: lane l's svh of columns l and
// l + 64 (scaled by 1 / sqrt(128)), the row's route weight and destination row (uniform).
struct OneRow
{
    float sv0, sv1, rw;
    int64_t dest;
};

template <int MODE>
__device__ __forceinline__ OneRow one_row_inputs(const GemmParams& p, const Tile& t, int lane)
{
    OneRow o;
    o.sv0 = h2f(t.svh[lane]) * HAD_SCALE;
    o.sv1 = h2f(t.svh[lane + 64]) * HAD_SCALE;
    o.rw = 1.0f;
    o.dest = t.row0;
    if constexpr (MODE == MODE_SCATTER_F32)
    {
        o.rw = h2f(p.route_weight[t.row0]);
        o.dest = p.token[t.row0];
    }
    return o;
}

// The epilogue of a tile whose only row is row 0 (atomic modes), run by one wave: the row's 128 sums, as the waves left
// their column blocks in LDS (xs: block b's floatx4 of lane 16 kq + row at b * 64 + lane, columns 16 b + 4 kq + r), are
// gathered as columns l and l + 64 on lane l, so one H128 over 64 lanes replaces sixteen rows' worth of it. The
// butterfly stages run in the general epilogue's order over the column bits (0, 1, 4, 5, 6, then 2 and 3, each stage's
// sums a + b and differences a - b of the same operands), and the scaling multiplies in its order (x * svh / sqrt(128),
// then the route weight), so each output is the general epilogue's bit for bit.
template <int MODE>
__device__ __forceinline__ void one_row_epilogue(const GemmParams& p, const Tile& t, int lane, const float* xs,
                                                 const OneRow& in)
{
    auto at = [&](int c) { return xs[(c >> 4) * 256 + ((c >> 2) & 3) * 64 + (c & 3)]; };
    float x0 = at(lane), x1 = at(lane + 64);
    x0 = lane_butterfly<1>(x0, lane);                   // column bit 0
    x1 = lane_butterfly<1>(x1, lane);
    x0 = lane_butterfly<2>(x0, lane);                   // bit 1
    x1 = lane_butterfly<2>(x1, lane);
    pair_butterfly16(x0, x1);                           // bit 4
    pair_butterfly32(x0, x1);                           // bit 5
    {
        const float s = x0 + x1, d = x0 - x1;           // bit 6
        x0 = s;
        x1 = d;
    }
    x0 = lane_butterfly<4>(x0, lane);                   // bit 2
    x1 = lane_butterfly<4>(x1, lane);
    x0 = lane_butterfly<8>(x0, lane);                   // bit 3
    x1 = lane_butterfly<8>(x1, lane);
    float* o = reinterpret_cast<float*>(p.out) + in.dest * p.out_ld + t.which * p.n_tiles_each * TILE_N +
               t.nt * TILE_N + lane;
    unsafeAtomicAdd(o, x0 * in.sv0 * in.rw);
    unsafeAtomicAdd(o + 64, x1 * in.sv1 * in.rw);
}

// The act of one row's columns 2 l, 2 l + 1 of a 128-column block on lane l, from its fp16-rounded gate / up sums and
// suh_down pair: column bit 0 in registers, bits 1-4 across lanes l ^ 1 .. l ^ 8, bits 5 and 6 across l ^ 16 and
// l ^ 32 -- the stage order of the other mappings, so the same rounding. Packed fp16 pair.
__device__ __forceinline__ uint32_t act_pair(const float* g, const float* u, uint32_t s, float limit, int lane)
{
    float x[2];
    #pragma unroll
    for (int j = 0; j < 2; ++j)
    {
        const float gc = fminf(g[j], limit);
        const float uc = fminf(fmaxf(u[j], -limit), limit);
        x[j] = h2f(f2h(silu_mul(gc, uc))) * h2f((uint16_t) (s >> (16 * j)));   // fp16 rounding point of the reference
    }
    {
        const float s0 = x[0] + x[1], d0 = x[0] - x[1];
        x[0] = s0;
        x[1] = d0;
    }
    #pragma unroll
    for (int j = 0; j < 2; ++j)
    {
        x[j] = lane_butterfly<1>(x[j], lane);
        x[j] = lane_butterfly<2>(x[j], lane);
        x[j] = lane_butterfly<4>(x[j], lane);
        x[j] = lane_butterfly<8>(x[j], lane);
    }
    pair_butterfly16(x[0], x[1]);
    pair_butterfly32(x[0], x[1]);
    return (uint32_t) f2h(x[0] * HAD_SCALE) | ((uint32_t) f2h(x[1] * HAD_SCALE) << 16);
}

// The act of 8 consecutive columns 8 (l & 15) .. of a 128-column block for the row lane l holds (the row-major pass's
// mapping, 4 rows per wave, had128_lane8), from fp16-rounded sums and suh_down. Packed fp16.
__device__ __forceinline__ uint4 act_oct(const float (&g)[8], const float (&u)[8], uint4 s, float limit, int lane)
{
    float ss[8], x[8];
    unpack8(s, ss);
    #pragma unroll
    for (int j = 0; j < 8; ++j)
    {
        const float gc = fminf(g[j], limit);
        const float uc = fminf(fmaxf(u[j], -limit), limit);
        x[j] = h2f(f2h(silu_mul(gc, uc))) * ss[j];                          // fp16 rounding point of the reference
    }
    had128_lane8(x, lane);
    return pack8(x);
}

// act_had fused into the split-K gate|up GEMM of 64-row tiles (ATOMIC_F32 into fp32 gu, both tensors). Every
// workgroup of a (row tile, column block nt) pair -- gate and up, each K slice -- counts its arrival after its adds;
// the one that arrives last (2 k_split arrivals) computes act for the tile's rows over block nt with the activation
// pass's own per-row arithmetic (act_had_row), so the result is the separate pass's. Wave w takes rows 16 w .. + 15.
// No workgroup waits for another: the last one simply goes on.
// Ordering without device-wide cache maintenance (an agent-scope fence writes back and invalidates the whole L2 of
// the XCD, which every workgroup here would pay): an arriving workgroup waits until its adds are acknowledged
// (vmcnt), then counts with a returning device-scope atomic; the last one reads the sums with device-scope atomic
// loads (global loads at device scope, which is also what the compiler makes of an idempotent device-scope
// read-modify-write), so it sees every add that was acknowledged before its arrival count.
__device__ __forceinline__ void act_after_last_slice(const GemmParams& p, const Tile& t, int group, int wave, int lane)
{
    __shared__ int last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's adds are performed before the arrival
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(p.act_arrive + (int64_t) group * p.n_tiles_each + t.nt, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == 2 * max(p.k_split, 1) - 1;
    __syncthreads();
    if (!last) return;                                  // uniform over the workgroup
    const int I = p.n_tiles_each * TILE_N;
    const int64_t W = 2 * (int64_t) I;
    const float* gu = reinterpret_cast<const float*>(p.out);
    const uint16_t* suh_e = p.act_suh + (int64_t) t.e * p.act_suh_stride;
    if (t.rows_valid <= 4)
    {
        // small tiles (the common case of a few tokens): wave 0 alone, with the one-row or four-row mapping, a
        // sixteenth or a quarter of the 16-row mapping's work, the same rounding
        if (wave != 0) return;
        if (t.rows_valid == 1)
        {
            const int64_t r = t.row0;
            const int c = t.nt * TILE_N + 2 * lane;
            float g[2], u[2];
            #pragma unroll
            for (int j = 0; j < 2; ++j)
            {
                g[j] = h2f(f2h(__hip_atomic_load(gu + r * W + c + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)));
                u[j] = h2f(f2h(__hip_atomic_load(gu + r * W + I + c + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)));
            }
            const uint32_t pk = act_pair(g, u, *reinterpret_cast<const uint32_t*>(suh_e + c), p.act_limit, lane);
            const int64_t chunk = (r >> 4) * (I / 8) + t.nt * 16 + (lane >> 2);
            reinterpret_cast<uint32_t*>(p.act_out + chunk * 128 + (r & 15) * 8)[lane & 3] = pk;
            return;
        }
        const int q = lane >> 4, c16 = lane & 15;
        const int64_t r = (int64_t) t.row0 + min(q, t.rows_valid - 1);
        const int c = t.nt * TILE_N + 8 * c16;
        float g[8], u[8];
        load_gu8<true, true>(gu, r * W + c, g);
        load_gu8<true, true>(gu, r * W + I + c, u);
        const uint4 pk = act_oct(g, u, *reinterpret_cast<const uint4*>(suh_e + c), p.act_limit, lane);
        if (q < t.rows_valid)
        {
            const int64_t chunk = (r >> 4) * (I / 8) + t.nt * 16 + c16;
            *reinterpret_cast<uint4*>(p.act_out + chunk * 128 + (r & 15) * 8) = pk;
        }
        return;
    }
    const int rl = lane & 15, cq = lane >> 4;
    const int g0 = 16 * wave;
    if (g0 >= t.rows_valid) return;
    const int64_t r = (int64_t) t.row0 + min(g0 + rl, t.rows_valid - 1);
    float x[32];
    act_had_row<true, false, true>(p.out, r, t.nt, cq, I, p.act_suh + (int64_t) t.e * p.act_suh_stride, p.act_limit, x);
    if (g0 + rl >= t.rows_valid) return;
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        float o[8];
        #pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = x[8 * i + j];
        const int64_t chunk = (r >> 4) * (I / 8) + t.nt * 16 + 4 * i + cq;
        *reinterpret_cast<uint4*>(p.act_out + chunk * 128 + (r & 15) * 8) = pack8(o);
    }
}

// The activation pass for one thin tile's rows over its K slice (whole 128-column blocks of act, at most
// ACTIN_MAX_KB / 4 = 3, one per wave), into LDS as the T16 blocks the main loop multiplies: stage s of the slice is
// 1 KB at dst + s KB, lane l's 16 bytes = row l & 15, k chunk l >> 4 (the layout of one T16 activation load). Each row
// gets the separate pass's arithmetic (clamped SwiGLU rounded to fp16, x suh_down, H128, x 1/sqrt(128), fp16), so the
// slice holds exactly the act that pass would store. The workgroups of the first output column block also store their
// slice's valid rows to act_out (T16), one writer per element, so the act of the call stays in the workspace as the
// other placement leaves it. Two phases, so that the thin tile's first trellis loads go out between them: act_load
// issues the gate|up sum and suh_down loads, act_store computes and writes.
// One row (every tile of a one-token call with distinct experts): lane l takes columns 2 l and 2 l + 1 of the wave's
// block. Up to 4 rows: lane l takes row l >> 4 and the 8 consecutive columns 8 (l & 15) ..
// of the wave's block (the row-major pass's mapping, had128_lane8: a quarter of the work per row of the 16-row
// mapping, the same rounding); rows 4-15 of the slice stay unwritten, and only rows past the tile's last multiply
// them. Taller tiles take the 16-row T16 mapping (act_had_row), loading and computing in the second phase.
static_assert(ACTIN_MAX_KB <= 16, "one act block per wave");

struct ActIn
{
    float g[8], u[8];
    uint4 s;
};
__device__ __forceinline__ void act_load(const GemmParams& p, const Tile& t, int wave, int lane, ActIn& a)
{
    if (t.rows_valid > 4 || wave >= t.num_kb / 4) return;
    const int I = p.size_k;
    if (t.rows_valid == 1)
    {
        // one row: lane l takes columns 2 l and 2 l + 1 of the wave's block
        const int64_t r = t.row0;
        const int c = (t.kb0 / 4 + wave) * 128 + 2 * lane;
        const float2 g = *reinterpret_cast<const float2*>(p.act_gu + r * 2 * (int64_t) I + c);
        const float2 u = *reinterpret_cast<const float2*>(p.act_gu + r * 2 * (int64_t) I + I + c);
        a.g[0] = h2f(f2h(g.x)); a.g[1] = h2f(f2h(g.y));        // the sums as the fp16 gate|up of the reference
        a.u[0] = h2f(f2h(u.x)); a.u[1] = h2f(f2h(u.y));
        a.s.x = *reinterpret_cast<const uint32_t*>(p.act_suh + (int64_t) t.e * p.act_suh_stride + c);
        return;
    }
    const int q = lane >> 4, c16 = lane & 15;
    const int64_t r = (int64_t) t.row0 + min(q, t.rows_valid - 1);
    const int c = (t.kb0 / 4 + wave) * 128 + 8 * c16;
    load_gu8<true, false>(p.act_gu, r * 2 * (int64_t) I + c, a.g);
    load_gu8<true, false>(p.act_gu, r * 2 * (int64_t) I + I + c, a.u);
    a.s = *reinterpret_cast<const uint4*>(p.act_suh + (int64_t) t.e * p.act_suh_stride + c);
}
__device__ __forceinline__ void act_store(const GemmParams& p, const Tile& t, int wave, int lane, const ActIn& a,
                                          unsigned char* dst)
{
    if (wave >= t.num_kb / 4) return;
    const int I = p.size_k;
    const int blk = t.kb0 / 4 + wave;
    uint4* o = reinterpret_cast<uint4*>(dst);
    if (t.rows_valid == 1)
    {
        const uint32_t pk = act_pair(a.g, a.u, a.s.x, p.act_limit, lane);
        // T16: stage lane / 16 of the block, k chunk (lane / 4) % 4, row 0, values 2 (lane % 4) ..
        reinterpret_cast<uint32_t*>(dst)[((4 * wave + (lane >> 4)) * 64 + ((lane >> 2) & 3) * 16) * 4 + (lane & 3)] = pk;
        if (t.nt == 0)
        {
            const int64_t r = t.row0;
            const int64_t chunk = (r >> 4) * (I / 8) + blk * 16 + (lane >> 2);
            reinterpret_cast<uint32_t*>(p.act_out + chunk * 128 + (r & 15) * 8)[lane & 3] = pk;
        }
        return;
    }
    if (t.rows_valid <= 4)
    {
        const int q = lane >> 4, c16 = lane & 15;
        const int64_t r = (int64_t) t.row0 + min(q, t.rows_valid - 1);
        const uint4 pk = act_oct(a.g, a.u, a.s, p.act_limit, lane);
        o[(4 * wave + (c16 >> 2)) * 64 + (c16 & 3) * 16 + q] = pk;
        if (t.nt == 0 && q < t.rows_valid)
        {
            const int64_t chunk = (r >> 4) * (I / 8) + blk * 16 + c16;
            *reinterpret_cast<uint4*>(p.act_out + chunk * 128 + (r & 15) * 8) = pk;
        }
        return;
    }
    const int rl = lane & 15, cq = lane >> 4;
    const int64_t r = (int64_t) t.row0 + min(rl, t.rows_valid - 1);
    float x[32];
    act_had_row<true, false, false>(p.act_gu, r, blk, cq, I, p.act_suh + (int64_t) t.e * p.act_suh_stride,
                                    p.act_limit, x);
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        float v[8];
        #pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = x[8 * i + j];
        const uint4 pk = pack8(v);
        o[(4 * wave + i) * 64 + cq * 16 + rl] = pk;
        if (t.nt == 0 && rl < t.rows_valid)
        {
            const int64_t chunk = (r >> 4) * (I / 8) + blk * 16 + 4 * i + cq;
            *reinterpret_cast<uint4*>(p.act_out + chunk * 128 + (r & 15) * 8) = pk;
        }
    }
}

// Thin tiles of at most 16 rows (one row group; the MBN == 1 kernels, which run most of the decode path's tiles): every
// wave decodes the weights of its own 32 output columns (Decoder cols) into its part of the double-buffered stage tile
// and multiplies the row group by them, so no wave reads weights another wave decoded and the stages need no barrier
// (the LDS accesses of one wave complete in order). Each output element still adds its K stages in order, as the
// shared-tile loop does, so the results are its results bit for bit. Afterwards the accumulators go through LDS so that
// wave 0 holds the group over all 128 columns, the layout of the shared epilogue. (Taller thin tiles keep the shared
// loop: there every wave would load all of the tile's activation rows, and a 1024-token layer ran 3.5% slower.)
// ACT_IN: the activation operand is computed by the workgroup itself (act_load / act_store around the first
// trellis loads) and read from LDS instead of loaded.
// NT: the trellis words are loaded non-temporal (set where each weight is read once; GemmParams::weights_nt).
template <int BITS, int MODE, bool ACT_IN = false, bool NT = false>
__device__ __forceinline__ void thin_tile(const GemmParams& p, const Tile& t, int group, int wave, int lane,
                                          unsigned char* lds_raw)
{
    uint16_t* lds_b = reinterpret_cast<uint16_t*>(lds_raw);
    const int num_kb = t.num_kb;
    using Dec = Decoder<BITS, NT>;
    constexpr int NR = Dec::NR;
    const Dec dec(p, t, wave, lane, num_kb, true);
    const Mma mm(p, t, 0, lane, num_kb, 64);                       // the A operand of row group 0
    // ACT_IN: stage s's activation fragment from the slice in LDS (stages past the last clamped, like the loads)
    auto act_from_lds = [&](int s) {
        const uint4* a = reinterpret_cast<const uint4*>(lds_raw + LDS_MAIN_BYTES);
        return __builtin_bit_cast(half8_t, a[min(s, num_kb - 1) * 64 + lane]);
    };
    floatx4 acc[4][2];
    #pragma unroll
    for (int nb = 0; nb < 2; ++nb) acc[0][nb] = {};
    const bool one_row = atomic_mode(MODE) && t.rows_valid == 1;   // uniform
    OneRow one{};
    if (one_row) one = one_row_inputs<MODE>(p, t, lane);           // in flight with the pipeline's first loads
    {
        uint32_t raw[RAW_DEPTH][NR];
        half8_t act[ACT_DEPTH][4];
        {
            uint32_t r0[NR];
            ActIn ain;
            if constexpr (ACT_IN) act_load(p, t, wave, lane, ain);
            dec.load(0, r0);
            #pragma unroll
            for (int s = 1; s <= RAW_DEPTH; ++s) dec.load(s, raw[s % RAW_DEPTH]);
            if constexpr (ACT_IN)
            {
                act_store(p, t, wave, lane, ain, lds_raw + LDS_MAIN_BYTES);
                __syncthreads();
                #pragma unroll
                for (int s = 0; s < ACT_DEPTH; ++s) act[s][0] = act_from_lds(s);
            }
            else
                #pragma unroll
                for (int s = 0; s < ACT_DEPTH; ++s) mm.load_act<1>(s, act[s]);
            typename Dec::Out o;
            dec.decode(r0, o);
            dec.store(o, lds_b);
        }
        auto trip = [&](int s0, auto n_tag) {
            constexpr int N = decltype(n_tag)::value;
            #pragma unroll
            for (int u = 0; u < N; ++u)
            {
                const int s = s0 + u;
                half8_t f[2];
                mm.read_w2(lds_b + (u & 1) * LDS_TILE, wave, f);  // stage s, which this wave wrote
                typename Dec::Out o;
                dec.decode(raw[(u + 1) % RAW_DEPTH], o);          // stage s + 1
                Mma::mfma2<1>(f, act[u % ACT_DEPTH], acc);
                dec.store(o, lds_b + ((u + 1) & 1) * LDS_TILE);
                dec.load(s + 1 + RAW_DEPTH, raw[(u + 1) % RAW_DEPTH]);
                if constexpr (ACT_IN) act[u % ACT_DEPTH][0] = act_from_lds(s + ACT_DEPTH);
                else mm.load_act<1>(s + ACT_DEPTH, act[u % ACT_DEPTH]);
            }
        };
        using full_trip = std::integral_constant<int, UNROLL>;
        int s0 = 0;
        if (num_kb >= UNROLL)
        {
            trip(0, full_trip{});
            for (s0 = UNROLL; s0 + UNROLL <= num_kb; s0 += UNROLL) trip(s0, full_trip{});
        }
        if (s0 < num_kb) trip(s0, std::integral_constant<int, 2>{});
    }

    // wave 0 collects the group: every wave puts its two column blocks in LDS
    floatx4 full[1][8];
    floatx4* xs = reinterpret_cast<floatx4*>(lds_raw);
    __syncthreads();                                               // the stage tiles are dead
    xs[(2 * wave) * 64 + lane] = acc[0][0];
    xs[(2 * wave + 1) * 64 + lane] = acc[0][1];
    __syncthreads();
    if constexpr (atomic_mode(MODE))
        if (one_row)
        {
            if (wave == 0) one_row_epilogue<MODE>(p, t, lane, reinterpret_cast<const float*>(lds_raw), one);
            if constexpr (MODE == MODE_ATOMIC_F32)
                if (p.act_arrive) act_after_last_slice(p, t, group, wave, lane);   // every wave arrives
            return;
        }
    if (wave == 0)
        #pragma unroll
        for (int nb = 0; nb < 8; ++nb) full[0][nb] = xs[nb * 64 + lane];
    __syncthreads();                                               // LDS free for the epilogue's staging
    float* const stage = reinterpret_cast<float*>(lds_raw) + wave * (16 * SC_ROW);
    if constexpr (MODE == MODE_ATOMIC_F32)
    {
        if (p.act_arrive)                                          // every wave goes on to the arrival barrier
        {
            if (wave == 0) epilogue<MODE, 1, 0>(p, t, 0, lane, full, stage);
            act_after_last_slice(p, t, group, wave, lane);
            return;
        }
    }
    if (wave == 0) epilogue<MODE, 1, 0>(p, t, 0, lane, full, stage);
}

// The main loop of a 128-, 256- or 512-row tile: the waves share each decoded stage (a barrier per stage), each
// multiplying its own rows into acc. epi (may be null): where the wave stages its epilogue inputs. Returns the number
// of 16-row groups the wave multiplied (uniform over the wave).
template <int BITS, int MODE, int MBN, int WAVES>
__device__ __forceinline__ int tile_mainloop(const GemmParams& p, const Tile& t, int wave, int lane,
                                             unsigned char* lds_raw, EpiLds* epi, floatx4 (&acc)[MBN][8])
{
    uint16_t* lds_b = reinterpret_cast<uint16_t*>(lds_raw);
    const int num_kb = t.num_kb;
    using Dec = typename std::conditional<WAVES == 8, Decoder1<BITS>, Decoder<BITS>>::type;
    constexpr int NR = Dec::NR;
    // 8-wave workgroups interleave the 16-row groups over the waves (wave w multiplies groups w, w + 8, ...), so a
    // partial tile keeps both waves of every SIMD equally busy; 4-wave workgroups give each wave 16 MBN contiguous rows.
    constexpr int GSTRIDE = WAVES == 8 ? 8 : 0;
    const Dec dec(p, t, wave, lane, num_kb);
    const Mma mm(p, t, wave, lane, num_kb, 16 * MBN, GSTRIDE);
    const int n_groups = (t.rows_valid + 15) >> 4;
    const int n_w = GSTRIDE ? (n_groups > wave ? (n_groups - wave + GSTRIDE - 1) / GSTRIDE : 0)
                            : min(MBN, max(0, n_groups - MBN * wave));          // this wave's groups (uniform)

    #pragma unroll
    for (int mb = 0; mb < MBN; ++mb)
        #pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[mb][nb] = {};

    // Main loop, specialised on the number of 16-row groups a wave multiplies (MBA: 0 = decode only, 1 for a wave with
    // <= 16 valid rows, else MBN). Every variant runs the same barriers. Loads past the last stage are clamped to it, so
    // every path keeps the same loads in flight.
    // The epilogue's inputs: loaded before the pipeline's first loads, written to LDS after them (so the write waits
    // only for these), read back by the epilogue.
    uint32_t ep_svh;
    float ep_rw = 0.f;
    int64_t ep_dest = 0;
    auto epi_load = [&]() {
        ep_svh = reinterpret_cast<const uint32_t*>(t.svh)[lane];
        if constexpr (route_mode(MODE))
            if (lane < 16 * MBN)
            {
                const int mb = lane >> 4;
                const int r_local = (GSTRIDE ? 16 * (wave + GSTRIDE * mb) : 16 * MBN * wave + 16 * mb) + (lane & 15);
                const int64_t srow = (int64_t) t.row0 + min(r_local, t.rows_valid - 1);
                ep_rw = h2f(p.route_weight[srow]);
                ep_dest = (MODE == MODE_SCATTER_F32) ? p.token[srow] : (int64_t) p.route_index[srow];
            }
    };
    auto epi_store = [&]() {
        epi->svh[lane] = ep_svh;
        if constexpr (route_mode(MODE))
            if (lane < 16 * MBN)
            {
                epi->rw[lane] = ep_rw;
                epi->dest[lane] = ep_dest;
            }
    };
    auto mainloop = [&](auto mba_tag) {
        constexpr int MBA = decltype(mba_tag)::value;
        uint32_t raw[RAW_DEPTH][NR];
        half8_t act[ACT_DEPTH][MBN];
        {
            uint32_t r0[NR];
            if (MBA > 0 && epi) epi_load();
            dec.load(0, r0);
            #pragma unroll
            for (int s = 1; s <= RAW_DEPTH; ++s) dec.load(s, raw[s % RAW_DEPTH]);
            #pragma unroll
            for (int s = 0; s < ACT_DEPTH; ++s) mm.load_act<MBA>(s, act[s]);
            if (MBA > 0 && epi) epi_store();
            typename Dec::Out o;
            dec.decode(r0, o);
            dec.store(o, lds_b);
        }
        // N stages starting at s0 (a multiple of UNROLL, so buffer indices are compile-time)
        auto trip = [&](int s0, auto n_tag) {
            constexpr int N = decltype(n_tag)::value;
            #pragma unroll
            for (int u = 0; u < N; ++u)
            {
                const int s = s0 + u;
                __syncthreads();                                // stage s decoded; buffer (s + 1) & 1 free
                // Keep every stage's work between its barriers: hoisting a later stage's decode above the barrier
                // would make it wait for raw words loaded in the same trip.
                __builtin_amdgcn_sched_barrier(0);
                half8_t w[8];
                if constexpr (MBA > 0) mm.read_w(lds_b + (u & 1) * LDS_TILE, w);
                typename Dec::Out o;
                dec.decode(raw[(u + 1) % RAW_DEPTH], o);        // stage s + 1
                Mma::mfma<MBA>(w, act[u % ACT_DEPTH], acc);
                dec.store(o, lds_b + ((u + 1) & 1) * LDS_TILE);
                dec.load(s + 1 + RAW_DEPTH, raw[(u + 1) % RAW_DEPTH]);
                mm.load_act<MBA>(s + ACT_DEPTH, act[u % ACT_DEPTH]);
            }
        };
        // The first trip is peeled so that the loads in flight at the loop head are the same on entry and on the
        // back edge; the compiler's wait counts there then only wait for the stage they feed. num_kb is even
        // (K % 64 == 0), so what is left after whole trips is 0 or 2 stages.
        using full = std::integral_constant<int, UNROLL>;
        int s0 = 0;
        if (num_kb >= UNROLL)
        {
            trip(0, full{});
            for (s0 = UNROLL; s0 + UNROLL <= num_kb; s0 += UNROLL) trip(s0, full{});
        }
        if (s0 < num_kb) trip(s0, std::integral_constant<int, 2>{});
    };
    if constexpr (GSTRIDE > 0)
    {
        static_assert(MBN == 4, "interleaved groups: up to four per wave");
        switch (n_w)
        {
            case 4: mainloop(std::integral_constant<int, 4>{}); break;
            case 3: mainloop(std::integral_constant<int, 3>{}); break;
            case 2: mainloop(std::integral_constant<int, 2>{}); break;
            case 1: mainloop(std::integral_constant<int, 1>{}); break;
            default: mainloop(std::integral_constant<int, 0>{}); break;
        }
    }
    else if (MBN > 1 && n_w > 1) mainloop(std::integral_constant<int, MBN>{});
    else if (n_w > 0) mainloop(std::integral_constant<int, 1>{});
    else mainloop(std::integral_constant<int, 0>{});
    return n_w;
}

// 128-, 256- and 512-row tiles: the shared main loop, then every wave's epilogue over its rows.
template <int BITS, int MODE, int MBN, int WAVES>
__device__ __forceinline__ void shared_tile(const GemmParams& p, const Tile& t, int group, int wave, int lane,
                                            unsigned char* lds_raw, EpiLds* epi)
{
    constexpr int GSTRIDE = WAVES == 8 ? 8 : 0;
    floatx4 acc[MBN][8];
    const int n_w = tile_mainloop<BITS, MODE, MBN, WAVES>(p, t, wave, lane, lds_raw, epi, acc);

    if constexpr (atomic_mode(MODE)) __syncthreads();            // decoded tiles are dead; LDS becomes staging
    float* const stage = reinterpret_cast<float*>(lds_raw) + wave * (16 * SC_ROW);
    if constexpr (MODE == MODE_ATOMIC_F32 && MBN == 1 && WAVES == 4)
    {
        if (p.act_arrive)                                        // every wave goes on to the arrival barrier
        {
            if (n_w > 0) epilogue<MODE, MBN, GSTRIDE>(p, t, wave, lane, acc, stage, epi);
            act_after_last_slice(p, t, group, wave, lane);
            return;
        }
    }
    if (n_w == 0) return;
    epilogue<MODE, MBN, GSTRIDE>(p, t, wave, lane, acc, stage, epi);
}

// ------------------------------------------------------------------------------------------- kernel
// 128- and 256-row tiles: every wave decodes a quarter of each stage and multiplies its own 64 rows; two workgroups
// share a CU. Pipeline of stage s: barrier; read stage s's weight fragments; decode stage s+1 while stage s's MFMAs run;
// write stage s+1 into the other of two LDS buffers; issue loads for later stages.
template <int WAVES> constexpr int lds_scatter_bytes() { return WAVES * 16 * SC_ROW * 4; }

// MBN: 16-row groups per wave. 4 (the default): 256-row tiles, two workgroups per CU. 1 (thin): 64-row tiles of small
// batches (those of at most 16 rows split by columns over the waves, thin_tile); a quarter of the accumulators lets four
// workgroups share a CU.
// WAVES = 8: 512-row tiles, one workgroup per CU; each wave decodes half as much of every stage (one chunk per lane),
// so a decoded weight feeds twice the rows for the same VALU work per wave.
template <int BITS, int MODE, bool DENSE, int MBN = 4, int WAVES = 4, bool NT = false>
// (HIP's second launch bound is the minimum number of waves per SIMD: 2 leaves 256 VGPRs per wave, 4 leaves 128.)
__global__ __launch_bounds__(64 * WAVES, MBN == 4 ? 2 : 4)
void trellis_gemm_kernel(const GemmParams p)
{
    static_assert(WAVES == 4 || (WAVES == 8 && MBN == 4), "8-wave workgroups run 64 rows per wave");
    constexpr int SCB = lds_scatter_bytes<WAVES>();
    constexpr int LDS_BYTES = (atomic_mode(MODE) && SCB > LDS_MAIN_BYTES) ? SCB : LDS_MAIN_BYTES;
    __shared__ __align__(16) unsigned char lds_raw[LDS_BYTES];
    __shared__ EpiLds lds_epi[WAVES];

    if (p.zero4 > 0)                    // every workgroup, tile or not, clears its grid-strided share up front; the
    {                                   // stores drain while the tile computes
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < p.zero4;
             i += (int64_t) gridDim.x * blockDim.x)
            p.zero[i] = z;
    }
    int group, slot;
    xcd_group_slot((int) blockIdx.x, p.k_split > 1 ? p.n_slots * p.k_split : p.n_slots, group, slot);
    Tile t;
    if (!resolve_tile<DENSE>(p, group, slot, t)) return;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (MBN == 1 && t.rows_valid <= 16)                           // uniform over the workgroup
        thin_tile<BITS, MODE, false, NT>(p, t, group, wave, lane, lds_raw);
    else
        shared_tile<BITS, MODE, MBN, WAVES>(p, t, group, wave, lane, lds_raw, lds_epi + wave);
}

// The decode path's down GEMM with the activation pass inside (SCATTER_F32 on 64-row tiles of at most 16 rows): each
// workgroup computes the act of its tile's rows over its K slice from the fp32 gate|up sums (act_load, act_store) while
// its first trellis loads are in flight and multiplies it from LDS, so the gate|up launch ends without the pass. The
// host sends it only calls of at most 16 routes (so no tile holds more than 16 rows) and K slices of whole 128-column
// act blocks, at most ACTIN_MAX_KB stages each.
template <int BITS, bool NT>
__global__ __launch_bounds__(256, 4)
void trellis_gemm_actin_kernel(const GemmParams p)
{
    constexpr int SCB = lds_scatter_bytes<4>();
    constexpr int ACT_END = LDS_MAIN_BYTES + ACTIN_MAX_KB * 1024;
    __shared__ __align__(16) unsigned char lds_raw[SCB > ACT_END ? SCB : ACT_END];
    int group, slot;
    xcd_group_slot((int) blockIdx.x, p.k_split > 1 ? p.n_slots * p.k_split : p.n_slots, group, slot);
    Tile t;
    if (!resolve_tile<false>(p, group, slot, t)) return;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    thin_tile<BITS, MODE_SCATTER_F32, true, NT>(p, t, group, wave, lane, lds_raw);
}

template <int BITS>
int launch_gemm_actin(const GemmParams& p, hipStream_t s)
{
    const int groups8 = (p.n_groups + 7) / 8 * 8;
    const int64_t grid = (int64_t) groups8 * p.n_slots * (p.k_split > 1 ? p.k_split : 1);
    if (grid == 0) return EXL3_OK;
    if (grid > 0x7FFFFFFF) return fail("grid too large");
    if (p.weights_nt) trellis_gemm_actin_kernel<BITS, true><<<(unsigned) grid, 256, 0, s>>>(p);
    else trellis_gemm_actin_kernel<BITS, false><<<(unsigned) grid, 256, 0, s>>>(p);
    return EXL3_OK;
}

// A dense GEMM whose 256-row tiles would leave CUs idle (long K, few rows): the two K halves of one tile run in one
// workgroup of 8 waves, waves 0-3 over the first half and 4-7 over the second, each half the 4-wave main loop over its
// own double-buffered stage tiles (the barriers are shared: both halves run the same number of stages). The second
// half's accumulators are then added to the first's through LDS, one 16-row group at a time, and the first half's
// waves run the epilogue: twice the waves per tile with plain stores -- no zeroed output, no atomics, and the same
// summation order on every run (the sum over K: first half + second half, each in stage order).
constexpr int KPAIR_LDS_BYTES = 2 * LDS_MAIN_BYTES;
static_assert(KPAIR_LDS_BYTES >= 4 * 8 * 64 * 16, "one row group of four waves' accumulators");

template <int BITS, int MODE, bool DENSE>
__global__ __launch_bounds__(512, 2)
void trellis_gemm_kpair_kernel(const GemmParams p)
{
    static_assert(MODE == MODE_STORE_F32 || MODE == MODE_STORE_F16, "plain-store modes");
    __shared__ __align__(16) unsigned char lds_raw[KPAIR_LDS_BYTES];
    __shared__ EpiLds lds_epi[4];
    int group, slot;
    xcd_group_slot((int) blockIdx.x, p.n_slots, group, slot);
    Tile t;
    if (!resolve_tile<DENSE>(p, group, slot, t)) return;          // uniform over the workgroup
    const int lane = threadIdx.x & 63;
    const int wave8 = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int half = wave8 >> 2, wave = wave8 & 3;
    Tile th = t;
    th.num_kb = t.num_kb / 2;                                      // even: the host requires K % 128 == 0
    th.kb0 = t.kb0 + half * th.num_kb;
    floatx4 acc[4][8];
    const int n_w = tile_mainloop<BITS, MODE, 4, 4>(p, th, wave, lane, lds_raw + half * LDS_MAIN_BYTES,
                                                    half ? nullptr : lds_epi + wave, acc);
    floatx4* xs = reinterpret_cast<floatx4*>(lds_raw) + wave * 8 * 64 + lane;
    #pragma unroll
    for (int mb = 0; mb < 4; ++mb)
    {
        __syncthreads();                            // mb = 0: both main loops are done with the stage tiles
        if (half == 1 && mb < n_w)
            #pragma unroll
            for (int nb = 0; nb < 8; ++nb) xs[nb * 64] = acc[mb][nb];
        __syncthreads();
        if (half == 0 && mb < n_w)
            #pragma unroll
            for (int nb = 0; nb < 8; ++nb) acc[mb][nb] += xs[nb * 64];
    }
    if (half == 0 && n_w > 0) epilogue<MODE, 4, 0>(p, t, wave, lane, acc, nullptr, lds_epi + wave);
}

// The K-pair schedule for a dense store: 256-row tiles, one 8-wave workgroup per (tile, 128-column block).
template <int BITS, int MODE, bool DENSE>
int launch_gemm_kpair(const GemmParams& p, hipStream_t s)
{
    if constexpr (MODE == MODE_STORE_F32 || MODE == MODE_STORE_F16)
    {
        if (p.tile_rows != 256 || (p.size_k / TILE_K) % 4 != 0 || p.k_split > 1)
            return fail("internal: K-pair launch needs 256-row tiles and K %% 128 == 0");
        const int64_t grid = (int64_t) (p.n_groups + 7) / 8 * 8 * p.n_slots;
        if (grid == 0) return EXL3_OK;
        if (grid > 0x7FFFFFFF) return fail("grid too large");
        trellis_gemm_kpair_kernel<BITS, MODE, DENSE><<<(unsigned) grid, 512, 0, s>>>(p);
        return EXL3_OK;
    }
    return fail("internal: K-pair launch for mode %d", MODE);
}

// 512-row tiles run the 8-wave variant, 128- and 256-row tiles the 4-wave kernel (the only one built for ATOMIC_F32,
// whose split-K launches serve small batches), 64-row tiles the thin 4-wave variant.
template <int BITS, int MODE, bool DENSE>
int launch_gemm(const GemmParams& p, hipStream_t s)
{
    const int groups8 = (p.n_groups + 7) / 8 * 8;
    const int64_t grid = (int64_t) groups8 * p.n_slots * (p.k_split > 1 ? p.k_split : 1);
    if (grid == 0) return EXL3_OK;
    if (grid > 0x7FFFFFFF) return fail("grid too large");
    if (p.tile_rows == 64)
    {
        if constexpr (!DENSE)
            if (p.weights_nt)
            {
                trellis_gemm_kernel<BITS, MODE, DENSE, 1, 4, true><<<(unsigned) grid, 256, 0, s>>>(p);
                return EXL3_OK;
            }
        trellis_gemm_kernel<BITS, MODE, DENSE, 1><<<(unsigned) grid, 256, 0, s>>>(p);
        return EXL3_OK;
    }
    if constexpr (MODE == MODE_ATOMIC_F32)
    {
        if (p.tile_rows > 256) return fail("mode 3 (fp32 atomic rows) takes row tiles of at most 256 rows");
    }
    else if (p.tile_rows > 256)
    {
        trellis_gemm_kernel<BITS, MODE, DENSE, 4, 8><<<(unsigned) grid, 512, 0, s>>>(p);
        return EXL3_OK;
    }
    trellis_gemm_kernel<BITS, MODE, DENSE><<<(unsigned) grid, 256, 0, s>>>(p);
    return EXL3_OK;
}

// One translation unit per trellis width instantiates the kernels (they compile slowly); the entry points dispatch to
// them here. mode is one of the MODE_* values, dense selects the single-matrix schedule.
int launch_gemm_b2(int mode, bool dense, const GemmParams& p, hipStream_t s);
int launch_gemm_b3(int mode, bool dense, const GemmParams& p, hipStream_t s);
int launch_gemm_b4g(int mode, const GemmParams& p, hipStream_t s);
int launch_gemm_b4d(int mode, const GemmParams& p, hipStream_t s);
int launch_gemm_kpair_b2(int mode, const GemmParams& p, hipStream_t s);
int launch_gemm_kpair_b3(int mode, const GemmParams& p, hipStream_t s);
int launch_gemm_kpair_b4(int mode, const GemmParams& p, hipStream_t s);
int launch_gemm_actin_b2(const GemmParams& p, hipStream_t s);
int launch_gemm_actin_b3(const GemmParams& p, hipStream_t s);
int launch_gemm_actin_b4(const GemmParams& p, hipStream_t s);

}  // namespace exl3
