// Weight-stationary trellis GEMM for gfx950: the grouped gate|up / down stages of the EXL3 MoE prefill
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
//   * Activations and trellis words are read through buffer resources: fixed per-lane offsets plus a scalar stage
//     offset, and zero instead of a fault outside the operand.
// Variants of the same kernel: 16 rows per wave (64-row tiles, four workgroups per CU) for small tiles, and 8 waves
// (512-row tiles, one workgroup per CU, each wave decoding one chunk per lane) for 512-row tiles and large dense GEMMs.
#include "exl3_common.h"
#include "trellis_decode.h"

#include <algorithm>
#include <type_traits>

namespace exl3 {
namespace {

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
};

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

template <int BITS>
struct Decoder
{
    static constexpr int NDW = 8 * BITS;                  // dwords per tile
    static constexpr int NR = raw_words<BITS>();
    using Out = Chunks<2>;
    __amdgpu_buffer_rsrc_t raw;    // based at the wave's first tile of stage 0
    int stage_bytes, last_kb, tb, wcol0, wcol1;
    uint32_t off[NR];              // per-lane byte offsets of the raw words

    __device__ __forceinline__ Decoder(const GemmParams& p, const Tile& t, int dw, int lane, int num_kb)
    {
        const int j16 = lane & 15;
        const int ta = j16 >> 1;
        tb = j16 & 1;
        const int kt = dw >> 1;
        const int nt8 = 4 * (dw & 1) + (lane >> 4);
        stage_bytes = 2 * p.tiles_n * NDW * 4;
        const int64_t first = ((int64_t) (2 * t.kb0 + kt) * p.tiles_n + t.nt * 8 + 4 * (dw & 1)) * NDW;
        raw = buffer_rsrc(t.packed + first, ((int64_t) (p.size_k >> 4) * p.tiles_n * NDW - first) * 4);
        last_kb = num_kb - 1;
        const int tile_off = (lane >> 4) * NDW;
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
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(raw, off[0], so, 0);
            r[0] = v[0];
            r[1] = v[1];
        }
        else
        {
            #pragma unroll
            for (int i = 0; i < NR; ++i) r[i] = __builtin_amdgcn_raw_buffer_load_b32(raw, off[i], so, 0);
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

    __device__ __forceinline__ Mma(const GemmParams& p, const Tile& t, int mw, int lane, int num_kb, int rpw)
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
            const int row = t.row0 + min(rpw * mw + 16 * mb + tok, t.rows_valid - 1);
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
// Per 16-row group of multiplying wave mw (16 MBN rows per wave): H128 over the 128 columns of each row (lane l holds columns
// 16 nb + 4 (l >> 4) + r: 5 butterfly stages in registers, column bit 2 across lanes l ^ 16, bit 3 across l ^ 32),
// scale by svh / sqrt(128) (and the route weight), then store / scatter. The scatter stages each group through LDS
// (`stage`: 16 rows x SC_ROW floats of this wave) so that every atomic instruction covers 64 consecutive floats of
// one output row.
template <int MODE, int MBN>
__device__ __forceinline__ void epilogue(const GemmParams& p, const Tile& t, int mw, int lane, floatx4 (&acc)[MBN][8],
                                         float* stage)
{
    const int tok = lane & 15, kq = lane >> 4;
    const int rows_w = t.rows_valid - 16 * MBN * mw;
    const int out_col0 = t.which * p.n_tiles_each * TILE_N + t.nt * TILE_N;
    float sv[32];
    #pragma unroll
    for (int nb = 0; nb < 8; ++nb)
    {
        const uint2 v = *reinterpret_cast<const uint2*>(t.svh + 16 * nb + 4 * kq);
        sv[4 * nb + 0] = h2f(v.x & 0xFFFF) * HAD_SCALE;
        sv[4 * nb + 1] = h2f(v.x >> 16) * HAD_SCALE;
        sv[4 * nb + 2] = h2f(v.y & 0xFFFF) * HAD_SCALE;
        sv[4 * nb + 3] = h2f(v.y >> 16) * HAD_SCALE;
    }
    #pragma unroll
    for (int mb = 0; mb < MBN; ++mb)
    {
        if (16 * mb >= rows_w) break;                           // uniform over the wave
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

        const int r_local = 16 * MBN * mw + 16 * mb + tok;     // this lane's row within the tile
        const bool row_ok = r_local < t.rows_valid;
        const int64_t srow = (int64_t) t.row0 + min(r_local, t.rows_valid - 1);
        float rw = 1.0f;
        int64_t orow = srow;
        if constexpr (MODE == MODE_SCATTER_F32 || MODE == MODE_STORE_ROUTE_F32)
        {
            rw = h2f(p.route_weight[srow]);
            orow = (MODE == MODE_SCATTER_F32) ? p.token[srow] : (int64_t) p.route_index[srow];
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
                uint2 pk;
                pk.x = (uint32_t) f2h(v[0]) | ((uint32_t) f2h(v[1]) << 16);
                pk.y = (uint32_t) f2h(v[2]) | ((uint32_t) f2h(v[3]) << 16);
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
            const int nrows = min(16, rows_w - 16 * mb);
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

// ------------------------------------------------------------------------------------------- kernel
// 128- and 256-row tiles: every wave decodes a quarter of each stage and multiplies its own 64 rows; two workgroups
// share a CU. Pipeline of stage s: barrier; read stage s's weight fragments; decode stage s+1 while stage s's MFMAs run;
// write stage s+1 into the other of two LDS buffers; issue loads for later stages.
template <int WAVES> constexpr int lds_scatter_bytes() { return WAVES * 16 * SC_ROW * 4; }

// MBN: 16-row groups per wave. 4 (the default): 256-row tiles, two workgroups per CU. 1 (thin): 64-row tiles of small
// batches, where most waves only decode; a quarter of the accumulators lets four workgroups share a CU.
// WAVES = 8: 512-row tiles, one workgroup per CU; each wave decodes half as much of every stage (one chunk per lane),
// so a decoded weight feeds twice the rows for the same VALU work per wave.
template <int BITS, int MODE, bool DENSE, int MBN = 4, int WAVES = 4>
// (HIP's second launch bound is the minimum number of waves per SIMD: 2 leaves 256 VGPRs per wave, 4 leaves 128.)
__global__ __launch_bounds__(64 * WAVES, MBN == 4 ? 2 : 4)
void trellis_gemm_kernel(const GemmParams p)
{
    static_assert(WAVES == 4 || (WAVES == 8 && MBN == 4), "8-wave workgroups run 64 rows per wave");
    constexpr int SCB = lds_scatter_bytes<WAVES>();
    constexpr int LDS_BYTES = (atomic_mode(MODE) && SCB > LDS_MAIN_BYTES) ? SCB : LDS_MAIN_BYTES;
    __shared__ __align__(16) unsigned char lds_raw[LDS_BYTES];
    uint16_t* lds_b = reinterpret_cast<uint16_t*>(lds_raw);

    int group, slot;
    xcd_group_slot((int) blockIdx.x, p.k_split > 1 ? p.n_slots * p.k_split : p.n_slots, group, slot);
    Tile t;
    if (!resolve_tile<DENSE>(p, group, slot, t)) return;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int num_kb = t.num_kb;
    using Dec = typename std::conditional<WAVES == 8, Decoder1<BITS>, Decoder<BITS>>::type;
    constexpr int NR = Dec::NR;
    const Dec dec(p, t, wave, lane, num_kb);
    const Mma mm(p, t, wave, lane, num_kb, 16 * MBN);
    const int rows_w = t.rows_valid - 16 * MBN * wave;    // valid rows of this wave (uniform)

    floatx4 acc[MBN][8];
    #pragma unroll
    for (int mb = 0; mb < MBN; ++mb)
        #pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[mb][nb] = {};

    // Main loop, specialised on the number of 16-row groups a wave multiplies (MBA: 0 = decode only, 1 for a wave with
    // <= 16 valid rows, else MBN). Every variant runs the same barriers. Loads past the last stage are clamped to it, so
    // every path keeps the same loads in flight.
    auto mainloop = [&](auto mba_tag) {
        constexpr int MBA = decltype(mba_tag)::value;
        uint32_t raw[RAW_DEPTH][NR];
        half8_t act[ACT_DEPTH][MBN];
        {
            uint32_t r0[NR];
            dec.load(0, r0);
            #pragma unroll
            for (int s = 1; s <= RAW_DEPTH; ++s) dec.load(s, raw[s % RAW_DEPTH]);
            #pragma unroll
            for (int s = 0; s < ACT_DEPTH; ++s) mm.load_act<MBA>(s, act[s]);
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
    if (MBN > 1 && rows_w > 16) mainloop(std::integral_constant<int, MBN>{});
    else if (rows_w > 0) mainloop(std::integral_constant<int, 1>{});
    else mainloop(std::integral_constant<int, 0>{});

    if constexpr (atomic_mode(MODE)) __syncthreads();            // decoded tiles are dead; LDS becomes staging
    if (rows_w <= 0) return;
    epilogue<MODE>(p, t, wave, lane, acc, reinterpret_cast<float*>(lds_raw) + wave * (16 * SC_ROW));
}

// out[t, :] = sum_j partial[t*topk + j, :] in order j = 0 .. topk-1 (deterministic), skipping routes whose id is
// outside [0, n_experts) (their partial rows were never written).
__global__ __launch_bounds__(256)
void combine_routes_kernel(const float4* __restrict__ partial, float4* __restrict__ out, const void* __restrict__ ids,
                           int ids_dtype, int n_experts, int64_t tokens, int topk, int64_t n4)
{
    const int64_t total = tokens * n4;
    for (int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t) gridDim.x * blockDim.x)
    {
        const int64_t t = idx / n4, c = idx - t * n4;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int j = 0; j < topk; ++j)
        {
            const int64_t i = t * topk + j;
            if (ids)
            {
                const int64_t e = ids_dtype == EXL3_DTYPE_I64 ? reinterpret_cast<const int64_t*>(ids)[i]
                                                             : reinterpret_cast<const int32_t*>(ids)[i];
                if (e < 0 || e >= n_experts) continue;
            }
            const float4 v = partial[i * n4 + c];
            acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
        }
        out[idx] = acc;
    }
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

// 512-row tiles run the 8-wave variant, 128- and 256-row tiles the 4-wave kernel (the only one built for ATOMIC_F32,
// whose split-K launches serve small batches), 64-row tiles of grouped modes 0, 1 and 3 the thin 4-wave variant.
template <int BITS, int MODE, bool DENSE>
int launch_gemm(const GemmParams& p, hipStream_t s)
{
    const int groups8 = (p.n_groups + 7) / 8 * 8;
    const int64_t grid = (int64_t) groups8 * p.n_slots * (p.k_split > 1 ? p.k_split : 1);
    if (grid == 0) return EXL3_OK;
    if (grid > 0x7FFFFFFF) return fail("grid too large");
    if constexpr (MODE != MODE_STORE_ROUTE_F32)
    {
        if (p.tile_rows == 64)
        {
            trellis_gemm_kernel<BITS, MODE, DENSE, 1><<<(unsigned) grid, 256, 0, s>>>(p);
            return EXL3_OK;
        }
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

template <int MODE, bool DENSE>
int launch_bits(int bits, const GemmParams& p, hipStream_t s)
{
    switch (bits)
    {
        case 2: return launch_gemm<2, MODE, DENSE>(p, s);
        case 3: return launch_gemm<3, MODE, DENSE>(p, s);
        case 4: return launch_gemm<4, MODE, DENSE>(p, s);
        default: return fail("unsupported bits %d (2, 3 or 4)", bits);
    }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace
}  // namespace exl3

using namespace exl3;

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
    EXL3_CHECK(tile_rows == 128 || tile_rows == 256 || tile_rows == 512 ||
               (tile_rows == 64 && mode != EXL3_GEMM_STORE_ROUTE_F32),
               "tile_rows must be 128, 256 or 512 (or 64 in modes 0, 1, 3 and 4)");
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
    hipStream_t s = as_stream(stream);
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
        rc = launch_bits<MODE_SCATTER_F32, false>(bits, p, s);
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

template <int MODE>
int launch_dense_split2(GemmParams p, int bits, float* out, int64_t out_floats, hipStream_t s)
{
    const int total_kb = p.size_k / TILE_K;
    p.tile_rows = p.m <= 1024 ? 64 : 256;                       // thin tiles here too, up to 1024 rows (measured)
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
    p.svh0 = svh; p.tile_rows = dense_tile_rows(m, size_k); p.n_groups = (int) ((m + p.tile_rows - 1) / p.tile_rows);
    p.n_tiles_each = (int) (svh_len / TILE_N);
    p.n_slots = p.n_tiles_each; p.m = m; p.out = out; p.out_ld = svh_len;
    rc = dense_split_pays(m, p.n_slots, size_k)
             ? launch_dense_split2<MODE_ATOMIC_F32>(p, bits, out, m * svh_len, as_stream(stream))
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
    p.svh0 = svh; p.tile_rows = dense_tile_rows(m, size_k); p.n_groups = (int) ((m + p.tile_rows - 1) / p.tile_rows);
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
    if (out_dtype == EXL3_DTYPE_F32 && dense_split_pays(m, p.n_slots, k))
        rc = launch_dense_split2<MODE_ATOMIC_F32>(p, bits, reinterpret_cast<float*>(out), m * n, s);
    else
        rc = out_dtype == EXL3_DTYPE_F32 ? launch_bits<MODE_STORE_F32, true>(bits, p, s)
                                         : launch_bits<MODE_STORE_F16, true>(bits, p, s);
    if (rc) return rc;
    return hip_status("linear");
}

extern "C" int exl3_combine_routes(const float* partial, float* out, const void* topk_ids, int ids_dtype, int n_experts,
                                   int64_t tokens, int topk, int64_t n, void* stream)
{
    EXL3_CHECK(tokens >= 0 && topk > 0 && n > 0 && n % 4 == 0, "combine: bad shape");
    EXL3_CHECK(!topk_ids || ids_dtype == EXL3_DTYPE_I64 || ids_dtype == EXL3_DTYPE_I32, "topk_ids must be int64 or int32");
    if (tokens == 0) return EXL3_OK;
    EXL3_CHECK(partial && out, "null pointer");
    EXL3_CHECK(aligned16(partial) && aligned16(out), "partial/out must be 16-byte aligned");
    const int64_t total = tokens * (n / 4);
    const int64_t blocks = (total + 255) / 256;
    combine_routes_kernel<<<(unsigned) (blocks < 65536 ? blocks : 65536), 256, 0, as_stream(stream)>>>(
        reinterpret_cast<const float4*>(partial), reinterpret_cast<float4*>(out), topk_ids, ids_dtype, n_experts,
        tokens, topk, n / 4);
    return hip_status("combine_routes");
}

extern "C" int64_t exl3_smem_bytes(int64_t variant)
{
    if (variant < 0 || variant > 3) return -1;
    return (int64_t) (lds_scatter_bytes<8>() > LDS_MAIN_BYTES ? lds_scatter_bytes<8>() : LDS_MAIN_BYTES);
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
