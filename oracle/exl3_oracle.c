/*
 * exl3_oracle.c -- CPU restatement of the integer / bit-level half of the EXL3 grouped MoE prefill path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the parity tests, __graft_entry__.smoke() and the
 * bench's cpu_baseline leg compare the HIP kernels against. Nothing in the product path links, loads or
 * calls it; the product fails loudly when its HIP library is missing.
 *
 * What is restated here, and from where (paths relative to the reference repository):
 *   - route sort (stable argsort by expert, token/weight/expert arrays, counts, exclusive offsets):
 *       kernel/exl3_grouped_runtime.py:59-68
 *   - per-expert 128-row block table (block_expert, block_row0, meta, -1 tail):
 *       kernel/exl3_grouped_prefill.cu:63-96
 *   - trellis tile decode (16x16 tiles of 16*K uint16 words, tail-biting 16-bit state window, MCG codebook,
 *     fp16 sum of the two halves) and its position -> (k, n) permutation. The reference calls this through
 *     exllamav3's dq_dispatch<4,1> (kernel/exl3_grouped_prefill.cu:237) and reconstruct
 *     (kernel/test_fat_v2.py:91-94); exllamav3 @ c5d9c657 is not vendored, so the bit order within the
 *     stream is this build's own written spec (stated below).  -> parity unpinned against exllamav3.
 *     The reference's exllamav3 overlay (kernel/tuned-fused-kernel-patch/exl3patch/exllamav3/exllamav3_ext/
 *     quant/exl3_gemm_inner.cuh:9,280) includes exl3_dq.cuh and calls dq_dispatch<bits, cb>(shb, lane_id << 3,
 *     ...), which fixes the eight consecutive positions per lane used below; exl3_dq.cuh itself, where the
 *     codebook constants and the window extraction live, is not part of the overlay.
 *   - IEEE fp16 <-> fp32 conversion with round-to-nearest-even (the __float2half of the reference's stores).
 *
 * Trellis spec (K = bits per weight, 1 <= K <= 8; the kernels support K in {2, 3, 4}):
 *   tile words w[0 .. 16K) (uint16), read as little-endian dwords D[d] = w[2d] | w[2d+1] << 16.
 *   stream bit b (0 <= b < 256K) = bit (b mod 32) of D[b / 32].
 *   state of position p (0..255) = stream bits [(p+1)K - 16, (p+1)K) modulo 256K, the first of them as
 *   bit 0 of the state (tail-biting: positions p < 16/K - 1 reach into the end of the stream).
 *   decode(state): x = state * 0xCBAC1FED (mod 2^32); y = (x & 0x8FFF8FFF) ^ 0x3B603B60;
 *                  value = fp16( fp16(y & 0xFFFF) + fp16(y >> 16) )   (one fp16 add, round to nearest even)
 *   position p = 8l + j (l = 0..31, j = 0..7) sits at tile row k = 2(l mod 4) + (j & 1) + 8((j >> 1) & 1),
 *   tile column n = l / 4 + 8 (j >> 2).
 *   packed tensor [tiles_k, tiles_n, 16K], tile (tk, tn) holds W'[16tk + k][16tn + n].
 */
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#include <math.h>

/* ------------------------------------------------------------------------------------------ fp16 */

float orc_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t) (h >> 15) << 31;
    const uint32_t exp = (h >> 10) & 0x1F;
    uint32_t mant = h & 0x3FF;
    uint32_t bits;
    if (exp == 0)
    {
        if (mant == 0) bits = sign;
        else
        {   /* subnormal: value = mant * 2^-24, normalise */
            int e = -1;
            do { mant <<= 1; ++e; } while ((mant & 0x400) == 0);
            mant &= 0x3FF;
            bits = sign | ((uint32_t) (127 - 15 - e) << 23) | (mant << 13);
        }
    }
    else if (exp == 31) bits = sign | 0x7F800000u | (mant << 13);
    else bits = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t) ((x >> 16) & 0x8000);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u)                                   /* inf / nan */
        return sign | (ax > 0x7F800000u ? (uint16_t) (0x7E00 | ((ax >> 13) & 0x3FF)) : 0x7C00);
    if (ax >= 0x477FF000u) return sign | 0x7C00;             /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u)
    {   /* result is subnormal or zero: value / 2^-24, round to nearest even */
        if (ax < 0x33000000u) return sign;                   /* < 2^-25 rounds to 0 (2^-25 itself ties to 0) */
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7FFFFF) | 0x800000;
        const int shift = 126 - (int) e;                     /* value = m * 2^(e-150); want m * 2^(e-150+24) */
        const uint32_t q = m >> (shift);
        const uint32_t rem = m & ((1u << shift) - 1);
        const uint32_t halfway = 1u << (shift - 1);
        uint32_t r = q + ((rem > halfway) || (rem == halfway && (q & 1)));
        return sign | (uint16_t) r;
    }
    /* normal */
    uint32_t mant = ax & 0x7FFFFF;
    uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t q = (e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFF;
    if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) q += 1;   /* carry may bump the exponent: correct */
    return sign | (uint16_t) q;
}

void orc_f32_to_f16_array(const float* in, uint16_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(in[i]);
}

void orc_f16_to_f32_array(const uint16_t* in, float* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------------------------ trellis */

uint16_t orc_decode_state_mcg(uint32_t state)
{
    uint32_t x = (state & 0xFFFFu) * 0xCBAC1FEDu;
    x = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
    const float lo = orc_f16_to_f32((uint16_t) (x & 0xFFFF));
    const float hi = orc_f16_to_f32((uint16_t) (x >> 16));
    /* both halves have |v| in [1/8, 2): their fp32 sum is exact, so rounding it once to fp16 equals
       a native fp16 add */
    return orc_f32_to_f16(lo + hi);
}

void orc_decode_lut(uint16_t* out)
{
    for (uint32_t s = 0; s < 65536; ++s) out[s] = orc_decode_state_mcg(s);
}

static inline uint32_t stream_bit(const uint16_t* w, int bits, int64_t b)
{
    const int64_t len = 256 * (int64_t) bits;
    b %= len;
    if (b < 0) b += len;
    const uint32_t d = (uint32_t) w[2 * (b / 32)] | ((uint32_t) w[2 * (b / 32) + 1] << 16);
    return (d >> (b % 32)) & 1u;
}

/* 256 states of one tile, bit by bit straight from the spec */
void orc_tile_states(const uint16_t* words, int bits, uint16_t* states)
{
    for (int p = 0; p < 256; ++p)
    {
        const int64_t start = (int64_t) (p + 1) * bits - 16;
        uint32_t s = 0;
        for (int i = 0; i < 16; ++i) s |= stream_bit(words, bits, start + i) << i;
        states[p] = (uint16_t) s;
    }
}

/* Same states through a 64-bit window of two consecutive dwords (the stream length is a whole number of dwords,
   so a window that wraps past the end reads dwords NDW-1 and 0). Checked against orc_tile_states. */
void orc_tile_states_fast(const uint16_t* words, int bits, uint16_t* states)
{
    const int ndw = 8 * bits;
    const int64_t len = 256 * (int64_t) bits;
    for (int p = 0; p < 256; ++p)
    {
        int64_t s = ((int64_t) (p + 1) * bits - 16) % len;
        if (s < 0) s += len;
        const int d = (int) (s / 32);
        const int d1 = (d + 1) % ndw;
        const uint64_t lo = (uint64_t) words[2 * d] | ((uint64_t) words[2 * d + 1] << 16);
        const uint64_t hi = (uint64_t) words[2 * d1] | ((uint64_t) words[2 * d1 + 1] << 16);
        states[p] = (uint16_t) ((((hi << 32) | lo) >> (s % 32)) & 0xFFFF);
    }
}

void orc_tile_pos_to_kn(int p, int* k, int* n)
{
    const int l = p >> 3, j = p & 7;
    *k = 2 * (l & 3) + (j & 1) + 8 * ((j >> 1) & 1);
    *n = (l >> 2) + 8 * (j >> 2);
}

/* pack 256 K-bit symbols (symbol p = the top K bits of state p) into 16K uint16 words */
void orc_pack_tile(const uint8_t* symbols, int bits, uint16_t* words)
{
    const int nwords = 16 * bits;
    memset(words, 0, sizeof(uint16_t) * nwords);
    for (int p = 0; p < 256; ++p)
        for (int i = 0; i < bits; ++i)
        {
            const int b = p * bits + i;
            if ((symbols[p] >> i) & 1) words[b / 16] |= (uint16_t) (1u << (b % 16));
        }
}

/* packed [tiles_k, tiles_n, 16*bits] -> W' fp16 [tiles_k*16, tiles_n*16] row-major */
void orc_reconstruct(const uint16_t* packed, int tiles_k, int tiles_n, int bits, uint16_t* out)
{
    static uint16_t lut[65536];
    static int lut_ready = 0;
    if (!lut_ready) { orc_decode_lut(lut); lut_ready = 1; }
    const int nwords = 16 * bits;
    const int64_t ncols = (int64_t) tiles_n * 16;
    #pragma omp parallel for schedule(static)
    for (int tk = 0; tk < tiles_k; ++tk)
        for (int tn = 0; tn < tiles_n; ++tn)
        {
            uint16_t states[256];
            orc_tile_states_fast(packed + ((int64_t) tk * tiles_n + tn) * nwords, bits, states);
            for (int p = 0; p < 256; ++p)
            {
                int k, n;
                orc_tile_pos_to_kn(p, &k, &n);
                out[(int64_t) (tk * 16 + k) * ncols + tn * 16 + n] = lut[states[p]];
            }
        }
}

/* ------------------------------------------------------------------------------------------ routing */

/* Stable counting sort of the flat route list (index i = t*topk + j) by expert id.
   Restates kernel/exl3_grouped_runtime.py:59-68: order = argsort(ids.flatten(), stable=True),
   token_sorted = (i / topk)[order], weight_sorted = fp16(weights.flatten()[order]),
   expert_of_row = ids.flatten()[order], counts = bincount, expert_row0 = exclusive cumsum.
   Returns 0, or -1 if an id is outside [0, E). */
int orc_sort_routes(const int64_t* ids, const float* weights, int64_t T, int topk, int E,
                    int64_t* token_sorted, uint16_t* weight_sorted, int32_t* expert_of_row,
                    int32_t* counts, int32_t* expert_row0)
{
    const int64_t R = T * topk;
    memset(counts, 0, sizeof(int32_t) * E);
    for (int64_t i = 0; i < R; ++i)
    {
        if (ids[i] < 0 || ids[i] >= E) return -1;
        counts[ids[i]]++;
    }
    int64_t* cursor = (int64_t*) malloc(sizeof(int64_t) * (E > 0 ? E : 1));
    int64_t run = 0;
    for (int e = 0; e < E; ++e) { expert_row0[e] = (int32_t) run; cursor[e] = run; run += counts[e]; }
    for (int64_t i = 0; i < R; ++i)
    {
        const int64_t row = cursor[ids[i]]++;
        token_sorted[row] = i / topk;
        weight_sorted[row] = orc_f32_to_f16(weights[i]);
        expert_of_row[row] = (int32_t) ids[i];
    }
    free(cursor);
    return 0;
}

/* Restates kernel/exl3_grouped_prefill.cu:63-96 (TILE_M = 128 there; tile_rows here): block b of expert e covers
   sorted rows [expert_row0[e] + tile_rows i, ...). Entries b >= n_blocks get block_expert = -1; block_row0 there is
   left untouched (the reference never writes it). meta = {n_blocks, n_rows}. */
void orc_build_tiles(const int32_t* counts, int E, int tile_rows, int max_blocks, int32_t* block_expert,
                     int32_t* block_row0, int32_t* meta)
{
    int64_t row = 0, blk = 0;
    for (int e = 0; e < E; ++e)
    {
        const int nblk = (counts[e] + tile_rows - 1) / tile_rows;
        for (int i = 0; i < nblk; ++i)
        {
            const int64_t b = blk + i;
            if (b < max_blocks) { block_expert[b] = e; block_row0[b] = (int32_t) (row + (int64_t) tile_rows * i); }
        }
        row += counts[e];
        blk += nblk;
    }
    meta[0] = (int32_t) blk;
    meta[1] = (int32_t) row;
    for (int64_t b = blk; b < max_blocks; ++b) block_expert[b] = -1;
}

void orc_build_blocks(const int32_t* counts, int E, int max_blocks, int32_t* block_expert, int32_t* block_row0,
                      int32_t* meta)
{
    orc_build_tiles(counts, E, 128, max_blocks, block_expert, block_row0, meta);
}
