// Trellis tile decode for gfx950.
//
// A 16x16 tile is 256 positions; position p's 16-bit state is the window of stream bits
// [(p+1)K - 16, (p+1)K) (mod 256K) of the tile's little-endian dword stream, its first bit as bit 0.
// decode(state): x = state * 0xCBAC1FED mod 2^32; y = (x & 0x8FFF8FFF) ^ 0x3B603B60;
//                w = fp16(y.lo16) + fp16(y.hi16)  (one fp16 add).
// A lane decodes one chunk: the 8 positions p = 8c + j (c = chunk 0..31, j = 0..7), which sit at tile rows
// k = 2(c & 3) + (j & 1) + 8((j >> 1) & 1) and columns n = (c >> 2) + 8(j >> 2).
//
// gfx950 cost per weight: the 32-bit multiply by a 16-bit state is split into a 16x16 low-half multiply whose
// result lands in the upper word (SDWA) plus a 16x16+32 multiply-add that picks the state's half by op_sel,
// so no state ever needs shifting out of its dword; v_bitop3 does mask-and-xor in one op, and SDWA fp16 adds write
// each sum into its half of the packed output pair in place. About 4.4 VALU ops per weight at 4 bits.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace exl3 {

constexpr uint32_t MCG_MUL_LO = 0x1FEDu;       // low 16 bits of 0xCBAC1FED
constexpr uint32_t MCG_MUL_HI = 0xCBACu;       // high 16 bits
constexpr uint32_t MCG_XOR = 0x3B603B60u;
constexpr uint32_t MCG_MASK = 0x8FFF8FFFu;

// gfx950 forwards a VALU result written through an SDWA destination select (a partial-register write) to the
// next instruction stale: the consumer must be at least one instruction later. The compiler's hazard recognizer
// cannot see inside an asm statement, so every SDWA result below is consumed only by a VALU instruction of the same
// asm block at least one instruction later, and a block whose last writes are SDWA ends with an s_nop, so whatever the
// compiler places after the block reads them at least one wait state later. Inputs of these blocks must likewise not come
// from instructions with wait-state rules of their own (per-lane 64-bit shifts fed into them gave wrong results at
// random): callers hand them 32-bit funnel shifts, loads and DPP moves.

// x0 = (SEL0 ? hi : lo)(ra) * 0xCBAC1FED, x1 = (SEL1 ? hi : lo)(rb) * 0xCBAC1FED  (mod 2^32), as full 32-bit products.
#define EXL3_MCG_MUL2(S0, S1, OP0, OP1)                                                                               \
    asm("v_mul_lo_u16_sdwa %0, %4, %6 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:" S0 " src1_sel:DWORD\n\t"       \
        "v_mul_lo_u16_sdwa %1, %5, %6 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:" S1 " src1_sel:DWORD\n\t"       \
        "v_mad_u32_u16 %2, %4, %7, %0" OP0 "\n\t"                                                                    \
        "v_mad_u32_u16 %3, %5, %7, %1" OP1                                                                          \
        : "=&v"(t0), "=&v"(t1), "=&v"(x0), "=&v"(x1) : "v"(ra), "v"(rb), "s"(chi), "s"(clo))
template <int SEL0, int SEL1>
__device__ __forceinline__ void mcg_mul2(uint32_t ra, uint32_t rb, uint32_t& x0, uint32_t& x1)
{
    uint32_t t0, t1;
    const uint32_t chi = MCG_MUL_HI, clo = MCG_MUL_LO;
    if constexpr (!SEL0 && !SEL1) EXL3_MCG_MUL2("WORD_0", "WORD_0", "", "");
    else if constexpr (!SEL0 && SEL1) EXL3_MCG_MUL2("WORD_0", "WORD_1", "", " op_sel:[1,0,0,0]");
    else if constexpr (SEL0 && !SEL1) EXL3_MCG_MUL2("WORD_1", "WORD_0", " op_sel:[1,0,0,0]", "");
    else EXL3_MCG_MUL2("WORD_1", "WORD_1", " op_sel:[1,0,0,0]", " op_sel:[1,0,0,0]");
}
#undef EXL3_MCG_MUL2

__device__ __forceinline__ uint32_t mcg_mask(uint32_t x) { return (x & MCG_MASK) ^ MCG_XOR; }

// Two packed fp16 pairs: w0 = {fp16(ya.lo + ya.hi), fp16(yb.lo + yb.hi)}, w1 = {same for yc, yd}. The low halves are
// written first (upper half zeroed), then the high halves with the low ones preserved -- each read-modify-write two
// instructions after the write it reads -- and an s_nop guards the last partial write.
__device__ __forceinline__ void add_halves_2pairs(uint32_t ya, uint32_t yb, uint32_t yc, uint32_t yd,
                                                  uint32_t& w0, uint32_t& w1)
{
    asm("v_add_f16_sdwa %0, %2, %2 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "v_add_f16_sdwa %1, %4, %4 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "v_add_f16_sdwa %0, %3, %3 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "v_add_f16_sdwa %1, %5, %5 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "s_nop 1"
        : "=&v"(w0), "=&v"(w1) : "v"(ya), "v"(yb), "v"(yc), "v"(yd));
}

// Decoded chunk, as four packed fp16 pairs ordered for a [n][k] (k-contiguous) destination:
//   out[0] = (k0, k0+1) at column n0, out[1] = (k0+8, k0+9) at n0, out[2] = (k0, k0+1) at n0+8,
//   out[3] = (k0+8, k0+9) at n0+8, with k0 = 2(c & 3), n0 = c >> 2.
struct Chunk4 { uint32_t w[4]; };

// Per-lane constants locating chunk c's bits: the two dwords (lo, hi) holding them and the bit offset of the
// window of position 8c inside the 64-bit value hi:lo.
struct ChunkLoc { int dlo, dhi, off; };

template <int BITS>
__device__ __forceinline__ ChunkLoc chunk_loc(int c)
{
    constexpr int NDW = 8 * BITS;                          // dwords per tile
    const int b0 = 8 * c * BITS + BITS - 16;               // first stream bit of position 8c's window
    const int d0 = (b0 >= 0) ? (b0 >> 5) : -1;            // floor(b0 / 32), b0 >= -15
    ChunkLoc L;
    L.off = b0 - 32 * d0;
    L.dlo = (d0 + NDW) % NDW;
    L.dhi = (d0 + 1) % NDW;
    return L;
}

// Decode the chunk whose stream bits sit in hi:lo starting at bit `off` (BITS in {1,2,3,4}).
template <int BITS>
__device__ __forceinline__ Chunk4 decode_chunk(uint32_t lo, uint32_t hi, int off)
{
    uint32_t x[8];
    if constexpr (BITS == 4)
    {
        // off == 20 for every chunk: states j and j+4 are the low/high halves of one shifted dword
        const uint32_t r0 = hi;                                      // states 3, 7
        const uint32_t r1 = __builtin_amdgcn_alignbit(hi, lo, 20);   // states 0, 4
        const uint32_t r2 = __builtin_amdgcn_alignbit(hi, lo, 24);   // states 1, 5
        const uint32_t r3 = __builtin_amdgcn_alignbit(hi, lo, 28);   // states 2, 6
        mcg_mul2<0, 1>(r1, r1, x[0], x[4]);
        mcg_mul2<0, 1>(r2, r2, x[1], x[5]);
        mcg_mul2<0, 1>(r3, r3, x[2], x[6]);
        mcg_mul2<0, 1>(r0, r0, x[3], x[7]);
    }
    else
    {
        const uint64_t q = ((uint64_t) hi << 32) | lo;
        uint32_t r[8];
        #pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = (uint32_t) (q >> (off + j * BITS));
        #pragma unroll
        for (int j = 0; j < 8; j += 2) mcg_mul2<0, 0>(r[j], r[j + 1], x[j], x[j + 1]);
    }
    uint32_t y[8];
    #pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = mcg_mask(x[j]);
    Chunk4 c;
    add_halves_2pairs(y[0], y[1], y[2], y[3], c.w[0], c.w[1]);
    add_halves_2pairs(y[4], y[5], y[6], y[7], c.w[2], c.w[3]);
    return c;
}

// Decode four independent states (low and high halves of ra and rb) -> packed fp16 pairs (wa for ra, wb for rb).
__device__ __forceinline__ void decode_state_pairs(uint32_t ra, uint32_t rb, uint32_t& wa, uint32_t& wb)
{
    uint32_t x0, x1, x2, x3;
    mcg_mul2<0, 1>(ra, ra, x0, x1);
    mcg_mul2<0, 1>(rb, rb, x2, x3);
    add_halves_2pairs(mcg_mask(x0), mcg_mask(x1), mcg_mask(x2), mcg_mask(x3), wa, wb);
}

}  // namespace exl3
