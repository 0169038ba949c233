/*
 * exl3_grouped.h -- C ABI of the MI355X (gfx950) EXL3 grouped routed-expert MoE prefill library.
 *
 * Every pointer argument is a device pointer (caller-allocated; the library never allocates or frees
 * device memory). fp16 tensors are passed as uint16_t* (IEEE binary16 bit patterns). `stream` is a
 * hipStream_t (NULL = the default stream); work is enqueued there with no host synchronisation. Work runs on
 * the calling thread's current HIP device.
 *
 * Accumulating outputs (grouped GEMM modes 1 and 3, the fat GEMM scatter and its long-K store, the decode op's out)
 * are updated with hardware fp32 atomics (built with -munsafe-fp-atomics): they must be ordinary coarse-grained device
 * allocations (hipMalloc, torch CUDA tensors), not fine-grained or host-coherent memory, where such atomics can be lost.
 *
 * Every entry point validates its arguments before touching the GPU and returns
 *   EXL3_OK (0), EXL3_ERR_ARG (1: bad argument, nothing launched) or EXL3_ERR_HIP (2: launch failed);
 * the message for the last non-zero status of the calling thread is exl3_last_error().
 *
 * Reference file:line citations are relative to the reference repository
 * (siddharth1825/glm53-exl3-prefill); "pybind op" means the torch-extension op the entry point replaces.
 *
 * Trellis tensors: [tiles_k, tiles_n, 16*bits] int16 per matrix (bits in {2,3,4}); a tile holds the 16x16
 * weights W'[16 tk + k][16 tn + n] as 256 bits-wide symbols with a tail-biting 16-bit state window and the
 * MCG codebook: position p's state is stream bits [(p+1)K - 16, (p+1)K) mod 256K of the tile's little-endian dword
 * stream, x = state * 0xCBAC1FED mod 2^32, y = (x & 0x8FFF8FFF) ^ 0x3B603B60, w = fp16(y.lo) + fp16(y.hi), and
 * position p = 8c + j sits at k = 2(c & 3) + (j & 1) + 8((j >> 1) & 1), n = (c >> 2) + 8(j >> 2) (the bit-level
 * restatement is oracle/exl3_oracle.c).
 */
#ifndef EXL3_GROUPED_H
#define EXL3_GROUPED_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXL3_OK 0
#define EXL3_ERR_ARG 1
#define EXL3_ERR_HIP 2

#define EXL3_DTYPE_F32 0
#define EXL3_DTYPE_F16 1
#define EXL3_DTYPE_BF16 2
#define EXL3_DTYPE_I32 3
#define EXL3_DTYPE_I64 4

#define EXL3_LAYOUT_ROWS 0           /* fp16 [rows, width] row-major */
#define EXL3_LAYOUT_T16 1            /* fp16 [ceil(rows/16)*16, width] in 16-row groups: element (r, c) at
                                        (((r/16) * (width/8) + c/8) * 16 + r%16) * 8 + c%8; the grouped GEMM's
                                        activation operand loads are then contiguous */

#define EXL3_GEMM_STORE_F16 0      /* grouped_gemm mode 0: fp16 store into [rows, n_tensors*N] */
#define EXL3_GEMM_SCATTER_F32 1    /* grouped_gemm mode 1: fp32 atomic add into out[token_sorted[r]] * w[r] */
#define EXL3_GEMM_STORE_ROUTE_F32 2 /* grouped_gemm mode 2: fp32 store of w[r] * y[r] into out[route_index[r]] */
#define EXL3_GEMM_ATOMIC_F32 3      /* grouped_gemm mode 3: fp32 atomic add of y[r] into out[r] (split-K gate|up) */
#define EXL3_GEMM_STORE_F16_T16 4   /* grouped_gemm mode 4: mode 0 with out in the T16 layout (what act_had_t16 reads) */

/* Message for the calling thread's last failing call ("" if none). */
const char* exl3_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int exl3_abi_version(void);

/*
 * Route sort: the torch glue of grouped_prefill (kernel/exl3_grouped_runtime.py:59-68) as GPU kernels.
 * Stable sort of the flat route list i = t*topk + j by expert id:
 *   token_sorted[r] = i/topk, weight_sorted[r] = fp16(topk_weights[i]), expert_of_row[r] = topk_ids[i],
 *   route_index[r] = i (optional output, NULL to skip; new, used by the deterministic combine),
 *   counts[e] = #routes of e, expert_row0[e] = exclusive prefix sum of counts.
 * ids_dtype: EXL3_DTYPE_I64 or EXL3_DTYPE_I32; weights_dtype: EXL3_DTYPE_F32, _F16 or _BF16.
 * Routes whose id is outside [0, n_experts) are dropped; the rows they would have filled (the tail past
 * sum(counts)) are written as token 0, weight 0, expert 0, and the number of dropped routes is added to the
 * int32 at workspace offset 0 (read it after the stream completes to detect bad routing).
 * workspace: device scratch of exl3_sort_routes_workspace_bytes(...) bytes; its contents need no initialising.
 */
size_t exl3_sort_routes_workspace_bytes(int64_t tokens, int topk, int n_experts);
int exl3_sort_routes(const void* topk_ids, int ids_dtype, const void* topk_weights, int weights_dtype,
                     int64_t tokens, int topk, int n_experts,
                     int64_t* token_sorted, uint16_t* weight_sorted, int32_t* expert_of_row,
                     int32_t* route_index, int32_t* counts, int32_t* expert_row0,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * Router top-k in front of the sort (new; the glue the reference's path takes as given: GLM-5.3-Flash's noaux_tc
 * router -- sigmoid scores in fp32, selection by score + e_score_correction_bias, top-k, weights from the un-biased
 * scores renormalised to sum 1 (norm_topk_prob) times routed_scaling_factor).
 *   logits [tokens, >= n_experts] (row stride logits_ld elements) fp32 / fp16 / bf16; bias fp32 [n_experts] or NULL.
 *   topk_ids [tokens, topk] int64 or int32, decreasing selection score (ties: lower expert id); topk_weights fp32
 *   [tokens, topk] = s / sum(s) * scale (renorm != 0, sum in selection order) or s * scale.
 * NaN scores are never chosen; when fewer than topk finite scores exist the remaining ids are -1 (dropped by
 * exl3_sort_routes) with weight 0. topk <= 16, n_experts <= 1024.
 */
int exl3_route_topk(const void* logits, int logits_dtype, int64_t logits_ld, const float* bias, int64_t tokens,
                    int n_experts, int topk, int renorm, float scale, void* topk_ids, int ids_dtype,
                    float* topk_weights, void* stream);

/*
 * Block table (pybind op build_blocks, kernel/exl3_grouped_prefill.cu:63-96 and :285-294).
 * counts int32 [n_experts] -> for each 128-row block b of each expert (experts in order):
 *   block_expert[b] = e, block_row0[b] = expert_row0[e] + 128*i; entries b >= n_blocks get block_expert = -1
 *   (block_row0 is not written there); meta = {n_blocks, n_rows}. n_experts <= 1024 ("too many experts").
 */
int exl3_build_blocks(const int32_t* counts, int n_experts, int max_blocks,
                      int32_t* block_expert, int32_t* block_row0, int32_t* meta, void* stream);

/*
 * Row-tile table of `tile_rows` rows per entry (64, 128, 256 or 512): exl3_build_blocks is this with 128. New (no
 * reference counterpart): the grouped GEMM amortises each decoded trellis tile over up to 256 (512) rows of one
 * expert when given a 256-row (512-row) table (max_tiles >= R/tile_rows + n_experts).
 */
int exl3_build_tiles(const int32_t* counts, int n_experts, int tile_rows, int max_tiles,
                     int32_t* tile_expert, int32_t* tile_row0, int32_t* meta, void* stream);
/*
 * Two row-tile tables for one launch pair (new): tile_rows-row tiles (128, 256 or 512), except that each expert's
 * last tile goes to a second table of thin_rows-row tiles (64) when it holds at most thin_rows rows;
 * the grouped GEMM runs the second table on its thin kernel (tile_rows 64, any mode). Tails are -1 as in
 * exl3_build_tiles; meta int32[3] = {full tiles, rows, thin tiles}. Bounds: max_full >= R/tile_rows + n_experts,
 * max_thin >= min(n_experts, R). The same launch also zeroes zero[0 .. zero_floats) (16-byte aligned, a multiple of 4
 * floats; 0 and NULL for none): the fp32 output the down GEMM's atomic scatter adds into.
 */
int exl3_build_tiles_split(const int32_t* counts, int n_experts, int tile_rows, int thin_rows, int max_full,
                           int max_thin, int32_t* full_expert, int32_t* full_row0, int32_t* thin_expert,
                           int32_t* thin_row0, int32_t* meta, float* zero, int64_t zero_floats, void* stream);
/*
 * exl3_sort_routes followed by exl3_build_tiles_split on its counts, in two launches instead of four (new; the torch
 * glue of kernel/exl3_grouped_runtime.py:59-68 and the block table of kernel/exl3_grouped_prefill.cu:63-96 as one
 * prefill-path preparation): the same sorted routes, counts, expert_row0, dropped count (the workspace's first int32),
 * tables, meta and cleared buffer, bit for bit. Arguments and checks are those of the two entry points, and the
 * workspace must be 16-byte aligned.
 */
int exl3_sort_routes_split_tiles(const void* topk_ids, int ids_dtype, const void* topk_weights, int weights_dtype,
                                 int64_t tokens, int topk, int n_experts, int64_t* token_sorted,
                                 uint16_t* weight_sorted, int32_t* expert_of_row, int32_t* route_index,
                                 int32_t* counts, int32_t* expert_row0, void* workspace, size_t workspace_bytes,
                                 int tile_rows, int thin_rows, int max_full, int max_thin, int32_t* full_expert,
                                 int32_t* full_row0, int32_t* thin_expert, int32_t* thin_row0, int32_t* meta,
                                 float* zero, int64_t zero_floats, void* stream);

/*
 * Input Hadamard (pybind op row_had, kernel/exl3_grouped_prefill.cu:101-115 and :296-311):
 *   dst[r, :] = fp16( H128( src[gather ? token_sorted[r] : r, :] * suh[expert_of_row[r], :] ) / sqrt(128) )
 * per 128-column block, fp32 inside. src fp16 [*, K] contiguous, dst fp16 [rows, K] contiguous,
 * suh fp16 rows of length K at stride suh_stride elements (e.g. w13_suh[:, 0] has stride 2K).
 * K % 128 == 0 and suh_len == K ("K must be a multiple of 128 and match suh").
 */
int exl3_row_had(const uint16_t* src, uint16_t* dst, const int64_t* token_sorted, const int32_t* expert_of_row,
                 const uint16_t* suh, int64_t suh_stride, int64_t suh_len, int64_t rows, int K, int gather,
                 void* stream);
/* exl3_row_had with the destination in layout dst_layout (EXL3_LAYOUT_ROWS or EXL3_LAYOUT_T16); expert_of_row may be
 * NULL (every row uses suh row 0: a single linear). New. */
int exl3_row_had_ex(const uint16_t* src, uint16_t* dst, const int64_t* token_sorted, const int32_t* expert_of_row,
                    const uint16_t* suh, int64_t suh_stride, int64_t suh_len, int64_t rows, int K, int gather,
                    int dst_layout, void* stream);

/*
 * Clamped SwiGLU + down Hadamard (pybind op act_had, kernel/exl3_grouped_prefill.cu:118-141 and :313-322):
 *   a = fp16( silu(min(g, limit)) * clamp(u, -limit, limit) ), g = gu[r, :I], u = gu[r, I:]  (fp32 math)
 *   act[r, :] = fp16( H128( a * suh_down[expert_of_row[r], :] ) / sqrt(128) )
 * gu fp16 [rows, gu_width] contiguous with gu_width == 2*I, act fp16 [rows, I], I % 128 == 0.
 */
int exl3_act_had(const uint16_t* gu, int64_t gu_width, uint16_t* act, const int32_t* expert_of_row,
                 const uint16_t* suh_down, int64_t suh_stride, int64_t rows, int I, float limit, void* stream);
/* exl3_act_had with act in layout dst_layout (EXL3_LAYOUT_ROWS or EXL3_LAYOUT_T16); expert_of_row may be NULL (every
 * row uses suh_down row 0). New. */
int exl3_act_had_ex(const uint16_t* gu, int64_t gu_width, uint16_t* act, const int32_t* expert_of_row,
                    const uint16_t* suh_down, int64_t suh_stride, int64_t rows, int I, float limit, int dst_layout,
                    void* stream);
/* exl3_act_had_ex(..., EXL3_LAYOUT_T16) reading gate|up as fp32 partial sums (grouped GEMM mode 3), each rounded to
 * fp16 first -- the reference's fp16 gu -- so the result is what the fp16 gu of the same sums would give. New. */
int exl3_act_had_f32(const float* gu, int64_t gu_width, uint16_t* act, const int32_t* expert_of_row,
                     const uint16_t* suh_down, int64_t suh_stride, int64_t rows, int I, float limit, void* stream);
/* exl3_act_had_ex(..., EXL3_LAYOUT_T16) reading gate|up in the T16 layout too (grouped GEMM mode 4): every load is a
 * contiguous 16-row x 8-column block. Same result as the row-major input. New. */
int exl3_act_had_t16(const uint16_t* gu, int64_t gu_width, uint16_t* act, const int32_t* expert_of_row,
                     const uint16_t* suh_down, int64_t suh_stride, int64_t rows, int I, float limit, void* stream);

/*
 * Grouped weight-stationary trellis GEMM over all experts (pybind op grouped_gemm,
 * kernel/exl3_grouped_prefill.cu:148-279 and :324-378).
 *   a: fp16 [a_rows, size_k] contiguous (rows sorted by expert).
 *   packed_gate / packed_up: trellis of expert e at packed + e*expert_stride_words, laid out
 *     [tiles_k, tiles_n, 16*bits] int16 contiguous; packed_up == NULL for the single-tensor (down) stage.
 *     size_k == 16*tiles_k, size_k % 32 == 0, N_each = 16*tiles_n with N_each % 128 == 0.
 *   svh_gate / svh_up: fp16 rows of N_each at stride svh_stride (svh_up NULL iff packed_up NULL).
 *   block table (build_blocks) with max_blocks entries; counts / expert_row0 int32 [n_experts].
 *   mode EXL3_GEMM_STORE_F16: out fp16 [a_rows, n_tensors*N_each],
 *        out[r, which*N_each + n] = fp16( H128_n(a[r] @ W'_e,which) / sqrt(128) * svh_e,which[n] )
 *   mode EXL3_GEMM_SCATTER_F32 (single tensor only): out fp32 [out_rows, N_each], caller-zeroed,
 *        out[token_sorted[r], n] += fp32(route_weight[r]) * ( H128_n(a[r] @ W'_e) / sqrt(128) * svh_e[n] )
 *        with device-scope fp32 atomics (order of additions is not deterministic).
 *   mode EXL3_GEMM_STORE_ROUTE_F32 (single tensor, new): out fp32 [T*topk, N_each],
 *        out[route_index[r], n] = fp32(route_weight[r]) * ( same ): one row per route, plain stores; with
 *        exl3_combine_routes it gives mode 1's result in a fixed summation order.
 * gate/up tensors must share expert strides (as [E, 2, ...] views do).
 */
int exl3_grouped_gemm(const uint16_t* a, int64_t a_rows, int size_k,
                      const uint16_t* packed_gate, const uint16_t* packed_up, int64_t expert_stride_words,
                      int tiles_k, int tiles_n, int bits,
                      const uint16_t* svh_gate, const uint16_t* svh_up, int64_t svh_stride,
                      const int32_t* block_expert, const int32_t* block_row0, int max_blocks,
                      const int32_t* counts, const int32_t* expert_row0, int n_experts,
                      const int64_t* token_sorted, const uint16_t* route_weight, const int32_t* route_index,
                      void* out, int64_t out_rows, int mode, void* stream);

/*
 * exl3_grouped_gemm with two extensions (new): a_layout (EXL3_LAYOUT_ROWS, or EXL3_LAYOUT_T16 for an `a` written by
 * the _ex Hadamard passes) and tile_rows, the rows per block-table entry (128: the reference's build_blocks table,
 * what exl3_grouped_gemm passes; 256 or 512: a table from exl3_build_tiles(..., 256 | 512, ...); 512-row tiles run
 * an 8-wave kernel; 64: a table from exl3_build_tiles(..., 64, ...) or the thin table of exl3_build_tiles_split, run
 * by a thin kernel with 16 rows per wave). Same modes and outputs.
 */
int exl3_grouped_gemm_ex(const uint16_t* a, int64_t a_rows, int size_k, int a_layout,
                         const uint16_t* packed_gate, const uint16_t* packed_up, int64_t expert_stride_words,
                         int tiles_k, int tiles_n, int bits,
                         const uint16_t* svh_gate, const uint16_t* svh_up, int64_t svh_stride,
                         const int32_t* block_expert, const int32_t* block_row0, int max_blocks, int tile_rows,
                         const int32_t* counts, const int32_t* expert_row0, int n_experts,
                         const int64_t* token_sorted, const uint16_t* route_weight, const int32_t* route_index,
                         void* out, int64_t out_rows, int mode, void* stream);

/*
 * exl3_grouped_gemm_ex with K split into k_split slices of whole 64-column pairs of stages (new; the decode path's
 * launches, which have too few output tiles to fill the GPU otherwise). Each slice runs the full epilogue on its
 * partial product and adds it to the output, so k_split > 1 needs an accumulating mode: EXL3_GEMM_SCATTER_F32, or
 * EXL3_GEMM_ATOMIC_F32 -- out fp32 [a_rows, n_tensors*N_each], caller-zeroed,
 *        out[r, which*N_each + n] += H128_n(a[r] @ W'_e,which) / sqrt(128) * svh_e,which[n]
 * (valid with k_split == 1 too; tile_rows 64, 128 or 256; 64 runs the thin kernel, 16 rows per wave and four
 * workgroups per CU, for small tiles).
 * 1 <= k_split <= size_k / 64; the slice count used is
 * ceil(K_stages / per_slice) with per_slice = ceil(K_stages / k_split) rounded up to even (K_stages = size_k / 32).
 */
int exl3_grouped_gemm_split(const uint16_t* a, int64_t a_rows, int size_k, int a_layout,
                            const uint16_t* packed_gate, const uint16_t* packed_up, int64_t expert_stride_words,
                            int tiles_k, int tiles_n, int bits,
                            const uint16_t* svh_gate, const uint16_t* svh_up, int64_t svh_stride,
                            const int32_t* block_expert, const int32_t* block_row0, int max_blocks, int tile_rows,
                            const int32_t* counts, const int32_t* expert_row0, int n_experts,
                            const int64_t* token_sorted, const uint16_t* route_weight, const int32_t* route_index,
                            void* out, int64_t out_rows, int mode, int k_split, void* stream);
/*
 * exl3_grouped_gemm_split that also clears zero[0 .. zero_floats) (fp32, 16-byte aligned, a multiple of 4 floats;
 * max_blocks > 0) as a side job of the same launch (new): every workgroup stores its grid-strided share of zeros
 * before its tile. The prefill path passes the down scatter's output to its gate|up launch, whose stores then drain
 * under MFMA-bound work instead of holding a launch of their own. zero must not overlap a or out.
 */
int exl3_grouped_gemm_clear(const uint16_t* a, int64_t a_rows, int size_k, int a_layout,
                            const uint16_t* packed_gate, const uint16_t* packed_up, int64_t expert_stride_words,
                            int tiles_k, int tiles_n, int bits, const uint16_t* svh_gate, const uint16_t* svh_up,
                            int64_t svh_stride, const int32_t* block_expert, const int32_t* block_row0, int max_blocks,
                            int tile_rows, const int32_t* counts, const int32_t* expert_row0, int n_experts,
                            const int64_t* token_sorted, const uint16_t* route_weight, const int32_t* route_index,
                            void* out, int64_t out_rows, int mode, int k_split, float* zero, int64_t zero_floats,
                            void* stream);

/*
 * Deterministic route combine (new; pairs with grouped_gemm mode 2): out[t, :] = sum_{j < topk} partial[t*topk + j, :]
 * in order j = 0, 1, ..., skipping routes whose id in topk_ids (optional, int64 or int32 [tokens, topk]) lies outside
 * [0, n_experts). partial fp32 [tokens*topk, n], out fp32 [tokens, n] (overwritten), n % 4 == 0, 1 <= topk <= 32.
 */
int exl3_combine_routes(const float* partial, float* out, const void* topk_ids, int ids_dtype, int n_experts,
                        int64_t tokens, int topk, int64_t n, void* stream);

/*
 * exl3_combine_routes with the sums written in out_dtype (new): EXL3_DTYPE_F32, or EXL3_DTYPE_BF16 / EXL3_DTYPE_F16,
 * each fp32 sum rounded once to nearest even (every NaN -> bf16 0x7FC0) -- bit for bit the fp32 combine followed by
 * the cast the reference's wrapper applies (kernel/exl3_grouped_runtime.py:107, out.to(x.dtype)), without the fp32
 * round trip. out [tokens, n] of that dtype, 16-byte (fp32) or 8-byte aligned.
 */
int exl3_combine_routes_dt(const float* partial, void* out, int out_dtype, const void* topk_ids, int ids_dtype,
                           int n_experts, int64_t tokens, int topk, int64_t n, void* stream);

/*
 * Per-expert weight-stationary trellis GEMM, the exl3_fat_gemm drop-in (pybind ops fat_gemm_v2 /
 * fat_gemm_v2_scatter / smem_bytes, kernel/exl3_fat_gemm_v2.cu:236-333; PR77 signature
 * exl3_fat_gemm(a, packed, out, svh, K, mcg, mul1), kernel/test_fat_v2.py:122,134).
 *   a fp16 [m, size_k]; packed [size_k/16, n/16, 16*bits] int16; svh fp16 [n]; out fp32.
 *   store:   out[m, n]  = H128_n(a @ W') / sqrt(128) * svh          (out [m, n])
 *   scatter: out[token_idx[i], :] += fp32(route_weight[i]) * (same)  (out [out_rows, n], device atomics)
 * bits must be 2, 3 or 4 with mcg != 0 and mul1 == 0 (the reference accepts only bits 4: "only K4 MCG tensors");
 * size_k % 64 == 0, n % 128 == 0. variant in [0, 3] (the reference's four smem/pipeline variants) selects the row-tile
 * schedule: 0 = 64-row tiles (thin kernel), 1 = the shape-tuned policy (64- or 512-row tiles; the reference's
 * production variant), 2 = 256-row tiles, 3 = 512-row tiles (8-wave kernel). exl3_smem_bytes(variant) returns the LDS
 * bytes per workgroup of the kernels that variant launches (the largest, the scatter form's: 33792 for 0 and 2, 67584
 * for 1 and 3), or -1 if unknown. Every variant gives bit-identical results. A store with size_k >= 2048 that would
 * leave CUs idle first zeroes out and then adds two K halves into it with fp32 atomics (exact: two additions onto zero
 * commute), so out must not overlap a, packed or svh.
 */
int exl3_fat_gemm(const uint16_t* a, int64_t m, int size_k, const uint16_t* packed, int tiles_k, int tiles_n,
                  int packed_words, float* out, int64_t out_rows, const uint16_t* svh, int64_t svh_len,
                  int bits, int mcg, int mul1, int variant, void* stream);
int exl3_fat_gemm_scatter(const uint16_t* a, int64_t m, int size_k, const uint16_t* packed, int tiles_k,
                          int tiles_n, int packed_words, float* out, int64_t out_rows, const uint16_t* svh,
                          int64_t svh_len, const int64_t* token_idx, const uint16_t* route_weight,
                          int bits, int mcg, int mul1, int variant, void* stream);
int64_t exl3_smem_bytes(int64_t variant);

/*
 * Dense EXL3 linear (LinearEXL3 forward at M = rows; the dense / shared-expert projection the reference lists next to
 * this path, no kernel of its own there). Same weight convention as the expert GEMMs:
 *   h = fp16( H128(x * suh) / sqrt(128) )                (per 128-column block of K)
 *   y = H128( h . W' ) / sqrt(128) * svh                 (W' = decoded trellis [K, N], fp32 accumulate)
 * x fp16 [m, k] row-major (k % 128 == 0); packed [k/16, n/16, 16*bits] int16 (n % 128 == 0); suh fp16 [k], svh fp16
 * [n]; work: caller-owned scratch of exl3_linear_workspace_bytes(m, k) bytes (h in the T16 layout); out [m, n] fp32
 * (out_dtype EXL3_DTYPE_F32) or fp16 (EXL3_DTYPE_F16). New.
 */
int64_t exl3_linear_workspace_bytes(int64_t m, int k);
int exl3_linear(const uint16_t* x, int64_t m, int k, const uint16_t* packed, int tiles_k, int tiles_n, int bits,
                const uint16_t* suh, const uint16_t* svh, uint16_t* work, void* out, int out_dtype, void* stream);

/*
 * Trellis reconstruct (exllamav3 ext.reconstruct(w, packed, K, mcg, mul1), called by the reference's tests
 * at kernel/test_fat_v2.py:91-94 and harness/proto_fp8.py:70): packed [tiles_k, tiles_n, 16*bits] ->
 * out fp16 [16*tiles_k, 16*tiles_n] row-major (W' in logical [k][n] order).
 */
int exl3_reconstruct(uint16_t* out, const uint16_t* packed, int tiles_k, int tiles_n, int bits, int mcg,
                     int mul1, void* stream);

/*
 * Decode arbitrary 16-bit trellis states with the GEMM's own device decoder: out[i] = fp16 bits of
 * decode(states[i]). No counterpart in the reference; it exists so the decoder can be pinned bit-exactly
 * over all 65536 states. n must be even.
 */
int exl3_decode_states(const uint16_t* states, uint16_t* out, int64_t n, void* stream);

/*
 * Decode-path MoE: the whole routed-expert op for small batches, the `tokens <= cap` side of the reference wrapper's
 * switch (kernel/exl3_grouped_runtime.py:93-98), where the overlay calls exllamav3's fused exl3_moe
 * (kernel/tuned-fused-kernel-patch/exl3patch/exllamav3/exllamav3_ext/quant/exl3_moe.cu:133-345). Same result as
 * the grouped prefill on the same inputs (route sort, gather + H128(x * suh_gate), gate|up, fp16 gu, SwiGLU with limit,
 * H128(act * suh_down), down, scatter by token with the fp16 route weight), with both GEMMs split over K for batches
 * too small to fill the GPU. Graph-capture-safe: a fixed launch sequence for given sizes, no allocation, no memset
 * (fill kernels clear what accumulates), no host reads.
 *   x fp16 [tokens, hidden] row-major; topk_ids [tokens, topk] int64 / int32 (ids outside [0, n_experts) are dropped);
 *   topk_weights [tokens, topk] fp32 / fp16 / bf16 (rounded to fp16).
 *   packed_gate / packed_up: trellis [hidden/16, inter/16, 16*bits] of expert e at + e*w13_expert_stride_words
 *   (the [E, 2, ...] stacked views); suh_gate fp16 [E, hidden] at suh13_stride (gate and up share it);
 *   svh_gate / svh_up fp16 [E, inter] at svh13_stride; packed_down [inter/16, hidden/16, 16*bits] at
 *   w2_expert_stride_words; suh_down fp16 [E, inter] at suh2_stride; svh_down fp16 [E, hidden] at svh2_stride.
 *   out fp32 [tokens, hidden], overwritten (16-byte aligned). workspace: exl3_moe_decode_workspace_bytes(...) bytes,
 *   256-byte aligned, caller-owned. Calls that share a workspace must not overlap. New.
 */
/*
 * The decode path's route preparation in one launch (new): for tokens*topk <= 2048 routes, the stable sort of
 * exl3_sort_routes (same token_sorted / weight_sorted / expert_of_row / counts / expert_row0, no route_index, no
 * workspace) and the tile table of exl3_build_tiles(counts, n_experts, tile_rows, max_tiles, ...) including meta,
 * plus a zero fill of two optional fp32 buffers (16-byte aligned, lengths multiples of 4 floats).
 */
int exl3_route_prep_small(const void* topk_ids, int ids_dtype, const void* topk_weights, int weights_dtype,
                          int64_t tokens, int topk, int n_experts, int tile_rows, int max_tiles,
                          int64_t* token_sorted, uint16_t* weight_sorted, int32_t* expert_of_row, int32_t* counts,
                          int32_t* expert_row0, int32_t* tile_expert, int32_t* tile_row0, int32_t* meta,
                          float* zero_a, int64_t zero_a_floats, float* zero_b, int64_t zero_b_floats, void* stream);

int64_t exl3_moe_decode_workspace_bytes(int64_t tokens, int topk, int n_experts, int hidden, int inter);
int exl3_moe_decode(const uint16_t* x, int64_t tokens, int hidden, const void* topk_ids, int ids_dtype,
                    const void* topk_weights, int weights_dtype, int topk, int n_experts, int inter, int bits,
                    const uint16_t* packed_gate, const uint16_t* packed_up, int64_t w13_expert_stride_words,
                    const uint16_t* suh_gate, int64_t suh13_stride, const uint16_t* svh_gate, const uint16_t* svh_up,
                    int64_t svh13_stride, const uint16_t* packed_down, int64_t w2_expert_stride_words,
                    const uint16_t* suh_down, int64_t suh2_stride, const uint16_t* svh_down, int64_t svh2_stride,
                    float limit, float* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * exl3_moe_decode without a workspace argument: the workspace is a fixed 32 MiB scratch array in device memory that
 * the library holds on every GPU it runs on until the process ends, so the call allocates nothing. No counterpart in
 * the reference; it is for callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Limit: calls whose exl3_moe_decode_workspace_bytes(tokens, topk, n_experts, hidden, inter)
 * exceeds 32 MiB are rejected with EXL3_ERR_ARG (256 tokens x top-8 at hidden 4096, inter 768 fit). Every call on one
 * GPU shares that GPU's scratch: calls that overlap on one GPU (concurrent streams or threads) race and must not be
 * issued. Same arguments, result and graph-capture safety as exl3_moe_decode otherwise.
 */
int exl3_moe_decode_noalloc(const uint16_t* x, int64_t tokens, int hidden, const void* topk_ids, int ids_dtype,
                            const void* topk_weights, int weights_dtype, int topk, int n_experts, int inter, int bits,
                            const uint16_t* packed_gate, const uint16_t* packed_up, int64_t w13_expert_stride_words,
                            const uint16_t* suh_gate, int64_t suh13_stride, const uint16_t* svh_gate,
                            const uint16_t* svh_up, int64_t svh13_stride, const uint16_t* packed_down,
                            int64_t w2_expert_stride_words, const uint16_t* suh_down, int64_t suh2_stride,
                            const uint16_t* svh_down, int64_t svh2_stride, float limit, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_GROUPED_H */
