"""Torch-facing operators with the reference extension's names, argument order and error behaviour.

Reference ops (paths relative to the reference repository):
  build_blocks, row_had, act_had, grouped_gemm   kernel/exl3_grouped_prefill.cu:283-386 (pybind module)
  fat_gemm_v2, fat_gemm_v2_scatter, smem_bytes   kernel/exl3_fat_gemm_v2.cu:298-333
  reconstruct                                     exllamav3 ext.reconstruct, called at kernel/test_fat_v2.py:91-94
New ops (no reference counterpart): route_topk (the router top-k), linear_exl3 (the dense EXL3 linear), sort_routes (the torch glue of
kernel/exl3_grouped_runtime.py:59-68 as a GPU counting sort) and decode_states (pins the device trellis decoder).

Each op checks dtypes / shapes / strides on the host first (a bad call raises RuntimeError, like the
reference's TORCH_CHECK, before anything touches a GPU), then enqueues HIP kernels on the current stream of
the tensors' device through the C ABI. Nothing here allocates device memory except sort_routes' optional
workspace.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

_DT = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16,
       torch.int32: _lib.DTYPE_I32, torch.int64: _lib.DTYPE_I64}


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _p(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _require_cuda(*ts) -> torch.device:
    for t in ts:
        if t is not None:
            _check(t.is_cuda, "tensors must be CUDA")
    dev = next(t for t in ts if t is not None).device
    for t in ts:
        if t is not None:
            _check(t.device == dev, "tensors must be on the same device")
    return dev


class _On:
    """Device guard + current stream handle for one op call."""

    def __init__(self, dev: torch.device):
        self.dev = dev

    def __enter__(self):
        self.guard = torch.cuda.device(self.dev)
        self.guard.__enter__()
        return ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)

    def __exit__(self, *exc):
        self.guard.__exit__(*exc)
        return False


# ------------------------------------------------------------------------------------------- routing
def sort_routes_workspace_bytes(tokens: int, topk: int, n_experts: int) -> int:
    return int(_lib.load().exl3_sort_routes_workspace_bytes(tokens, topk, n_experts))


def sort_routes(topk_ids: torch.Tensor, topk_weights: torch.Tensor, n_experts: int, token_sorted: torch.Tensor,
                weight_sorted: torch.Tensor, expert_of_row: torch.Tensor, counts: torch.Tensor,
                expert_row0: torch.Tensor, workspace: Optional[torch.Tensor] = None,
                route_index: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Stable sort of routes by expert (replaces kernel/exl3_grouped_runtime.py:59-68). Returns the workspace;
    its first int32 holds the number of dropped routes (ids outside [0, n_experts)). route_index (int32 [R],
    optional) receives each sorted row's flat route index t*topk + j."""
    _check(topk_ids.dim() == 2 and topk_weights.shape == topk_ids.shape, "topk_ids / topk_weights must be [T, topk]")
    _check(topk_ids.dtype in (torch.int64, torch.int32), "topk_ids must be int64 or int32")
    _check(topk_weights.dtype in (torch.float32, torch.float16, torch.bfloat16),
           "topk_weights must be float32, float16 or bfloat16")
    _check(topk_ids.is_contiguous() and topk_weights.is_contiguous(), "routing tensors must be contiguous")
    T, k = topk_ids.shape
    R = T * k
    _check(token_sorted.dtype == torch.int64 and weight_sorted.dtype == torch.float16 and
           expert_of_row.dtype == torch.int32, "sorted outputs: int64 tokens, fp16 weights, int32 experts")
    _check(token_sorted.numel() == R and weight_sorted.numel() == R and expert_of_row.numel() == R,
           "sorted outputs must have T*topk elements")
    _check(counts.dtype == torch.int32 and expert_row0.dtype == torch.int32 and counts.numel() == n_experts and
           expert_row0.numel() == n_experts, "counts / expert_row0 must be int32 [E]")
    _check(0 < n_experts <= 1024, "too many experts")
    if route_index is not None:
        _check(route_index.dtype == torch.int32 and route_index.numel() == R and route_index.is_contiguous(),
               "route_index must be contiguous int32 [T*topk]")
    need = sort_routes_workspace_bytes(T, k, n_experts)
    dev = _require_cuda(topk_ids, topk_weights, token_sorted, weight_sorted, expert_of_row, counts, expert_row0)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    _check(workspace.numel() * workspace.element_size() >= need, "sort workspace too small")
    with _On(dev) as s:
        _lib.call("exl3_sort_routes", _p(topk_ids), _DT[topk_ids.dtype], _p(topk_weights), _DT[topk_weights.dtype],
                  T, k, n_experts, _p(token_sorted), _p(weight_sorted), _p(expert_of_row), _p(route_index),
                  _p(counts), _p(expert_row0), _p(workspace), workspace.numel() * workspace.element_size(), s)
    return workspace


def route_topk(logits: torch.Tensor, e_score_correction_bias: Optional[torch.Tensor] = None, topk: int = 8,
               routed_scaling_factor: float = 2.5, renormalize: bool = True,
               ids_dtype: torch.dtype = torch.int64) -> tuple[torch.Tensor, torch.Tensor]:
    """Router top-k feeding sort_routes (new; GLM-5.3-Flash's noaux_tc router): sigmoid scores in fp32, selection by
    score + bias, top-k in decreasing order (ties: lower expert id), weights = un-biased scores renormalised to sum 1
    (renormalize) times routed_scaling_factor. logits [T, E] fp32/fp16/bf16 (rows may be strided); returns
    (topk_ids [T, topk] ids_dtype, topk_weights [T, topk] fp32)."""
    _check(logits.dim() == 2 and logits.dtype in (torch.float32, torch.float16, torch.bfloat16), "logits must be [T, E]")
    _check(logits.stride(1) == 1 or logits.size(0) == 0, "logits rows must be contiguous")
    T, E = logits.shape
    _check(0 < E <= 1024, "too many experts")
    _check(0 < int(topk) <= min(16, E), "topk must be in [1, min(16, n_experts)]")
    _check(ids_dtype in (torch.int64, torch.int32), "topk_ids must be int64 or int32")
    if e_score_correction_bias is not None:
        _check(e_score_correction_bias.dtype == torch.float32 and e_score_correction_bias.is_contiguous()
               and e_score_correction_bias.numel() == E, "bias must be contiguous fp32 [E]")
    ids = torch.empty(T, int(topk), dtype=ids_dtype, device=logits.device)
    weights = torch.empty(T, int(topk), dtype=torch.float32, device=logits.device)
    if T == 0:
        return ids, weights
    dev = _require_cuda(logits, ids, weights, *([e_score_correction_bias] if e_score_correction_bias is not None else []))
    with _On(dev) as s:
        _lib.call("exl3_route_topk", _p(logits), _DT[logits.dtype], logits.stride(0), _p(e_score_correction_bias), T, E,
                  int(topk), int(bool(renormalize)), float(routed_scaling_factor), _p(ids), _DT[ids_dtype], _p(weights),
                  s)
    return ids, weights


def build_blocks(counts: torch.Tensor, block_expert: torch.Tensor, block_row0: torch.Tensor, meta: torch.Tensor) -> None:
    """kernel/exl3_grouped_prefill.cu:285-294 (128-row blocks)."""
    build_tiles(counts, block_expert, block_row0, meta, 128)


def build_tiles(counts: torch.Tensor, tile_expert: torch.Tensor, tile_row0: torch.Tensor, meta: torch.Tensor,
                tile_rows: int) -> None:
    """build_blocks with `tile_rows` (64, 128, 256 or 512) rows per entry (new; 256- and 512-row tables feed
    grouped_gemm's tile_rows=256 / 512 schedules)."""
    _check(counts.dtype == torch.int32 and tile_expert.dtype == torch.int32 and tile_row0.dtype == torch.int32
           and meta.dtype == torch.int32, "int32 tensors")
    _check(counts.numel() <= 1024, "too many experts")
    _check(int(tile_rows) in (64, 128, 256, 512), "tile_rows must be 64, 128, 256 or 512")
    _check(tile_row0.numel() >= tile_expert.numel() and meta.numel() >= 2, "block table shapes")
    _check(counts.is_contiguous() and tile_expert.is_contiguous() and tile_row0.is_contiguous()
           and meta.is_contiguous(), "contiguous tensors")
    dev = _require_cuda(counts, tile_expert, tile_row0, meta)
    with _On(dev) as s:
        _lib.call("exl3_build_tiles", _p(counts), counts.numel(), int(tile_rows), tile_expert.numel(),
                  _p(tile_expert), _p(tile_row0), _p(meta), s)


# ------------------------------------------------------------------------------------------- Hadamard passes
def build_tiles_split(counts: torch.Tensor, full_expert: torch.Tensor, full_row0: torch.Tensor,
                      thin_expert: torch.Tensor, thin_row0: torch.Tensor, meta: torch.Tensor, tile_rows: int = 256,
                      thin_rows: int = 64, zero: Optional[torch.Tensor] = None) -> None:
    """Two tile tables (new): `tile_rows`-row tiles with each expert's small last tile (<= thin_rows rows) moved to a
    `thin_rows`-row table for the grouped GEMM's thin kernel. meta int32[3] = {full tiles, rows, thin tiles}.
    zero (optional, fp32 contiguous, numel % 4 == 0): cleared by the same launch (the down scatter's output)."""
    for t in (counts, full_expert, full_row0, thin_expert, thin_row0, meta):
        _check(t.dtype == torch.int32 and t.is_contiguous(), "int32 contiguous tensors")
    _check(full_row0.numel() >= full_expert.numel() and thin_row0.numel() >= thin_expert.numel() and
           meta.numel() >= 3, "tables: row0 at least as long as expert, meta int32[3]")
    _check(zero is None or (zero.dtype == torch.float32 and zero.is_contiguous() and zero.numel() % 4 == 0),
           "zero must be fp32 contiguous with a multiple of 4 elements")
    tensors = (counts, full_expert, full_row0, thin_expert, thin_row0, meta) + ((zero,) if zero is not None else ())
    dev = _require_cuda(*tensors)
    with _On(dev) as s:
        _lib.call("exl3_build_tiles_split", _p(counts), counts.numel(), int(tile_rows), int(thin_rows),
                  full_expert.numel(), thin_expert.numel(), _p(full_expert), _p(full_row0), _p(thin_expert),
                  _p(thin_row0), _p(meta), _p(zero) if zero is not None else None,
                  zero.numel() if zero is not None else 0, s)


def sort_routes_split_tiles(topk_ids: torch.Tensor, topk_weights: torch.Tensor, n_experts: int,
                            token_sorted: torch.Tensor, weight_sorted: torch.Tensor, expert_of_row: torch.Tensor,
                            counts: torch.Tensor, expert_row0: torch.Tensor, full_expert: torch.Tensor,
                            full_row0: torch.Tensor, thin_expert: torch.Tensor, thin_row0: torch.Tensor,
                            meta: torch.Tensor, tile_rows: int = 256, thin_rows: int = 64,
                            zero: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
                            route_index: Optional[torch.Tensor] = None) -> torch.Tensor:
    """sort_routes followed by build_tiles_split on its counts, in two launches instead of four (new): the same
    outputs bit for bit. Returns the sort workspace (first int32: the dropped routes)."""
    _check(topk_ids.dim() == 2 and topk_weights.shape == topk_ids.shape, "topk_ids / topk_weights must be [T, topk]")
    _check(topk_ids.dtype in (torch.int64, torch.int32), "topk_ids must be int64 or int32")
    _check(topk_weights.dtype in (torch.float32, torch.float16, torch.bfloat16),
           "topk_weights must be float32, float16 or bfloat16")
    _check(topk_ids.is_contiguous() and topk_weights.is_contiguous(), "routing tensors must be contiguous")
    T, k = topk_ids.shape
    R = T * k
    _check(token_sorted.dtype == torch.int64 and weight_sorted.dtype == torch.float16 and
           expert_of_row.dtype == torch.int32, "sorted outputs: int64 tokens, fp16 weights, int32 experts")
    _check(token_sorted.numel() == R and weight_sorted.numel() == R and expert_of_row.numel() == R,
           "sorted outputs must have T*topk elements")
    _check(counts.dtype == torch.int32 and expert_row0.dtype == torch.int32 and counts.numel() == n_experts and
           expert_row0.numel() == n_experts, "counts / expert_row0 must be int32 [E]")
    _check(0 < n_experts <= 1024, "too many experts")
    if route_index is not None:
        _check(route_index.dtype == torch.int32 and route_index.numel() == R and route_index.is_contiguous(),
               "route_index must be contiguous int32 [T*topk]")
    for t in (full_expert, full_row0, thin_expert, thin_row0, meta):
        _check(t.dtype == torch.int32 and t.is_contiguous(), "int32 contiguous tensors")
    _check(full_row0.numel() >= full_expert.numel() and thin_row0.numel() >= thin_expert.numel() and
           meta.numel() >= 3, "tables: row0 at least as long as expert, meta int32[3]")
    _check(zero is None or (zero.dtype == torch.float32 and zero.is_contiguous() and zero.numel() % 4 == 0),
           "zero must be fp32 contiguous with a multiple of 4 elements")
    need = sort_routes_workspace_bytes(T, k, n_experts)
    tensors = (topk_ids, topk_weights, token_sorted, weight_sorted, expert_of_row, counts, expert_row0, full_expert,
               full_row0, thin_expert, thin_row0, meta) + ((zero,) if zero is not None else ())
    dev = _require_cuda(*tensors)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    _check(workspace.numel() * workspace.element_size() >= need, "sort workspace too small")
    with _On(dev) as s:
        _lib.call("exl3_sort_routes_split_tiles", _p(topk_ids), _DT[topk_ids.dtype], _p(topk_weights),
                  _DT[topk_weights.dtype], T, k, n_experts, _p(token_sorted), _p(weight_sorted), _p(expert_of_row),
                  _p(route_index), _p(counts), _p(expert_row0), _p(workspace),
                  workspace.numel() * workspace.element_size(), int(tile_rows), int(thin_rows), full_expert.numel(),
                  thin_expert.numel(), _p(full_expert), _p(full_row0), _p(thin_expert), _p(thin_row0), _p(meta),
                  _p(zero) if zero is not None else None, zero.numel() if zero is not None else 0, s)
    return workspace


def t16_rows(rows: int) -> int:
    """Rows a T16-layout buffer of `rows` logical rows holds (whole 16-row groups)."""
    return (rows + 15) // 16 * 16


def row_had(src: torch.Tensor, dst: torch.Tensor, token_sorted: Optional[torch.Tensor], expert_of_row: torch.Tensor,
            suh: torch.Tensor, gather: bool, dst_layout: int = 0, rows: Optional[int] = None) -> None:
    """kernel/exl3_grouped_prefill.cu:297-311. dst_layout (new): 0 row-major dst [rows, K]; 1 the T16 layout the
    grouped GEMM reads (dst holds t16_rows(rows) rows; `rows` gives the logical row count)."""
    K = dst.shape[1]
    if dst_layout == 0:
        rows = dst.shape[0]
    else:
        _check(dst_layout == 1 and rows is not None and dst.shape[0] >= t16_rows(rows),
               "T16 dst needs rows= and t16_rows(rows) rows")
    _check(K % 128 == 0 and suh.size(-1) == K, "K must be a multiple of 128 and match suh")
    _check(src.dtype == torch.float16 and dst.dtype == torch.float16 and suh.dtype == torch.float16,
           "fp16 tensors")
    _check(src.dim() == 2 and src.size(1) == K and src.is_contiguous() and dst.is_contiguous(),
           "src / dst must be contiguous [*, K]")
    _check(suh.dim() == 2 and suh.stride(1) == 1, "suh must be [E, K] with unit inner stride")
    _check(expert_of_row.dtype == torch.int32 and expert_of_row.numel() >= rows, "expert_of_row int32 [rows]")
    if gather:
        _check(token_sorted is not None and token_sorted.dtype == torch.int64 and token_sorted.numel() >= rows,
               "token_sorted int64 [rows]")
    else:
        _check(src.size(0) >= rows, "src has too few rows")
    dev = _require_cuda(src, dst, expert_of_row, suh, token_sorted if gather else None)
    with _On(dev) as s:
        _lib.call("exl3_row_had_ex", _p(src), _p(dst), _p(token_sorted) if gather else None, _p(expert_of_row),
                  _p(suh), suh.stride(0), suh.size(-1), rows, K, 1 if gather else 0, int(dst_layout), s)


def act_had(gu: torch.Tensor, act: torch.Tensor, expert_of_row: torch.Tensor, suh_down: torch.Tensor,
            limit: float, dst_layout: int = 0, gu_layout: int = 0, rows: Optional[int] = None) -> None:
    """kernel/exl3_grouped_prefill.cu:313-322. dst_layout (new): 0 row-major act [rows, I]; 1 T16 (rows = gu rows,
    act holds t16_rows(rows) rows). gu may be fp32 (new; the partial sums of a split-K gate|up, grouped_gemm mode 3),
    rounded to fp16 on load, with dst_layout 1. gu_layout (new): 1 = fp16 gu in the T16 layout (grouped_gemm mode 4,
    with dst_layout 1; `rows` gives its logical rows)."""
    I = act.shape[1]
    if dst_layout == 0:
        rows = act.shape[0]
    else:
        rows = gu.shape[0] if rows is None else int(rows)
        _check(dst_layout == 1 and act.shape[0] >= t16_rows(rows), "T16 act needs t16_rows(rows) rows")
    _check(gu_layout in (0, 1) and (gu_layout == 0 or (dst_layout == 1 and gu.dtype == torch.float16 and
                                                       gu.size(0) >= t16_rows(rows))),
           "a T16 gu is fp16 with t16_rows(rows) rows and writes a T16 act")
    _check(gu.size(1) == 2 * I and I % 128 == 0, "gate|up width must be 2I, I multiple of 128")
    _check(gu.dtype in (torch.float16, torch.float32) and act.dtype == torch.float16 and
           suh_down.dtype == torch.float16, "fp16 tensors (gu fp16 or fp32)")
    _check(gu.dtype == torch.float16 or dst_layout == 1, "fp32 gu writes the T16 layout")
    _check(gu.is_contiguous() and act.is_contiguous() and gu.size(0) >= rows, "gu / act must be contiguous")
    _check(suh_down.dim() == 2 and suh_down.size(1) == I and suh_down.stride(1) == 1, "suh_down must be [E, I]")
    _check(expert_of_row.dtype == torch.int32 and expert_of_row.numel() >= rows, "expert_of_row int32 [rows]")
    dev = _require_cuda(gu, act, expert_of_row, suh_down)
    with _On(dev) as s:
        if gu_layout == 1:
            _lib.call("exl3_act_had_t16", _p(gu), gu.size(1), _p(act), _p(expert_of_row), _p(suh_down),
                      suh_down.stride(0), rows, I, float(limit), s)
        elif gu.dtype == torch.float32:
            _lib.call("exl3_act_had_f32", _p(gu), gu.size(1), _p(act), _p(expert_of_row), _p(suh_down),
                      suh_down.stride(0), rows, I, float(limit), s)
        else:
            _lib.call("exl3_act_had_ex", _p(gu), gu.size(1), _p(act), _p(expert_of_row), _p(suh_down),
                      suh_down.stride(0), rows, I, float(limit), int(dst_layout), s)


# ------------------------------------------------------------------------------------------- grouped GEMM
def grouped_gemm(a: torch.Tensor, packed_gate: torch.Tensor, packed_up: Optional[torch.Tensor],
                 svh_gate: torch.Tensor, svh_up: Optional[torch.Tensor], block_expert: torch.Tensor,
                 block_row0: torch.Tensor, counts: torch.Tensor, expert_row0: torch.Tensor,
                 token_sorted: Optional[torch.Tensor], route_weight: Optional[torch.Tensor], out: torch.Tensor,
                 mode: int, route_index: Optional[torch.Tensor] = None, tile_rows: int = 128, a_layout: int = 0,
                 a_rows: Optional[int] = None, k_split: int = 1, zero: Optional[torch.Tensor] = None) -> None:
    """kernel/exl3_grouped_prefill.cu:326-378. mode 0: fp16 store; mode 1: fp32 atomic scatter into
    out[token_sorted[r]]; mode 2 (new): fp32 store of the weighted row into out[route_index[r]] (out [T*topk, N]),
    summed per token by combine_routes in a fixed order; mode 3 (new): fp32 atomic add of the unweighted row into
    out[r] (out [rows, n_tensors*N], caller-zeroed); mode 4 (new): mode 0 into a T16-layout out (what act_had reads
    with gu_layout=1). tile_rows (new): rows per block-table entry, 128 for
    build_blocks' table (the reference's), 256 or 512 for a build_tiles(..., 256 | 512) table (512 runs the 8-wave
    kernel), 64 (a thin kernel for small tiles, 16 rows per wave). a_layout (new): 0 row-major a,
    1 T16 (a from row_had / act_had with dst_layout=1; a_rows gives its logical rows). k_split (new): slices of K
    whose partial products are added into out (modes 1 and 3 only). zero (new, optional fp32 contiguous, numel % 4 ==
    0, not overlapping a or out): cleared by the same launch, e.g. the output a later mode-1 launch adds into."""
    _check(int(tile_rows) in (64, 128, 256, 512), "tile_rows must be 64, 128, 256 or 512")
    _check(int(k_split) >= 1 and int(k_split) <= a.size(1) // 64, "k_split must be in [1, K / 64]")
    _check(int(k_split) == 1 or mode in (1, 3), "k_split > 1 needs mode 1 or 3")
    _check(a_layout in (0, 1), "unknown layout")
    if a_rows is None:
        a_rows = a.size(0)
    _check(a_layout == 0 or a.size(0) >= t16_rows(a_rows), "T16 a needs t16_rows(a_rows) rows")
    _check(a.dtype == torch.float16 and a.is_contiguous(), "a fp16 contiguous")
    _check(packed_gate.dim() == 4 and packed_gate.dtype in (torch.int16, torch.uint16) and
           packed_gate.stride(3) == 1 and packed_gate.stride(2) == packed_gate.size(3) and
           packed_gate.stride(1) == packed_gate.size(2) * packed_gate.size(3),
           "packed [E, tiles_k, tiles_n, 64] with contiguous inner dims (expert stride may be larger: [E,2,...] views)")
    words = packed_gate.size(3)
    _check(words in (32, 48, 64), "packed tile width must be 16*bits words, bits in {2, 3, 4}")
    bits = words // 16
    size_k, tiles_k, tiles_n = a.size(1), packed_gate.size(1), packed_gate.size(2)
    _check(size_k == tiles_k * 16 and size_k % 64 == 0, "K mismatch")
    size_n_each = tiles_n * 16
    _check(size_n_each % 128 == 0, "N must be a multiple of 128")
    n_tensors = 2 if packed_up is not None else 1
    expert_stride = packed_gate.stride(0)
    _check(svh_gate.dtype == torch.float16 and svh_gate.dim() == 2 and svh_gate.stride(1) == 1, "svh fp16 [E, N]")
    svh_stride = svh_gate.stride(0)
    _check(svh_gate.size(-1) == size_n_each, "svh N mismatch")
    if packed_up is not None:
        _check(packed_up.shape == packed_gate.shape and packed_up.stride() == packed_gate.stride() and
               svh_up is not None and svh_up.stride() == svh_gate.stride() and svh_up.shape == svh_gate.shape,
               "gate/up strides must match")
    E = counts.numel()
    _check(packed_gate.size(0) >= E and svh_gate.size(0) >= E, "fewer experts in the weights than in counts")
    _check(block_expert.dtype == torch.int32 and block_row0.dtype == torch.int32 and counts.dtype == torch.int32
           and expert_row0.dtype == torch.int32, "int32 block table")
    max_blocks = block_expert.numel()
    if mode in (0, 4):
        _check(out.dtype == torch.float16 and out.dim() == 2 and out.size(1) == n_tensors * size_n_each and
               out.is_contiguous() and out.size(0) >= (a_rows if mode == 0 else t16_rows(a_rows)),
               "mode 0: out fp16 [rows, n_tensors*N] (mode 4: T16, t16_rows(rows) rows)")
    elif mode == 1:
        _check(out.dtype == torch.float32 and out.dim() == 2 and out.size(1) == size_n_each and n_tensors == 1 and
               out.is_contiguous(), "mode 1: out fp32 [T, N], single tensor")
        _check(token_sorted is not None and route_weight is not None and token_sorted.dtype == torch.int64 and
               route_weight.dtype == torch.float16, "routing dtypes")
    elif mode == 2:
        _check(out.dtype == torch.float32 and out.dim() == 2 and out.size(1) == size_n_each and n_tensors == 1 and
               out.is_contiguous(), "mode 2: out fp32 [routes, N], single tensor")
        _check(route_index is not None and route_weight is not None and route_index.dtype == torch.int32 and
               route_weight.dtype == torch.float16, "mode 2 needs route_index (int32) and route_weight (fp16)")
    elif mode == 3:
        _check(out.dtype == torch.float32 and out.dim() == 2 and out.size(1) == n_tensors * size_n_each and
               out.is_contiguous() and out.size(0) >= a_rows, "mode 3: out fp32 [rows, n_tensors*N]")
        _check(int(tile_rows) <= 256, "mode 3 takes row tiles of 64, 128 or 256 rows")
    else:
        raise RuntimeError("mode must be 0, 1, 2, 3 or 4")
    _check(zero is None or (zero.dtype == torch.float32 and zero.is_contiguous() and zero.numel() % 4 == 0),
           "zero must be fp32 contiguous with a multiple of 4 elements")
    weighted = mode in (1, 2)
    dev = _require_cuda(a, packed_gate, packed_up, svh_gate, svh_up, block_expert, block_row0, counts,
                        expert_row0, out, token_sorted if mode == 1 else None, route_weight if weighted else None,
                        route_index if mode == 2 else None, zero)
    args = (_p(a), int(a_rows), size_k, int(a_layout), _p(packed_gate), _p(packed_up), expert_stride, tiles_k, tiles_n,
            bits, _p(svh_gate), _p(svh_up), svh_stride, _p(block_expert), _p(block_row0), max_blocks, int(tile_rows),
            _p(counts), _p(expert_row0), E, _p(token_sorted) if mode == 1 else None,
            _p(route_weight) if weighted else None, _p(route_index) if mode == 2 else None, _p(out), out.size(0), mode,
            int(k_split))
    with _On(dev) as s:
        if zero is None:
            _lib.call("exl3_grouped_gemm_split", *args, s)
        else:
            _lib.call("exl3_grouped_gemm_clear", *args, _p(zero), zero.numel(), s)


def combine_routes(partial: torch.Tensor, out: torch.Tensor, topk: int, topk_ids: Optional[torch.Tensor] = None,
                   n_experts: int = 0) -> None:
    """out[t] = sum_j partial[t*topk + j] in order j = 0..topk-1 (new; pairs with grouped_gemm mode 2). Routes whose id
    in topk_ids lies outside [0, n_experts) are skipped. out fp32, or bf16 / fp16: each fp32 sum rounded once, as
    casting the fp32 result would (the reference wrapper's out.to(x.dtype), kernel/exl3_grouped_runtime.py:107)."""
    T, n = out.shape
    _check(partial.dtype == torch.float32 and out.dtype in (torch.float32, torch.bfloat16, torch.float16) and
           partial.is_contiguous() and out.is_contiguous(),
           "combine: partial fp32, out fp32 / bf16 / fp16, contiguous")
    _check(partial.dim() == 2 and partial.size(0) == T * topk and partial.size(1) == n and n % 4 == 0,
           "combine: partial must be [T*topk, N], N % 4 == 0")
    _check(1 <= int(topk) <= 32, "combine: topk must be in [1, 32]")
    if topk_ids is not None:
        _check(topk_ids.dtype in (torch.int64, torch.int32) and topk_ids.is_contiguous() and
               topk_ids.numel() == T * topk and 0 < n_experts <= 1024, "combine: topk_ids [T, topk] int64/int32")
    dev = _require_cuda(partial, out, topk_ids)
    with _On(dev) as s:
        _lib.call("exl3_combine_routes_dt", _p(partial), _p(out), _DT[out.dtype], _p(topk_ids),
                  _DT[topk_ids.dtype] if topk_ids is not None else 0, int(n_experts), T, int(topk), n, s)


# ------------------------------------------------------------------------------------------- per-expert entry
def _fat_check(a, packed, out, svh, K, mcg, mul1):
    """kernel/exl3_fat_gemm_v2.cu:236-252 (bits 2 and 3 accepted in addition to 4)."""
    _check(a.is_contiguous() and packed.is_contiguous() and out.is_contiguous() and svh.is_contiguous(),
           "tensors must be contiguous")
    _check(a.dtype == torch.float16, "a must be float16")
    _check(packed.dtype in (torch.int16, torch.uint16), "packed must be int16")
    _check(out.dtype == torch.float32, "out must be float32")
    _check(svh.dtype == torch.float16, "svh must be float16")
    _check(a.dim() == 2 and packed.dim() == 3 and out.dim() == 2 and svh.dim() == 1, "rank mismatch")
    _check(int(K) in (2, 3, 4) and bool(mcg) and not bool(mul1), "only K2/K3/K4 MCG tensors")
    _check(a.size(1) == packed.size(0) * 16, "a K dimension does not match packed tensor")
    _check(svh.numel() == packed.size(1) * 16, "svh N dimension does not match packed tensor")
    _check(svh.numel() % 128 == 0, "N must be divisible by 128")
    _check(packed.size(2) == 16 * int(K), "packed block width must be 16*K int16 words")
    _check(a.size(1) % 64 == 0, "K must be divisible by 64")


def fat_gemm_v2(a: torch.Tensor, packed: torch.Tensor, out: torch.Tensor, svh: torch.Tensor, K: int, mcg: bool,
                mul1: bool, variant: int = 1) -> None:
    """kernel/exl3_fat_gemm_v2.cu:298-303: out[M, N] = H128(a @ W') / sqrt(128) * svh (fp32). variant: the row-tile
    schedule (see smem_bytes); every variant gives bit-identical results."""
    _fat_check(a, packed, out, svh, K, mcg, mul1)
    _check(out.size(0) == a.size(0) and out.size(1) == svh.numel(), "out shape must be [M, N]")
    _check(0 <= int(variant) <= 3, "unknown variant")
    dev = _require_cuda(a, packed, out, svh)
    with _On(dev) as s:
        _lib.call("exl3_fat_gemm", _p(a), a.size(0), a.size(1), _p(packed), packed.size(0), packed.size(1),
                  packed.size(2), _p(out), out.size(0), _p(svh), svh.numel(), int(K), int(bool(mcg)),
                  int(bool(mul1)), int(variant), s)


def fat_gemm_v2_scatter(a: torch.Tensor, packed: torch.Tensor, out: torch.Tensor, svh: torch.Tensor,
                        token_idx: torch.Tensor, route_weight: torch.Tensor, K: int, mcg: bool, mul1: bool,
                        variant: int = 1) -> None:
    """kernel/exl3_fat_gemm_v2.cu:305-314: out[token_idx[m]] += fp32(route_weight[m]) * y[m] (device atomics)."""
    _fat_check(a, packed, out, svh, K, mcg, mul1)
    _check(out.size(1) == svh.numel(), "out N dimension mismatch")
    _check(token_idx.is_contiguous() and route_weight.is_contiguous(), "routing tensors")
    _check(token_idx.dtype == torch.int64 and route_weight.dtype == torch.float16, "routing dtypes")
    _check(token_idx.numel() == a.size(0) and route_weight.numel() == a.size(0),
           "routing tensors must have M elements")
    _check(0 <= int(variant) <= 3, "unknown variant")
    dev = _require_cuda(a, packed, out, svh, token_idx, route_weight)
    with _On(dev) as s:
        _lib.call("exl3_fat_gemm_scatter", _p(a), a.size(0), a.size(1), _p(packed), packed.size(0), packed.size(1),
                  packed.size(2), _p(out), out.size(0), _p(svh), svh.numel(), _p(token_idx), _p(route_weight),
                  int(K), int(bool(mcg)), int(bool(mul1)), int(variant), s)


def exl3_fat_gemm(a: torch.Tensor, packed: torch.Tensor, out: torch.Tensor, svh: torch.Tensor, K: int, mcg: bool,
                  mul1: bool) -> None:
    """PR77's per-expert op with its argument order, ext.exl3_fat_gemm(a, packed, out, svh, K, mcg, mul1)
    (kernel/test_fat_v2.py:122): fat_gemm_v2 with the shape-tuned schedule (variant 1)."""
    fat_gemm_v2(a, packed, out, svh, K, mcg, mul1, 1)


def exl3_fat_gemm_scatter(a: torch.Tensor, packed: torch.Tensor, out: torch.Tensor, svh: torch.Tensor,
                          tok: torch.Tensor, rw: torch.Tensor, K: int, mcg: bool, mul1: bool) -> None:
    """PR77's scatter op with its argument order, ext.exl3_fat_gemm_scatter(a, packed, out, svh, tok, rw, K, mcg,
    mul1) (kernel/test_fat_v2.py:134): fat_gemm_v2_scatter with the shape-tuned schedule (variant 1)."""
    fat_gemm_v2_scatter(a, packed, out, svh, tok, rw, K, mcg, mul1, 1)


def linear_workspace_bytes(m: int, k: int) -> int:
    """Bytes of the scratch buffer linear_exl3 needs for m rows of width k (the input Hadamard in the T16 layout)."""
    return int(_lib.load().exl3_linear_workspace_bytes(int(m), int(k)))


def linear_exl3(x: torch.Tensor, packed: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, K: int = 4,
                out: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.float16,
                work: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dense EXL3 linear (new; the LinearEXL3 forward the reference's path sits next to):
    y = H128(H128(x * suh)/sqrt(128) @ W')/sqrt(128) * svh over x fp16 [M, in], packed [in/16, out/16, 16*K] int16,
    suh fp16 [in], svh fp16 [out]; returns y [M, out] in out_dtype (fp16 or fp32). `work` (uint8 or any dtype, at
    least linear_workspace_bytes(M, in) bytes) is allocated when not given."""
    _check(x.dim() == 2 and x.dtype == torch.float16 and x.is_contiguous(), "x must be contiguous fp16 [M, in]")
    _check(packed.dim() == 3 and packed.dtype == torch.int16 and packed.is_contiguous(),
           "packed must be contiguous int16 [in/16, out/16, 16*K]")
    _check(packed.size(2) == 16 * int(K), "packed block width must be 16*K int16 words")
    _check(suh.dtype == torch.float16 and svh.dtype == torch.float16 and suh.is_contiguous() and svh.is_contiguous(),
           "suh/svh must be contiguous fp16")
    M, k = x.shape
    n = packed.size(1) * 16
    _check(k == packed.size(0) * 16 and suh.numel() == k, "x in-features must match the packed tensor and suh")
    _check(svh.numel() == n, "svh must have out-features elements")
    _check(out_dtype in (torch.float16, torch.float32), "out must be fp16 or fp32")
    if out is None:
        out = torch.empty(M, n, dtype=out_dtype, device=x.device)
    _check(out.dtype == out_dtype and tuple(out.shape) == (M, n) and out.is_contiguous(), "out must be [M, out]")
    need = linear_workspace_bytes(M, k)
    if work is None:
        work = torch.empty(max(need, 16), dtype=torch.uint8, device=x.device)
    _check(work.is_contiguous() and work.numel() * work.element_size() >= need, "work buffer too small")
    dev = _require_cuda(x, packed, suh, svh, out, work)
    with _On(dev) as s:
        _lib.call("exl3_linear", _p(x), M, k, _p(packed), packed.size(0), packed.size(1), int(K), _p(suh), _p(svh),
                  _p(work), _p(out), 0 if out_dtype == torch.float32 else 1, s)
    return out


# ------------------------------------------------------------------------------------------- decode path
SMALL_ROUTES = 2048


def route_prep_small(topk_ids: torch.Tensor, topk_weights: torch.Tensor, n_experts: int, token_sorted: torch.Tensor,
                     weight_sorted: torch.Tensor, expert_of_row: torch.Tensor, counts: torch.Tensor,
                     expert_row0: torch.Tensor, tile_expert: torch.Tensor, tile_row0: torch.Tensor,
                     meta: torch.Tensor, tile_rows: int = 128, zero: tuple = ()) -> None:
    """The decode path's route preparation in one launch (new): sort_routes + build_tiles for at most 2048 routes,
    and a zero fill of up to two contiguous fp32 tensors in `zero`."""
    _check(topk_ids.dim() == 2 and topk_weights.shape == topk_ids.shape, "topk_ids / topk_weights must be [T, topk]")
    _check(topk_ids.dtype in (torch.int64, torch.int32) and topk_ids.is_contiguous(), "topk_ids int64/int32")
    _check(topk_weights.dtype in (torch.float32, torch.float16, torch.bfloat16) and topk_weights.is_contiguous(),
           "topk_weights fp32/fp16/bf16")
    T, k = topk_ids.shape
    R = T * k
    _check(R <= SMALL_ROUTES, f"route_prep_small takes at most {SMALL_ROUTES} routes")
    _check(token_sorted.dtype == torch.int64 and weight_sorted.dtype == torch.float16 and
           expert_of_row.dtype == torch.int32 and min(token_sorted.numel(), weight_sorted.numel(),
                                                      expert_of_row.numel()) >= R, "sorted outputs [R]")
    _check(counts.dtype == torch.int32 and expert_row0.dtype == torch.int32 and counts.numel() >= n_experts and
           expert_row0.numel() >= n_experts, "counts / expert_row0 int32 [E]")
    _check(tile_expert.dtype == torch.int32 and tile_row0.dtype == torch.int32 and meta.dtype == torch.int32 and
           tile_row0.numel() >= tile_expert.numel() and meta.numel() >= 2, "int32 tile table")
    _check(len(zero) <= 2 and all(z.dtype == torch.float32 and z.is_contiguous() and z.numel() % 4 == 0
                                  for z in zero), "zero: up to two contiguous fp32 tensors of whole float4s")
    z = list(zero) + [None] * (2 - len(zero))
    dev = _require_cuda(topk_ids, topk_weights, token_sorted, weight_sorted, expert_of_row, counts, expert_row0,
                        tile_expert, tile_row0, meta, *zero)
    with _On(dev) as s:
        _lib.call("exl3_route_prep_small", _p(topk_ids), _DT[topk_ids.dtype], _p(topk_weights),
                  _DT[topk_weights.dtype], T, k, int(n_experts), int(tile_rows), tile_expert.numel(),
                  _p(token_sorted), _p(weight_sorted), _p(expert_of_row), _p(counts), _p(expert_row0),
                  _p(tile_expert), _p(tile_row0), _p(meta), _p(z[0]), 0 if z[0] is None else z[0].numel(), _p(z[1]),
                  0 if z[1] is None else z[1].numel(), s)


def moe_decode_workspace_bytes(tokens: int, topk: int, n_experts: int, hidden: int, inter: int) -> int:
    """Bytes of the workspace moe_decode needs (sorted routes, tile table, the Hadamard'd rows, fp32 gate|up sums)."""
    v = int(_lib.load().exl3_moe_decode_workspace_bytes(int(tokens), int(topk), int(n_experts), int(hidden),
                                                         int(inter)))
    _check(v >= 0, "bad decode sizes")
    return v


def moe_decode(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor, w13_trellis: torch.Tensor,
               w13_suh: torch.Tensor, w13_svh: torch.Tensor, w2_trellis: torch.Tensor, w2_suh: torch.Tensor,
               w2_svh: torch.Tensor, limit: float, out: Optional[torch.Tensor] = None,
               workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode-path MoE (new; replaces the overlay's fused exl3_moe call on the `tokens <= cap` side of
    kernel/exl3_grouped_runtime.py:93-98): x fp16 [T, H], topk_ids [T, topk] int64/int32, topk_weights [T, topk]
    fp32/fp16/bf16, the stacked layer tensors (w13_trellis [E, 2, H/16, I/16, 16*bits], w13_suh [E, 2, H] with
    gate == up, w13_svh [E, 2, I], w2_trellis [E, I/16, H/16, 16*bits], w2_suh [E, I], w2_svh [E, H]) -> out fp32
    [T, H]. One fixed launch sequence that allocates nothing when `out` and `workspace` (uint8, at least
    moe_decode_workspace_bytes(...) bytes, 256-byte aligned) are given, so the call can be captured in a graph."""
    _check(x.dim() == 2 and x.dtype == torch.float16 and x.is_contiguous(), "x must be contiguous fp16 [T, H]")
    T, H = x.shape
    _check(topk_ids.dim() == 2 and topk_ids.size(0) == T and topk_weights.shape == topk_ids.shape,
           "topk_ids / topk_weights must be [T, topk]")
    _check(topk_ids.dtype in (torch.int64, torch.int32) and topk_ids.is_contiguous(), "topk_ids int64/int32")
    _check(topk_weights.dtype in (torch.float32, torch.float16, torch.bfloat16) and topk_weights.is_contiguous(),
           "topk_weights fp32/fp16/bf16")
    topk = topk_ids.size(1)
    _check(w13_trellis.dim() == 5 and w13_trellis.size(1) == 2 and w13_trellis.dtype in (torch.int16, torch.uint16),
           "w13_trellis must be [E, 2, H/16, I/16, 16*bits] int16")
    E = w13_trellis.size(0)
    words = w13_trellis.size(4)
    _check(words in (32, 48, 64), "trellis tile width must be 16*bits words, bits in {2, 3, 4}")
    bits = words // 16
    _check(w13_trellis.size(2) * 16 == H, "w13_trellis K must match x")
    inter = w13_trellis.size(3) * 16
    g, u = w13_trellis[:, 0], w13_trellis[:, 1]
    for t in (g, u):
        _check(t.stride(3) == 1 and t.stride(2) == words and t.stride(1) == t.size(2) * words,
               "w13_trellis inner dims must be contiguous")
    _check(w2_trellis.dim() == 4 and w2_trellis.shape == (E, inter // 16, H // 16, words) and
           w2_trellis.dtype == w13_trellis.dtype and w2_trellis.stride(3) == 1 and w2_trellis.stride(2) == words and
           w2_trellis.stride(1) == w2_trellis.size(2) * words, "w2_trellis must be [E, I/16, H/16, 16*bits]")
    _check(w13_suh.shape == (E, 2, H) and w13_svh.shape == (E, 2, inter) and w2_suh.shape == (E, inter) and
           w2_svh.shape == (E, H), "sign / scale vector shapes")
    for t in (w13_suh, w13_svh, w2_suh, w2_svh):
        _check(t.dtype == torch.float16 and t.stride(-1) == 1, "suh / svh must be fp16 with contiguous rows")
    _check(w13_svh[:, 0].stride() == w13_svh[:, 1].stride(), "gate / up svh strides must match")
    if out is None:
        out = torch.empty(T, H, dtype=torch.float32, device=x.device)
    _check(out.dtype == torch.float32 and tuple(out.shape) == (T, H) and out.is_contiguous(), "out must be fp32 [T, H]")
    need = moe_decode_workspace_bytes(T, topk, E, H, inter)
    if workspace is None:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=x.device)
    _check(workspace.is_contiguous() and workspace.numel() * workspace.element_size() >= need,
           "decode workspace too small")
    dev = _require_cuda(x, topk_ids, topk_weights, w13_trellis, w13_suh, w13_svh, w2_trellis, w2_suh, w2_svh, out,
                        workspace)
    with _On(dev) as s:
        _lib.call("exl3_moe_decode", _p(x), T, H, _p(topk_ids), _DT[topk_ids.dtype], _p(topk_weights),
                  _DT[topk_weights.dtype], topk, E, inter, bits, _p(g), _p(u), g.stride(0), _p(w13_suh[:, 0]),
                  w13_suh.stride(0), _p(w13_svh[:, 0]), _p(w13_svh[:, 1]), w13_svh.stride(0), _p(w2_trellis),
                  w2_trellis.stride(0), _p(w2_suh), w2_suh.stride(0), _p(w2_svh), w2_svh.stride(0), float(limit),
                  _p(out), _p(workspace), workspace.numel() * workspace.element_size(), s)
    return out


def smem_bytes(variant: int) -> int:
    """kernel/exl3_fat_gemm_v2.cu:316-326: LDS bytes per workgroup of the kernels `variant` launches (the largest of
    them: the scatter form stages output rows), -1 if unknown. Variants select the row-tile schedule: 0 64-row tiles,
    1 the shape-tuned policy (64- or 512-row tiles), 2 256-row tiles, 3 512-row tiles."""
    return int(_lib.load().exl3_smem_bytes(int(variant)))


# ------------------------------------------------------------------------------------------- trellis utilities
def reconstruct(w: torch.Tensor, packed: torch.Tensor, K: int, mcg: bool, mul1: bool) -> None:
    """exllamav3 ext.reconstruct(w, packed, K, mcg, mul1): W' fp16 [16 tiles_k, 16 tiles_n]."""
    _check(packed.dim() == 3 and packed.is_contiguous() and packed.dtype in (torch.int16, torch.uint16),
           "packed must be contiguous int16 [tiles_k, tiles_n, 16*K]")
    _check(int(K) in (2, 3, 4) and bool(mcg) and not bool(mul1), "only K2/K3/K4 MCG tensors")
    _check(packed.size(2) == 16 * int(K), "packed block width must be 16*K int16 words")
    _check(w.dtype == torch.float16 and w.is_contiguous() and w.shape == (packed.size(0) * 16, packed.size(1) * 16),
           "w must be contiguous fp16 [16 tiles_k, 16 tiles_n]")
    dev = _require_cuda(w, packed)
    with _On(dev) as s:
        _lib.call("exl3_reconstruct", _p(w), _p(packed), packed.size(0), packed.size(1), int(K), int(bool(mcg)),
                  int(bool(mul1)), s)


def decode_states(states: torch.Tensor, out: torch.Tensor) -> None:
    """out[i] = fp16 decode(states[i]) with the GEMM's device decoder (states int16/uint16, even count)."""
    _check(states.dtype in (torch.int16, torch.uint16) and out.dtype in (torch.float16, torch.int16, torch.uint16),
           "16-bit tensors")
    _check(states.is_contiguous() and out.is_contiguous() and states.numel() == out.numel() and
           states.numel() % 2 == 0, "contiguous, equal, even sizes")
    dev = _require_cuda(states, out)
    with _On(dev) as s:
        _lib.call("exl3_decode_states", _p(states), _p(out), states.numel(), s)
