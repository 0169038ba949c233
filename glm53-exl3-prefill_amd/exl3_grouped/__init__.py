"""MI355X (gfx950) EXL3 grouped routed-expert MoE prefill: torch-facing ops over the libexl3_grouped.so C ABI."""
from .ops import (act_had, build_blocks, build_tiles, build_tiles_split, combine_routes, decode_states, exl3_fat_gemm,
                  exl3_fat_gemm_scatter, fat_gemm_v2, fat_gemm_v2_scatter, grouped_gemm,  # noqa: F401
                  linear_exl3, linear_workspace_bytes, moe_decode, moe_decode_workspace_bytes, reconstruct, route_prep_small, route_topk,
                  row_had, smem_bytes, sort_routes, sort_routes_split_tiles, sort_routes_workspace_bytes, t16_rows)
from . import _lib  # noqa: F401


def library_path() -> str:
    """Path of the loaded (or to-be-loaded) native library."""
    return _lib.path()
