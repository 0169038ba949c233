"""Serving integration for the grouped EXL3 MoE prefill on MI355X (same contract as the reference's
kernel/exl3_grouped_runtime.py, whose functions and behaviour this module mirrors).

Installed into vLLM's exl3 overlay module by patch_exl3_grouped.py when EXL3_GROUPED_PREFILL != "0".
Prefill calls (tokens > the fused kernel's row cap) go through one launch per stage over all experts
(kernel/exl3_grouped_runtime.py:93-98). Decode calls (tokens <= cap), which the reference leaves to the overlay's
fused exl3_moe (a CUDA kernel with no build on this GPU), go to moe_decode: the same stages with split-K GEMMs and a
per-device workspace sized once for the row cap, one fixed launch sequence that a HIP graph can capture.
Expert-parallel calls (layer.expert_map set) and layers without w13_trellis keep the original path untouched.

Env:
  EXL3_GROUPED_PREFILL=1     enable (read by the hook)
  EXL3_GROUPED_DECODE=0      leave decode calls (tokens <= cap) to the original path (default: moe_decode)
  EXL3_GROUPED_THIN=0        run every expert tile on the main GEMM kernel (default: an expert's last tile of <= 64
                             rows runs on the thin kernel, four workgroups per CU, in a second launch)
  EXL3_GROUPED_SCATTER=...   down-projection output: "atomic" (fp32 atomic scatter by token, the reference's
                             method), "combine" (per-route fp32 rows + a fixed-order sum per token: deterministic) or
                             "auto" (the default: combine for chunks of >= COMBINE_MIN_ROUTES routes, else atomic)
  EXL3_GROUPED_COMBINE_MIN_ROUTES=<n>   the "auto" threshold in routes (tokens x topk; default 16384)
  EXL3_GROUPED_WORKSPACE=0   allocate the prefill intermediates per call (default: one reused buffer per device)
  EXL3_GROUPED_LIB=<path>    prebuilt libexl3_grouped.so (default: exl3_grouped/libexl3_grouped.so beside this file)
"""
import logging
import os
import sys
import time

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
if _HERE not in sys.path:
    sys.path.insert(0, _HERE)

logger = logging.getLogger("vllm.exl3.grouped")
_ext = None
_logged = False


def _load_ext():
    """Load the native library once (kernel/exl3_grouped_runtime.py:20-47 JIT-compiles instead; here the
    library is built ahead of time for gfx950). Raises if it is missing."""
    global _ext
    if _ext is not None:
        return _ext
    t0 = time.time()
    import exl3_grouped
    exl3_grouped._lib.load()
    _ext = exl3_grouped
    logger.info("EXL3 grouped prefill library loaded in %.2fs from %s", time.time() - t0, exl3_grouped.library_path())
    return _ext


SCATTER_MODES = ("atomic", "combine", "auto")
# "auto" takes the combine method from this many routes (tokens x topk) up: the per-route rows plus the sum per token
# cost less than the atomic scatter once most rows sit in full 256-row expert tiles, whose epilogues are atomic-bound
# (headline routing: 2.12-2.13 vs 2.17 ms at 8192 tokens, 0.802 vs 0.817 ms at 2048), and more when most tiles are
# thin (1024 tokens, softmax routing: 0.74 vs 0.725 ms). The combine rows take routes x hidden fp32 of workspace.
COMBINE_MIN_ROUTES = 16384
TILE_ROWS_CHOICES = (128, 256, 512)
TILE_ROWS = 256


def scatter_mode() -> str:
    m = os.environ.get("EXL3_GROUPED_SCATTER", "auto")
    if m not in SCATTER_MODES:
        raise RuntimeError(f"EXL3_GROUPED_SCATTER must be one of {SCATTER_MODES}, got {m!r}")
    return m


def resolve_scatter(scatter: str | None, routes: int) -> str:
    """The down-projection output method of a call of `routes` routes: "atomic" or "combine" ("auto" and None, which
    means the EXL3_GROUPED_SCATTER setting, resolve by COMBINE_MIN_ROUTES)."""
    m = scatter or scatter_mode()
    if m not in SCATTER_MODES:
        raise RuntimeError(f"scatter must be one of {SCATTER_MODES}, got {m!r}")
    if m == "auto":
        v = os.environ.get("EXL3_GROUPED_COMBINE_MIN_ROUTES")
        try:
            threshold = COMBINE_MIN_ROUTES if v is None else int(v)
        except ValueError:
            threshold = -1
        if threshold < 0:
            raise RuntimeError(f"EXL3_GROUPED_COMBINE_MIN_ROUTES must be a non-negative integer, got {v!r}")
        return "combine" if routes >= threshold else "atomic"
    return m


def tile_rows() -> int:
    """Rows per expert row tile of the grouped GEMMs (EXL3_GROUPED_TILE_ROWS, default TILE_ROWS): 512-row tiles run
    the 8-wave GEMM kernel, which decodes each trellis stage once for twice the MFMA work (slower than the 256-row
    default on the configs measured)."""
    v = os.environ.get("EXL3_GROUPED_TILE_ROWS")
    if v is None:
        return TILE_ROWS
    if not v.isdigit() or int(v) not in TILE_ROWS_CHOICES:
        raise RuntimeError(f"EXL3_GROUPED_TILE_ROWS must be one of {TILE_ROWS_CHOICES}, got {v!r}")
    return int(v)


def thin_tiles_enabled() -> bool:
    return os.environ.get("EXL3_GROUPED_THIN", "1") != "0"


THIN_ROWS = 64

# The prefill intermediates (sorted routes, tile tables, h13, gu, act: ~0.85 GB at 8192 tokens; with the combine output
# also the per-route fp32 rows, 1.07 GB more at H = 4096) live in one buffer per device, reused by every call: steady-state
# calls allocate nothing but their output, and the kernels keep working on memory they have touched before. Calls on one
# device must be ordered on one stream (the model runner's); EXL3_GROUPED_WORKSPACE=0 allocates per call instead.
# When a call needs more, the buffer grows to at least WS_GROWTH times its old size (so rising chunk sizes re-allocate a
# few times, not on every call) and the outgrown buffer is released: one live workspace per device. Graph capture is
# the exception: a HIP graph captured over an earlier call still addresses the old buffer, so an outgrown buffer is kept
# while the current stream is capturing or once the caller has asked for it (keep_outgrown_prefill_workspaces(True),
# or reserve_prefill_workspace(..., keep_outgrown=True)); release_outgrown_prefill_workspaces frees those once no such
# graph is replayed. The reference's prefill path is eager-only (kernel/exl3_grouped_runtime.py:4-5), so freeing is the
# default.
WS_GROWTH = 1.25
WS_ALIGN = 2 << 20
_prefill_ws: dict = {}
_prefill_ws_outgrown: dict = {}
_keep_outgrown = False


def _device_index(dev: torch.device) -> int:
    if dev.type != "cuda":
        return -1                           # host buffers (CPU tests of the workspace policy)
    return dev.index if dev.index is not None else torch.cuda.current_device()


def workspace_enabled() -> bool:
    return os.environ.get("EXL3_GROUPED_WORKSPACE", "1") != "0"


class _Carve:
    """Tensors carved out of one byte buffer at 256-byte boundaries (a first pass with buf=None only sizes them)."""

    def __init__(self, buf=None, dev=None):
        self.buf, self.dev, self.off = buf, dev, 0

    def __call__(self, shape, dtype):
        n = 1
        for d in shape:
            n *= int(d)
        nbytes = n * dtype.itemsize
        start = (self.off + 255) // 256 * 256
        self.off = start + nbytes
        if self.buf is None:
            return torch.empty(shape, dtype=dtype, device=self.dev) if self.dev is not None else None
        return self.buf[start:start + nbytes].view(dtype).view(shape)


def _prefill_buffers(dev, plan):
    """plan(take) requests every intermediate via take(shape, dtype) and returns them; served from the device's prefill
    workspace (grown to fit) or, with the workspace off, from the allocator."""
    if not workspace_enabled():
        return plan(_Carve(None, dev))
    sizing = _Carve()
    plan(sizing)
    return plan(_Carve(_prefill_workspace(dev, sizing.off)))


def _capturing(dev) -> bool:
    return dev.type == "cuda" and torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def _prefill_workspace(dev, nbytes: int) -> torch.Tensor:
    key = _device_index(dev)
    ws = _prefill_ws.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(nbytes, 256)
        if ws is not None:
            size = max(size, int(ws.numel() * WS_GROWTH))
            if _keep_outgrown or _capturing(dev):
                _prefill_ws_outgrown.setdefault(key, []).append(ws)
        size = (size + WS_ALIGN - 1) // WS_ALIGN * WS_ALIGN
        _prefill_ws[key] = None
        ws = None                           # the outgrown buffer returns to the allocator before the new one is taken
        ws = torch.empty(size, dtype=torch.uint8, device=dev)
        _prefill_ws[key] = ws
    return ws


def keep_outgrown_prefill_workspaces(keep: bool = True) -> None:
    """Keep (True) or release (False, the default) a prefill workspace that a larger call outgrows. Keep them while HIP
    graphs captured over earlier calls may still be replayed; outgrown buffers are always kept during a capture."""
    global _keep_outgrown
    _keep_outgrown = bool(keep)


def live_prefill_workspaces(device=None) -> int:
    """Prefill workspaces this module holds (current + outgrown kept), on every device or on one."""
    keys = [_device_index(torch.device(device))] if device is not None else set(_prefill_ws) | set(_prefill_ws_outgrown)
    return sum((_prefill_ws.get(k) is not None) + len(_prefill_ws_outgrown.get(k, [])) for k in keys)


def release_outgrown_prefill_workspaces(device=None) -> None:
    """Free the prefill workspaces that larger calls replaced and that were kept (on every device, or one), once no HIP
    graph captured over an earlier, smaller call is replayed any more."""
    for key in ([_device_index(torch.device(device))] if device is not None else list(_prefill_ws_outgrown)):
        _prefill_ws_outgrown.pop(key, None)


def reserve_prefill_workspace(device, tokens: int, topk: int, n_experts: int, hidden: int, inter: int,
                              scatter: str | None = None, rows_per_tile: int | None = None,
                              keep_outgrown: bool | None = None) -> torch.Tensor:
    """Size the device's prefill workspace for a chunk of `tokens` (the largest the scheduler sends) before the first
    call, e.g. ahead of memory profiling or graph capture, so that no later call grows it. keep_outgrown (if given)
    sets keep_outgrown_prefill_workspaces. Returns the buffer."""
    if keep_outgrown is not None:
        keep_outgrown_prefill_workspaces(keep_outgrown)
    scatter = resolve_scatter(scatter, tokens * topk)
    tr = rows_per_tile or tile_rows()
    thin = thin_tiles_enabled()
    sizing = _Carve()
    _prefill_plan(_load_ext(), tokens, hidden, topk, n_experts, inter, tr, scatter, thin)(sizing)
    return _prefill_workspace(torch.device(device), sizing.off)


def _prefill_plan(gp, T: int, K: int, topk: int, E: int, I: int, tr: int, scatter: str, thin: bool):
    """The intermediates of one grouped_prefill call of T tokens, requested in a fixed order through take(shape, dtype):
    the sorted routes, the tile tables (rows_per_tile tr, plus the thin table), and h13 / gu / act in the T16 layout."""
    R = T * topk
    max_blocks = R // tr + E
    R16 = gp.t16_rows(R)

    def plan(take):
        return dict(
            token_sorted=take((R,), torch.int64), weight_sorted=take((R,), torch.float16),
            expert_of_row=take((R,), torch.int32), counts=take((E,), torch.int32), expert_row0=take((E,), torch.int32),
            route_index=take((R,), torch.int32) if scatter == "combine" else None,
            sort_ws=take((gp.sort_routes_workspace_bytes(T, topk, E),), torch.uint8),
            block_expert=take((max_blocks,), torch.int32), block_row0=take((max_blocks,), torch.int32),
            thin_expert=take((min(E, R),), torch.int32) if thin else None,
            thin_row0=take((min(E, R),), torch.int32) if thin else None,
            meta=take((3 if thin else 2,), torch.int32),
            # the GEMMs' activation operands (h13, act) and gu in the T16 layout, which makes their loads contiguous
            h13=take((R16, K), torch.float16), gu=take((R16, 2 * I), torch.float16), act=take((R16, I), torch.float16),
            # the combine mode's per-route fp32 rows of the down projection
            partial=take((R, K), torch.float32) if scatter == "combine" else None)
    return plan


def grouped_prefill(x2d: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, layer, limit: float,
                    stage_events: list | None = None, scatter: str | None = None,
                    rows_per_tile: int | None = None, thin_tiles: bool | None = None,
                    out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """x2d [T, K] (any float dtype), ids [T, topk] (int64 or int32), weights [T, topk] -> out [T, K] fp32.
    Restates kernel/exl3_grouped_runtime.py:50-83 with the route sort on the GPU (sort_routes).
    stage_events: if a list is given, a timing event recorded on the current stream after each stage is appended
    as (stage name, event), after a leading ("start", event).
    scatter: "atomic", "combine" or "auto" (default: EXL3_GROUPED_SCATTER, else "auto"; resolve_scatter).
    thin_tiles: run each expert's last tile of <= 64 rows on the thin GEMM kernel (default: EXL3_GROUPED_THIN, else
    on). Same arithmetic per row, so the same result.
    out_dtype (new): return out in this dtype (bf16 or fp16), as out.to(out_dtype) of the fp32 result would; the combine
    method writes it directly (no fp32 round trip through memory), the atomic scatter casts its fp32 target."""
    gp = _load_ext()

    def mark(name):
        if stage_events is not None:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            stage_events.append((name, ev))

    mark("start")
    dev = x2d.device
    T, K = x2d.shape
    topk = ids.shape[1]
    R = T * topk
    scatter = resolve_scatter(scatter, R)
    E = int(layer.w13_trellis.shape[0])
    I = int(layer._exl3_intermediate_local)
    x16 = x2d.to(torch.float16).contiguous()
    ids = ids.contiguous()
    weights = weights.contiguous()
    # row tiles of `tr` rows of one expert: each decoded trellis tile feeds up to `tr` rows of MFMA work
    # (the reference's 128-row block table is build_blocks; the GEMM accepts either)
    tr = rows_per_tile or tile_rows()
    if tr not in TILE_ROWS_CHOICES:
        raise RuntimeError(f"rows_per_tile must be one of {TILE_ROWS_CHOICES}, got {tr}")
    thin = thin_tiles_enabled() if thin_tiles is None else thin_tiles
    B = _prefill_buffers(dev, _prefill_plan(gp, T, K, topk, E, I, tr, scatter, thin))
    token_sorted, weight_sorted, expert_of_row = B["token_sorted"], B["weight_sorted"], B["expert_of_row"]
    counts, expert_row0, route_index = B["counts"], B["expert_row0"], B["route_index"]
    block_expert, block_row0, meta = B["block_expert"], B["block_row0"], B["meta"]
    out = None
    if thin:
        # the sort and the two tile tables (each expert's last tile of <= 64 rows goes to a second table, run by the
        # thin kernel) in two launches; the fp32 output the atomic down scatter adds into is cleared by the gate|up
        # launch, whose MFMA-bound workgroups hide the stores
        thin_expert, thin_row0 = B["thin_expert"], B["thin_row0"]
        out = torch.empty(T, K, dtype=torch.float32, device=dev) if scatter == "atomic" else None
        gp.sort_routes_split_tiles(ids, weights, E, token_sorted, weight_sorted, expert_of_row, counts, expert_row0,
                                   block_expert, block_row0, thin_expert, thin_row0, meta, tr, THIN_ROWS,
                                   workspace=B["sort_ws"], route_index=route_index)
        mark("sort_routes")                               # sort and tile tables
    else:
        gp.sort_routes(ids, weights, E, token_sorted, weight_sorted, expert_of_row, counts, expert_row0,
                       workspace=B["sort_ws"], route_index=route_index)
        mark("sort_routes")
        gp.build_tiles(counts, block_expert, block_row0, meta, tr)
        mark("build_blocks")
    h13 = B["h13"]
    gp.row_had(x16, h13, token_sorted, expert_of_row, layer.w13_suh[:, 0], True, dst_layout=1, rows=R)
    mark("row_had")
    gu = B["gu"]
    w13 = (layer.w13_trellis[:, 0], layer.w13_trellis[:, 1], layer.w13_svh[:, 0], layer.w13_svh[:, 1])
    gp.grouped_gemm(h13, *w13, block_expert, block_row0, counts, expert_row0, token_sorted, weight_sorted, gu, 4,
                    tile_rows=tr, a_layout=1, a_rows=R, zero=out if thin else None)
    if thin:
        gp.grouped_gemm(h13, *w13, thin_expert, thin_row0, counts, expert_row0, token_sorted, weight_sorted, gu, 4,
                        tile_rows=THIN_ROWS, a_layout=1, a_rows=R)
    mark("gemm_gate_up")
    act = B["act"]
    gp.act_had(gu, act, expert_of_row, layer.w2_suh, float(limit), dst_layout=1, gu_layout=1, rows=R)
    mark("act_had")
    if scatter == "atomic":
        if out is None:
            out = torch.zeros(T, K, dtype=torch.float32, device=dev)
            mark("zero_out")
        gp.grouped_gemm(act, layer.w2_trellis, None, layer.w2_svh, None,
                        block_expert, block_row0, counts, expert_row0, token_sorted, weight_sorted, out, 1,
                        tile_rows=tr, a_layout=1, a_rows=R)
        if thin:
            gp.grouped_gemm(act, layer.w2_trellis, None, layer.w2_svh, None,
                            thin_expert, thin_row0, counts, expert_row0, token_sorted, weight_sorted, out, 1,
                            tile_rows=THIN_ROWS, a_layout=1, a_rows=R)
        mark("gemm_down_scatter")
        return out if out_dtype is None else out.to(out_dtype)
    partial = B["partial"]
    gp.grouped_gemm(act, layer.w2_trellis, None, layer.w2_svh, None,
                    block_expert, block_row0, counts, expert_row0, None, weight_sorted, partial, 2,
                    route_index=route_index, tile_rows=tr, a_layout=1, a_rows=R)
    if thin:
        gp.grouped_gemm(act, layer.w2_trellis, None, layer.w2_svh, None,
                        thin_expert, thin_row0, counts, expert_row0, None, weight_sorted, partial, 2,
                        route_index=route_index, tile_rows=THIN_ROWS, a_layout=1, a_rows=R)
    mark("gemm_down_routes")
    direct = out_dtype in (torch.bfloat16, torch.float16)
    out = torch.empty(T, K, dtype=out_dtype if direct else torch.float32, device=dev)
    gp.combine_routes(partial, out, topk, ids, E)
    mark("combine")
    return out if direct or out_dtype is None else out.to(out_dtype)


def grouped_prefill_from_logits(x2d: torch.Tensor, router_logits: torch.Tensor, layer, limit: float,
                                e_score_correction_bias: torch.Tensor | None = None, topk: int = 8,
                                routed_scaling_factor: float = 2.5, renormalize: bool = True,
                                scatter: str | None = None) -> torch.Tensor:
    """The router glue in front of grouped_prefill, on the GPU (new): GLM-5.3-Flash's noaux_tc top-k (sigmoid scores,
    biased selection, renormalised un-biased weights x routed_scaling_factor) straight into the route sort and the
    grouped path. router_logits [T, E] as the gate linear produced them (fp32, fp16 or bf16)."""
    gp = _load_ext()
    ids, weights = gp.route_topk(router_logits, e_score_correction_bias, topk, routed_scaling_factor, renormalize)
    return grouped_prefill(x2d, ids, weights, layer, limit, scatter=scatter)


def decode_enabled() -> bool:
    return os.environ.get("EXL3_GROUPED_DECODE", "1") != "0"


# One decode workspace per device, shared by every MoE layer (layers run one after another on one stream). It is
# allocated once, by the first decode call on the device (or reserve_decode_workspace), and never replaced: a graph
# captured later keeps its address, so a later call that would need a larger one raises instead of swapping buffers.
_decode_ws: dict = {}


def reserve_decode_workspace(device, tokens: int, topk: int, n_experts: int, hidden: int, inter: int) -> torch.Tensor:
    """Allocate the device's decode workspace for batches of up to `tokens` (the wrapper sizes it for the overlay's
    row cap on the first decode call; call this before any graph capture to size it explicitly). Returns it; raises if
    the device already has a smaller one (its address may be captured in a graph)."""
    gp = _load_ext()
    dev = torch.device(device)
    need = gp.moe_decode_workspace_bytes(int(tokens), int(topk), int(n_experts), int(hidden), int(inter))
    key = _device_index(dev)
    ws = _decode_ws.get(key)
    if ws is None:
        ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        _decode_ws[key] = ws
        logger.info("EXL3 decode workspace: %.1f MiB on cuda:%d (%d tokens x top-%d, E=%d, H=%d, I=%d)",
                    ws.numel() / 2**20, key, tokens, topk, n_experts, hidden, inter)
    elif ws.numel() < need:
        raise RuntimeError(f"the decode workspace of cuda:{key} holds {ws.numel()} bytes, this call needs {need} "
                           f"({tokens} tokens x top-{topk}); it is never reallocated (a captured graph may hold its "
                           "address): size it for the largest batch with reserve_decode_workspace before first use")
    return ws


def moe_decode(x2d: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, layer, limit: float,
               out: torch.Tensor | None = None, cap: int | None = None) -> torch.Tensor:
    """Decode-path MoE for a small batch: x2d [T, H] (any float dtype), ids [T, topk], weights [T, topk] -> out fp32
    [T, H]. The workspace is the device's shared one (reserve_decode_workspace), sized on the first call for
    max(T, cap) tokens and never reallocated, so a call allocates nothing when `out` is given (the first call on a
    device should run before a graph capture)."""
    gp = _load_ext()
    T, H = x2d.shape
    topk = ids.shape[1]
    E = int(layer.w13_trellis.shape[0])
    I = int(layer._exl3_intermediate_local)
    ws = reserve_decode_workspace(x2d.device, max(T, int(cap or 0)), topk, E, H, I)
    x16 = x2d if x2d.dtype == torch.float16 and x2d.is_contiguous() else x2d.to(torch.float16).contiguous()
    return gp.moe_decode(x16, ids.contiguous(), weights.contiguous(), layer.w13_trellis, layer.w13_suh,
                         layer.w13_svh, layer.w2_trellis, layer.w2_suh, layer.w2_svh, float(limit), out=out,
                         workspace=ws)


def install(ov):
    """Wrap ov.apply_exl3_experts: prefill-sized calls use the grouped path; everything else is untouched
    (kernel/exl3_grouped_runtime.py:86-112)."""
    global _logged
    original = ov.apply_exl3_experts

    def apply_exl3_experts_grouped(x, topk_ids, topk_weights, layer, *, limit=ov.SWIGLU_LIMIT_DEFAULT, fused=None):
        global _logged
        tokens = x.shape[-2]
        temps = getattr(layer, "_exl3_fused_temps", None)
        cap = int(temps[0].shape[1]) if temps else 0
        expert_map = getattr(layer, "expert_map", None)
        if expert_map is not None or not hasattr(layer, "w13_trellis") or (tokens <= cap and not decode_enabled()):
            return original(x, topk_ids, topk_weights, layer, limit=limit, fused=fused)
        x2d = x.reshape(tokens, x.shape[-1])
        ids = topk_ids.reshape(tokens, -1).to(torch.long)
        weights = topk_weights.reshape(tokens, -1)
        if tokens <= cap:
            out = moe_decode(x2d, ids, weights, layer, float(limit), cap=cap)
            layer._exl3_last_apply = "decode"
            return out.to(dtype=x.dtype)
        # the output in x.dtype straight from the combine pass where it runs (the same values as out.to(x.dtype))
        out = grouped_prefill(x2d, ids, weights, layer, float(limit), out_dtype=x.dtype)
        layer._exl3_last_apply = "grouped"
        if not _logged:
            logger.info("EXL3 grouped prefill engaged (tokens=%d > cap=%d, experts=%d)", tokens, cap,
                        int(layer.w13_trellis.shape[0]))
            _logged = True
        return out.to(dtype=x.dtype)

    ov.apply_exl3_experts = apply_exl3_experts_grouped
    # the MoE method's apply() looks the function up at call time from the module globals, so the wrap sticks
    _load_ext()  # load at boot rather than on the first prefill
    logger.info("EXL3 grouped prefill installed (EXL3_GROUPED_PREFILL=1)")
