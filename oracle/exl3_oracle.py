"""CPU oracle for the EXL3 grouped routed-expert MoE prefill path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, and
there only as the checker (or the timed CPU baseline). The product path never imports it.

Two layers:
  * exl3_oracle.c (via ctypes): bit-level trellis decode, route sort, block table, fp16 rounding.
  * numpy (this file): the floating-point stages, restated kernel by kernel with the reference's rounding
    points, and the reference's per-expert loop.

Reference citations (paths relative to the reference repository):
  row_had      kernel/exl3_grouped_prefill.cu:101-115  h13[r] = fp16(H128(x[tok_r] * suh_gate[e_r]) / sqrt(128))
  act_had      kernel/exl3_grouped_prefill.cu:118-141  a = fp16(silu(min(g,L)) * clamp(u,-L,L)); act = fp16(H128(a*suh_down)/sqrt(128))
  grouped_gemm kernel/exl3_grouped_prefill.cu:148-279  mode 0: gu = fp16(H128_n(h13 @ W') / sqrt(128) * svh)
                                                        mode 1: out[tok] += fp32(w16) * H128_n(act @ W'_down)/sqrt(128) * svh
  fat gemm     kernel/exl3_fat_gemm_v2.cu:195-233      fp32 out (store) or out[tok] += fp32(w16) * y (scatter)
  expert loop  harness/proto_fp8.py:123-134 with the weight convention of :66-76
               (W = diag(suh) H W' H diag(svh)), evaluated in factored form.
Parity against exllamav3 itself (codebook constants, stream bit order, H128 rounding sequence) is unpinned:
exllamav3 and the overlay's apply_exl3_python_loop are not present (see exl3_oracle.c's header).
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

HAD_SCALE = 0.088388347648  # 1/sqrt(128) as the reference writes it (kernel/exl3_grouped_prefill.cu:43)
SWIGLU_LIMIT_DEFAULT = 10.0  # docs/research/02-glm-5.3-flash-architecture.md:33


def lib():
    """The C half of the oracle (built by oracle/Makefile)."""
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run `make -C oracle`)")
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16_array.argtypes = [P, P, ctypes.c_int64]
        L.orc_f16_to_f32_array.argtypes = [P, P, ctypes.c_int64]
        L.orc_decode_state_mcg.restype = ctypes.c_uint16
        L.orc_decode_state_mcg.argtypes = [ctypes.c_uint32]
        L.orc_decode_lut.argtypes = [P]
        L.orc_tile_states.argtypes = [P, ctypes.c_int, P]
        L.orc_tile_pos_to_kn.argtypes = [ctypes.c_int, P, P]
        L.orc_pack_tile.argtypes = [P, ctypes.c_int, P]
        L.orc_reconstruct.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]
        L.orc_sort_routes.restype = ctypes.c_int
        L.orc_sort_routes.argtypes = [P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, P, P, P, P, P]
        L.orc_build_blocks.argtypes = [P, ctypes.c_int, ctypes.c_int, P, P, P]
        L.orc_build_tiles.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P]
        _LIB = L
    return _LIB


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------------------------------------- fp16
def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 bits (uint16), round to nearest even, through the C restatement."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def round_f16(x: np.ndarray) -> np.ndarray:
    """Round values to the nearest fp16 and return them as float32 (numpy's float16 cast is RNE)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


# ---------------------------------------------------------------------------------------------- trellis
def decode_lut() -> np.ndarray:
    """fp16 bits of decode(state) for all 65536 states."""
    out = np.empty(65536, dtype=np.uint16)
    lib().orc_decode_lut(_p(out))
    return out


def tile_states(words: np.ndarray, bits: int) -> np.ndarray:
    w = np.ascontiguousarray(words, dtype=np.uint16).reshape(-1)
    assert w.size == 16 * bits
    out = np.empty(256, dtype=np.uint16)
    lib().orc_tile_states(_p(w), bits, _p(out))
    return out


def tile_pos_to_kn(p: int) -> tuple[int, int]:
    k = ctypes.c_int()
    n = ctypes.c_int()
    lib().orc_tile_pos_to_kn(p, ctypes.byref(k), ctypes.byref(n))
    return k.value, n.value


def pack_tile(symbols: np.ndarray, bits: int) -> np.ndarray:
    s = np.ascontiguousarray(symbols, dtype=np.uint8).reshape(-1)
    assert s.size == 256
    out = np.empty(16 * bits, dtype=np.uint16)
    lib().orc_pack_tile(_p(s), bits, _p(out))
    return out


def reconstruct(packed: np.ndarray) -> np.ndarray:
    """packed [tiles_k, tiles_n, 16*bits] (int16 or uint16) -> W' as float16 [tiles_k*16, tiles_n*16]."""
    p = np.ascontiguousarray(packed).view(np.uint16)
    tk, tn, words = p.shape
    assert words % 16 == 0
    bits = words // 16
    out = np.empty((tk * 16, tn * 16), dtype=np.uint16)
    lib().orc_reconstruct(_p(p), tk, tn, bits, _p(out))
    return out.view(np.float16)


# ---------------------------------------------------------------------------------------------- routing
def sort_routes(ids: np.ndarray, weights: np.ndarray, n_experts: int):
    """Stable sort of routes by expert: kernel/exl3_grouped_runtime.py:59-68."""
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    T, topk = ids.shape
    w = np.ascontiguousarray(weights, dtype=np.float32).reshape(T, topk)
    R = T * topk
    token_sorted = np.empty(R, dtype=np.int64)
    weight_sorted = np.empty(R, dtype=np.uint16)
    expert_of_row = np.empty(R, dtype=np.int32)
    counts = np.empty(n_experts, dtype=np.int32)
    expert_row0 = np.empty(n_experts, dtype=np.int32)
    rc = lib().orc_sort_routes(_p(ids), _p(w), T, topk, n_experts, _p(token_sorted), _p(weight_sorted),
                               _p(expert_of_row), _p(counts), _p(expert_row0))
    if rc != 0:
        raise ValueError("expert id out of range")
    return token_sorted, weight_sorted.view(np.float16), expert_of_row, counts, expert_row0


def route_topk(logits: np.ndarray, bias, topk: int, scale: float, renorm: bool = True):
    """GLM-5.3-Flash noaux_tc router (docs/research/02-glm-5.3-flash-architecture.md:33): s = sigmoid(logit) in fp32;
    the topk experts with the largest s + bias in decreasing order, ties to the lower expert id; weights = s / sum(s)
    * scale (sum in selection order, fp32) or s * scale. Returns (ids int64 [T, k], weights fp32 [T, k])."""
    lg = np.asarray(logits, np.float32).astype(np.float64)
    s = (1.0 / (1.0 + np.exp(-lg))).astype(np.float32)
    sel = s + (np.asarray(bias, np.float32) if bias is not None else np.float32(0))
    order = np.argsort(-sel, axis=1, kind="stable")[:, :topk]
    sc = np.take_along_axis(s, order, axis=1)
    w = np.empty_like(sc)
    for t in range(sc.shape[0]):
        tot = np.float32(0)
        for j in range(topk):
            tot = np.float32(tot + sc[t, j])
        w[t] = (sc[t] / tot * np.float32(scale)) if renorm else sc[t] * np.float32(scale)
    return order.astype(np.int64), w.astype(np.float32)


def build_blocks(counts: np.ndarray, max_blocks: int, init: int = 0, tile_rows: int = 128):
    """kernel/exl3_grouped_prefill.cu:63-96 (128-row blocks; other tile sizes for the 256-row schedule);
    block_row0 past n_blocks keeps `init`."""
    counts = np.ascontiguousarray(counts, dtype=np.int32)
    be = np.full(max_blocks, init, dtype=np.int32)
    br = np.full(max_blocks, init, dtype=np.int32)
    meta = np.zeros(2, dtype=np.int32)
    if tile_rows == 128:
        lib().orc_build_blocks(_p(counts), counts.size, max_blocks, _p(be), _p(br), _p(meta))
    else:
        lib().orc_build_tiles(_p(counts), counts.size, tile_rows, max_blocks, _p(be), _p(br), _p(meta))
    return be, br, meta


# ---------------------------------------------------------------------------------------------- Hadamard
def sylvester(n: int) -> np.ndarray:
    """Sylvester Hadamard matrix [[h, h], [h, -h]] of order n (entries +-1), as in harness/proto_fp8.py:61-64."""
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


_H128 = sylvester(128)


def had128(x: np.ndarray, scale: float = HAD_SCALE) -> np.ndarray:
    """H128 along the last axis in blocks of 128, times `scale`; computed in float64."""
    x = np.asarray(x, dtype=np.float64)
    sh = x.shape
    assert sh[-1] % 128 == 0
    y = x.reshape(-1, 128) @ _H128          # one [n, 128] x [128, 128] product, not a batch of small ones
    y *= scale
    return y.reshape(sh)


# ---------------------------------------------------------------------------------------------- layer
@dataclass
class Layer:
    """Stacked EXL3 expert tensors of one TP rank, attribute names and layouts as the vLLM layer carries them
    (kernel/test_grouped.py:76-81). Arrays are numpy; fp16 tensors are float16, trellis tensors int16."""
    w13_trellis: np.ndarray  # [E, 2, H/16, I/16, 16*bits]
    w13_suh: np.ndarray      # [E, 2, H]
    w13_svh: np.ndarray      # [E, 2, I]
    w2_trellis: np.ndarray   # [E, I/16, H/16, 16*bits]
    w2_suh: np.ndarray       # [E, I]
    w2_svh: np.ndarray       # [E, H]

    @property
    def n_experts(self):
        return self.w13_trellis.shape[0]

    @property
    def hidden(self):
        return self.w13_trellis.shape[2] * 16

    @property
    def intermediate(self):
        return self.w13_trellis.shape[3] * 16


class WeightCache:
    """Lazily reconstructed W' (float32) per (expert, matrix)."""

    def __init__(self, layer: Layer):
        self.layer = layer
        self._c = {}

    def get(self, e: int, which: str) -> np.ndarray:
        key = (e, which)
        if key not in self._c:
            if which == "gate":
                t = self.layer.w13_trellis[e, 0]
            elif which == "up":
                t = self.layer.w13_trellis[e, 1]
            else:
                t = self.layer.w2_trellis[e]
            self._c[key] = reconstruct(t).astype(np.float32)
        return self._c[key]


def row_had(src: np.ndarray, token_sorted, expert_of_row, suh: np.ndarray, gather: bool) -> np.ndarray:
    """kernel/exl3_grouped_prefill.cu:101-115. src fp16 [*, K]; suh [E, K] -> fp16 [rows, K]."""
    rows = src[token_sorted] if gather else src
    y = had128(rows.astype(np.float32) * suh[expert_of_row].astype(np.float32))
    return y.astype(np.float32).astype(np.float16)


def swiglu_clamped(g: np.ndarray, u: np.ndarray, limit: float) -> np.ndarray:
    """silu(min(g, L)) * clamp(u, -L, L) in fp32 (kernel/exl3_grouped_prefill.cu:133-135)."""
    g = np.minimum(g.astype(np.float32), np.float32(limit))
    u = np.clip(u.astype(np.float32), -np.float32(limit), np.float32(limit))
    with np.errstate(over="ignore"):
        return (g / (np.float32(1.0) + np.exp(-g))) * u


def act_had(gu: np.ndarray, expert_of_row, suh_down: np.ndarray, limit: float) -> np.ndarray:
    """kernel/exl3_grouped_prefill.cu:118-141. gu fp16 [rows, 2I] -> act fp16 [rows, I]."""
    I = gu.shape[1] // 2
    a = swiglu_clamped(gu[:, :I], gu[:, I:], limit).astype(np.float16).astype(np.float32)
    y = had128(a * suh_down[expert_of_row].astype(np.float32))
    return y.astype(np.float32).astype(np.float16)


def expert_gemm(a_rows: np.ndarray, w: np.ndarray, svh: np.ndarray, dtype=np.float64) -> np.ndarray:
    """H128_n(a @ W') / sqrt(128) * svh for one expert, unrounded (float64 by default)."""
    y = a_rows.astype(dtype) @ w.astype(dtype)
    return had128(y) * svh.astype(np.float64)


def grouped_gemm_mode0(h13, cache: WeightCache, counts, expert_row0, dtype=np.float64) -> np.ndarray:
    """gate|up stage: fp16 [rows, 2I]."""
    L = cache.layer
    I = L.intermediate
    out = np.zeros((h13.shape[0], 2 * I), dtype=np.float16)
    for e in np.nonzero(counts)[0]:
        r0, c = int(expert_row0[e]), int(counts[e])
        a = h13[r0:r0 + c]
        out[r0:r0 + c, :I] = expert_gemm(a, cache.get(e, "gate"), L.w13_svh[e, 0], dtype).astype(np.float32).astype(np.float16)
        out[r0:r0 + c, I:] = expert_gemm(a, cache.get(e, "up"), L.w13_svh[e, 1], dtype).astype(np.float32).astype(np.float16)
    return out


def grouped_gemm_mode1(act, cache: WeightCache, counts, expert_row0, token_sorted, weight_sorted, T,
                       dtype=np.float64) -> np.ndarray:
    """down stage with scatter: out fp32 [T, H] += fp32(w16) * y."""
    L = cache.layer
    out = np.zeros((T, L.hidden), dtype=np.float64)
    for e in np.nonzero(counts)[0]:
        r0, c = int(expert_row0[e]), int(counts[e])
        y = expert_gemm(act[r0:r0 + c], cache.get(e, "down"), L.w2_svh[e], dtype)
        y = y * weight_sorted[r0:r0 + c].astype(np.float64)[:, None]
        np.add.at(out, token_sorted[r0:r0 + c], y)
    return out.astype(np.float32)


def grouped_prefill(x: np.ndarray, ids: np.ndarray, weights: np.ndarray, layer: Layer, limit: float,
                    cache: WeightCache | None = None, dtype=np.float64, return_stages: bool = False):
    """Stage-by-stage restatement of grouped_prefill (kernel/exl3_grouped_runtime.py:50-83)."""
    cache = cache or WeightCache(layer)
    E = layer.n_experts
    T = x.shape[0]
    x16 = np.asarray(x).astype(np.float16)
    ts, ws, eor, counts, row0 = sort_routes(ids, weights, E)
    h13 = row_had(x16, ts, eor, layer.w13_suh[:, 0], True)
    gu = grouped_gemm_mode0(h13, cache, counts, row0, dtype)
    act = act_had(gu, eor, layer.w2_suh, limit)
    out = grouped_gemm_mode1(act, cache, counts, row0, ts, ws, T, dtype)
    if return_stages:
        return out, dict(token_sorted=ts, weight_sorted=ws, expert_of_row=eor, counts=counts, expert_row0=row0,
                         h13=h13, gu=gu, act=act)
    return out


def expert_loop(x: np.ndarray, ids: np.ndarray, weights: np.ndarray, layer: Layer, limit: float,
                cache: WeightCache | None = None, experts=None, dtype=np.float32, round_h13: bool = False,
                round_act: bool = False) -> np.ndarray:
    """The reference's per-expert loop (harness/proto_fp8.py:123-134) on the real-domain weights
    W = diag(suh) H W' H diag(svh) (:66-76), evaluated in factored form: x @ W = H((x*suh) H @ W') * svh.
    Rounding points: h = fp16 input rows, gate|up fp16, act fp16, route weight fp16; fp32 output.
    `experts` restricts the loop to a subset (the CPU-baseline sample).
    round_h13 / round_act add the grouped path's two extra fp16 rounding points, the rotated input rows (row_had,
    kernel/exl3_grouped_prefill.cu:101-115) and the rotated activation (act_had, :118-141); with both the loop computes
    what the staged path does, so the two flags split the staged path's distance from the loop between them."""
    cache = cache or WeightCache(layer)
    T = x.shape[0]
    H = layer.hidden
    x16 = np.asarray(x).astype(np.float16).astype(np.float32)
    w16 = np.asarray(weights, dtype=np.float32).astype(np.float16).astype(np.float32)
    out = np.zeros((T, H), dtype=np.float32)
    exps = range(layer.n_experts) if experts is None else experts
    for e in exps:
        tok, kpos = np.nonzero(ids == e)
        if tok.size == 0:
            continue
        h = x16[tok]
        hs = had128(h * layer.w13_suh[e, 0].astype(np.float32)).astype(dtype)
        if round_h13:
            hs = round_f16(hs).astype(dtype)
        gate = had128(hs @ cache.get(e, "gate").astype(dtype)) * layer.w13_svh[e, 0].astype(np.float32)
        same_suh = np.array_equal(layer.w13_suh[e, 0], layer.w13_suh[e, 1])
        hs_u = hs if same_suh else had128(h * layer.w13_suh[e, 1].astype(np.float32)).astype(dtype)
        if round_h13 and not same_suh:
            hs_u = round_f16(hs_u).astype(dtype)
        up = had128(hs_u @ cache.get(e, "up").astype(dtype)) * layer.w13_svh[e, 1].astype(np.float32)
        gate = round_f16(gate)
        up = round_f16(up)
        act = round_f16(swiglu_clamped(gate, up, limit))
        a = had128(act * layer.w2_suh[e].astype(np.float32)).astype(dtype)
        if round_act:
            a = round_f16(a).astype(dtype)
        down = had128(a @ cache.get(e, "down").astype(dtype)) * layer.w2_svh[e].astype(np.float32)
        v = (down * w16[tok, kpos][:, None]).astype(np.float32)
        if np.unique(tok).size == tok.size:    # top-k ids are distinct per token: one add per output element
            out[tok] += v
        else:
            np.add.at(out, tok, v)
    return out


def fat_gemm(a: np.ndarray, packed: np.ndarray, svh: np.ndarray, dtype=np.float64) -> np.ndarray:
    """Per-expert entry (kernel/exl3_fat_gemm_v2.cu:195-233, test reference kernel/test_fat_v2.py:87-95):
    reconstruct -> matmul -> H128 * svh, fp32 out."""
    w = reconstruct(packed).astype(np.float32)
    return expert_gemm(a, w, svh, dtype).astype(np.float32)


def linear(x: np.ndarray, packed: np.ndarray, suh: np.ndarray, svh: np.ndarray, out_dtype=np.float32,
           dtype=np.float64) -> np.ndarray:
    """Dense EXL3 linear, the LinearEXL3 forward on the real-domain weight diag(suh) H W' H diag(svh)
    (harness/proto_fp8.py:66-76) in factored form with the expert GEMM's rounding points: h = fp16(H128(x * suh)),
    y = H128(h @ W') * svh accumulated in fp32 or wider, then rounded to out_dtype."""
    rows = np.asarray(x).shape[0]
    h = row_had(np.asarray(x), None, np.zeros(rows, np.int64), np.asarray(suh)[None, :], False)
    return fat_gemm(h, packed, svh, dtype).astype(out_dtype)


def fat_gemm_scatter(a, packed, svh, token_idx, route_weight, out, dtype=np.float64) -> np.ndarray:
    """out[token_idx[m]] += fp32(route_weight[m]) * y[m] (kernel/exl3_fat_gemm_v2.cu:221-226; reference
    check kernel/test_fat_v2.py:135 uses index_add_)."""
    y = fat_gemm(a, packed, svh, dtype).astype(np.float64) * np.asarray(route_weight, np.float64)[:, None]
    o = np.asarray(out, dtype=np.float64).copy()
    np.add.at(o, np.asarray(token_idx), y)
    return o.astype(np.float32)


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
