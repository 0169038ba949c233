"""GPU parity of the decode path: moe_decode (the `tokens <= cap` side of kernel/exl3_grouped_runtime.py:93-98,
where the reference calls the overlay's fused exl3_moe) and its building blocks, the split-K grouped GEMM and the
fp32-input act_had.

Bars: the north-star rel L2 <= 1e-3 against the oracle expert loop (harness/proto_fp8.py:123-134 restated in
oracle/exl3_oracle.py); exact equality where the arithmetic is the same (fp32 act_had input rounded to fp16, a
one-slice mode-3 GEMM against the fp16 store); fp32 accumulation-order bounds where only the order of additions
differs (K slices, atomics). Graph capture: replays with fresh inputs against eager calls.
"""
import functools

import numpy as np
import pytest
import torch

import exl3_grouped as gp
import exl3_grouped_runtime as rt
import exl3_oracle as O
from exl3_grouped import synth

pytestmark = pytest.mark.gpu
LIMIT = 10.0
# Two runs of the decode op on the same inputs: the K slices add into gate|up with fp32 atomics in a varying order, so
# an fp16 rounding of gu can land one step apart between runs (like the reference's atomic scatter, the op is not
# bit-reproducible); the outputs then differ by ~1e-5 relative.
RERUN_TOL = 1e-4


def to_np_layer(L):
    return O.Layer(L.w13_trellis, L.w13_suh, L.w13_svh, L.w2_trellis, L.w2_suh, L.w2_svh)


def dt(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@functools.lru_cache(maxsize=6)
def layer_case(name, bits=None, svh_scale=1.0, seed=0):
    """A layer of config `name` (weights only) on the host and on the GPU."""
    L, _, _, _, cfg = synth.make_config(name, seed=seed, T=1, bits=bits, svh_scale=svh_scale)
    return L, cfg


@functools.lru_cache(maxsize=6)
def device_layer(name, bits=None, svh_scale=1.0, seed=0):
    L, cfg = layer_case(name, bits, svh_scale, seed)
    return synth.to_device(L, torch.device("cuda:0"))


def inputs(cfg, T, seed, routing="softmax"):
    x = synth.make_x(T, cfg["H"], seed)
    ids, w = synth.make_routing(routing, T, cfg["E"], cfg["topk"], seed=seed)
    return x, ids, w


def decode(TL, x, ids, w, dev, **kw):
    out = gp.moe_decode(dt(x, dev).to(torch.float16), dt(ids, dev), dt(w, dev), TL.w13_trellis, TL.w13_suh,
                        TL.w13_svh, TL.w2_trellis, TL.w2_suh, TL.w2_svh, LIMIT, **kw)
    torch.cuda.synchronize()
    return out


# ------------------------------------------------------------------------------------------- building blocks
def test_act_had_f32_equals_fp16_input(dev):
    rng = np.random.default_rng(3)
    R, I, E = 77, 768, 5
    gu32 = torch.from_numpy((rng.standard_normal((R, 2 * I)) * 6).astype(np.float32)).to(dev)
    eor = dt(rng.integers(0, E, R).astype(np.int32), dev)
    suh = dt(np.where(rng.random((E, I)) < 0.5, -1.0, 1.0).astype(np.float16), dev)
    a32 = torch.full((gp.t16_rows(R), I), float("nan"), dtype=torch.float16, device=dev)
    a16 = torch.full_like(a32, float("nan"))
    gp.act_had(gu32, a32, eor, suh, LIMIT, dst_layout=1)
    gp.act_had(gu32.half(), a16, eor, suh, LIMIT, dst_layout=1)
    assert torch.equal(a32.view(torch.int16), a16.view(torch.int16))      # bitwise; unwritten T16 padding is NaN


def closed_form_sort(ids, w, E):
    """Stable sort of routes by expert with out-of-range ids moved to the tail as (token 0, weight 0, expert 0): the
    semantics of the route sort, restated with numpy (checked against the oracle's sort where no id is dropped)."""
    flat = ids.reshape(-1)
    R, k = flat.size, ids.shape[1]
    valid = (flat >= 0) & (flat < E)
    order = np.argsort(np.where(valid, flat, E), kind="stable")
    live = np.arange(R) < valid.sum()
    ts = np.where(live, order // k, 0).astype(np.int64)
    ws = np.where(live, w.reshape(-1).astype(np.float16)[order], np.float16(0)).astype(np.float16)
    eor = np.where(live, flat[order], 0).astype(np.int32)
    counts = np.bincount(flat[valid], minlength=E).astype(np.int32)
    return ts, ws, eor, counts, (np.cumsum(counts) - counts).astype(np.int32)


@pytest.mark.parametrize("kind,T,E,k,tile_rows", [("softmax", 1, 288, 8, 128), ("softmax", 16, 288, 8, 128),
                                                  ("skewed", 256, 288, 8, 128), ("softmax", 200, 1024, 6, 64),
                                                  ("zipf", 128, 288, 8, 256), ("softmax", 2048, 8, 1, 512)])
def test_route_prep_small_bit_exact(dev, kind, T, E, k, tile_rows):
    """One launch against the stable sort and block table (kernel/exl3_grouped_prefill.cu:63-96,
    kernel/exl3_grouped_runtime.py:59-68), with int32 ids, dropped ids and bf16 weights on the side."""
    ids, w = synth.make_routing(kind, T, E, k, seed=T + E)
    wf = w.astype(np.float16).astype(np.float32)
    for g, r in zip(closed_form_sort(ids, wf, E), O.sort_routes(ids, wf, E)):
        assert np.array_equal(np.asarray(g).view(np.uint8), np.asarray(r).view(np.uint8))
    cases = [(ids, torch.int64, torch.float32)]
    if T > 3:
        dropped = ids.copy()
        dropped[3, 0] = -1
        dropped[T - 1, k - 1] = E + 3
        cases.append((dropped, torch.int32, torch.bfloat16))
    for ids_c, ids_dt, w_dt in cases:
        wt = torch.from_numpy(w).to(w_dt)
        ref = closed_form_sort(ids_c, wt.float().numpy(), E)
        R = ids_c.size
        mb = min(E, R) + R // tile_rows
        rbe, rbr, rmeta = O.build_blocks(ref[3], mb, init=-7, tile_rows=tile_rows)
        ts = torch.full((R,), -5, dtype=torch.int64, device=dev)
        ws = torch.full((R,), 7, dtype=torch.int16, device=dev).view(torch.float16)
        eor = torch.full((R,), -5, dtype=torch.int32, device=dev)
        counts = torch.full((E,), -5, dtype=torch.int32, device=dev)
        row0 = torch.full((E,), -5, dtype=torch.int32, device=dev)
        be = torch.full((mb,), -7, dtype=torch.int32, device=dev)
        br = torch.full((mb,), -7, dtype=torch.int32, device=dev)
        meta = torch.full((2,), -5, dtype=torch.int32, device=dev)
        za = torch.full((1000,), 3.0, device=dev)
        zb = torch.full((36,), 3.0, device=dev)
        gp.route_prep_small(dt(ids_c, dev).to(ids_dt), wt.to(dev), E, ts, ws, eor, counts, row0, be, br, meta,
                            tile_rows=tile_rows, zero=(za, zb))
        torch.cuda.synchronize()
        for g, r in zip((ts, ws, eor, counts, row0), ref):
            assert np.array_equal(g.cpu().numpy().view(np.uint8), np.asarray(r).view(np.uint8))
        n = int(rmeta[0])
        assert meta.tolist() == [int(v) for v in rmeta]
        assert np.array_equal(be.cpu().numpy(), rbe) and np.array_equal(br.cpu().numpy()[:n], rbr[:n])
        assert not za.any() and not zb.any()


def decode_workspace_buffers(ws, T, k, E, H, I):
    """The decode workspace's buffers by name, at the offsets exl3_moe_decode lays them out (moe_decode.hip
    decode_layout: each buffer 256-byte aligned, in this order; gu is followed by the activation pass's arrival
    counts, one int32 per (row tile, 128-column block), in the same buffer)."""
    R = T * k
    mb = min(E, R) + R // 64
    sizes = [("sort", gp.sort_routes_workspace_bytes(T, k, E)), ("ts", R * 8), ("ws", R * 2), ("eor", R * 4),
             ("counts", E * 4), ("row0", E * 4), ("be", mb * 4), ("br", mb * 4), ("meta", 8),
             ("h13", gp.t16_rows(R) * H * 2), ("gu", R * 2 * I * 4 + (mb * (I // 128) * 4 + 15) // 16 * 16),
             ("act", gp.t16_rows(R) * I * 2)]
    views, o = {}, 0
    for name, n in sizes:
        views[name] = ws[o:o + n]
        o += (n + 255) // 256 * 256
    assert ws.numel() >= o
    return views, mb


def decode_workspace_views(ws, T, k, E, H, I):
    """The decode workspace's sorted routes, tables, meta and h13."""
    R = T * k
    views, mb = decode_workspace_buffers(ws, T, k, E, H, I)
    return (views["ts"].view(torch.int64), views["ws"].view(torch.float16), views["eor"].view(torch.int32),
            views["counts"].view(torch.int32), views["row0"].view(torch.int32), views["be"].view(torch.int32),
            views["br"].view(torch.int32), views["meta"].view(torch.int32)[:2],
            views["h13"].view(torch.float16).view(gp.t16_rows(R), H), mb)


@pytest.mark.parametrize("name,T,drop", [("layer1k", 1, False), ("layer1k", 5, True), ("layer1k", 16, False),
                                         ("layer1k", 16, True), ("tiny", 1, False), ("tiny", 63, True)])
def test_decode_fused_prep_matches_separate_launches(dev, name, T, drop):
    """Up to 128 routes the decode op sorts, builds the tile table, clears and runs the input Hadamard in one launch,
    ranking each route by direct comparison. Its rows, tables and h13 must equal the closed-form stable sort, the
    block table (kernel/exl3_grouped_prefill.cu:63-96) and row_had over those rows (:101-115), bit for bit (also for
    2 routes, and 126, not a multiple of the four ids read per step, on 8 experts)."""
    L, cfg = layer_case(name, svh_scale=1 / 64)
    TL = device_layer(name, svh_scale=1 / 64)
    E, H, I, k = cfg["E"], cfg["H"], cfg["I"], cfg["topk"]
    x, ids, w = inputs(cfg, T, 40 + T)
    ids = ids.copy()
    if drop:
        ids[0, 1] = -1
        ids[T - 1, k - 1] = E + 2
    wt = torch.from_numpy(w).to(torch.bfloat16)
    R = T * k
    ws = torch.full((gp.moe_decode_workspace_bytes(T, k, E, H, I),), 0x5A, dtype=torch.uint8, device=dev)
    x16 = dt(x, dev).to(torch.float16)
    gp.moe_decode(x16, dt(ids, dev).to(torch.int32), wt.to(dev), TL.w13_trellis, TL.w13_suh, TL.w13_svh,
                  TL.w2_trellis, TL.w2_suh, TL.w2_svh, LIMIT, workspace=ws)
    torch.cuda.synchronize()
    ts, wsrt, eor, counts, row0, be, br, meta, h13, mb = decode_workspace_views(ws, T, k, E, H, I)
    ref = closed_form_sort(ids, wt.float().numpy(), E)
    for g, r in zip((ts, wsrt, eor, counts, row0), ref):
        assert np.array_equal(g.cpu().numpy().view(np.uint8), np.asarray(r).view(np.uint8))
    rbe, rbr, rmeta = O.build_blocks(ref[3], mb, init=-7, tile_rows=64)
    n = int(rmeta[0])
    assert meta.tolist() == [int(v) for v in rmeta]
    assert np.array_equal(be.cpu().numpy(), rbe) and np.array_equal(br.cpu().numpy()[:n], rbr[:n])
    h_ref = torch.zeros(gp.t16_rows(R), H, dtype=torch.float16, device=dev)
    gp.row_had(x16, h_ref, dt(ref[0], dev), dt(ref[2], dev), TL.w13_suh[:, 0], True, dst_layout=1, rows=R)
    rows = int(rmeta[1])                     # the valid rows: the tail's h13 is never read
    t16 = lambda a: a.view(-1, H // 8, 16, 8).permute(0, 2, 1, 3).reshape(-1, H)[:rows]
    assert torch.equal(t16(h13).view(torch.int16), t16(h_ref).view(torch.int16))


@pytest.mark.parametrize("name,T,drop", [("layer1k", 1, False), ("layer1k", 3, True), ("layer1k", 16, False),
                                         ("layer1k", 40, False), ("tiny", 1, False), ("tiny", 63, True)])
def test_decode_fused_act_matches_act_had(dev, name, T, drop):
    """The decode op has no activation launch. With at most 16 routes (one token) every down workgroup computes the
    act of its K slice itself from the fp32 gate|up sums (the first column block's workgroups also store it);
    otherwise the gate|up workgroup that adds the last K slice of a (row tile, 128-column block) computes that block
    of act from the finished sums. Either way the act must equal the activation pass (kernel/exl3_grouped_prefill.cu:
    118-141, here act_had over the same fp32 gu) bit for bit on every routed row -- with K split into slices (1 and 3
    tokens) and unsplit (16 and 40 tokens), dropped routes, and the tiny layer's 2 column blocks."""
    L, cfg = layer_case(name, svh_scale=1 / 64)
    TL = device_layer(name, svh_scale=1 / 64)
    E, H, I, k = cfg["E"], cfg["H"], cfg["I"], cfg["topk"]
    x, ids, w = inputs(cfg, T, 70 + T)
    ids = ids.copy()
    if drop:
        ids[0, 0] = -1
        ids[T - 1, k - 1] = E + 5
    R = T * k
    ws = torch.full((gp.moe_decode_workspace_bytes(T, k, E, H, I),), 0x5A, dtype=torch.uint8, device=dev)
    out = gp.moe_decode(dt(x, dev).to(torch.float16), dt(ids, dev), dt(w, dev).float(), TL.w13_trellis, TL.w13_suh,
                        TL.w13_svh, TL.w2_trellis, TL.w2_suh, TL.w2_svh, LIMIT, workspace=ws)
    torch.cuda.synchronize()
    views, mb = decode_workspace_buffers(ws, T, k, E, H, I)
    gu = views["gu"][:R * 2 * I * 4].view(torch.float32).view(R, 2 * I)
    act = views["act"].view(torch.float16).view(gp.t16_rows(R), I)
    eor = views["eor"].view(torch.int32)
    rows = int(views["meta"].view(torch.int32)[1].item())         # routed rows; dropped routes sit past them
    assert rows == R - (2 if drop else 0)
    ref = torch.full_like(act, float("nan"))
    gp.act_had(gu, ref, eor, TL.w2_suh, LIMIT, dst_layout=1, rows=R)
    torch.cuda.synchronize()
    t16 = lambda a: a.view(-1, I // 8, 16, 8).permute(0, 2, 1, 3).reshape(-1, I)[:rows]
    assert torch.equal(t16(act).view(torch.int16), t16(ref).view(torch.int16))
    assert torch.isfinite(out).all()


def sorted_case(cfg, T, seed, dev, tile_rows=128, routing="softmax"):
    x, ids, w = inputs(cfg, T, seed, routing)
    E = cfg["E"]
    ts, ws, eor, counts, row0 = O.sort_routes(ids, w, E)
    R = ids.size
    mb = min(E, R) + R // tile_rows
    be = torch.empty(mb, dtype=torch.int32, device=dev)
    br = torch.empty(mb, dtype=torch.int32, device=dev)
    meta = torch.zeros(2, dtype=torch.int32, device=dev)
    gp.build_tiles(dt(counts, dev), be, br, meta, tile_rows)
    return x, ids, w, (dt(ts, dev), dt(ws, dev), dt(eor, dev), dt(counts, dev), dt(row0, dev)), be, br


@pytest.mark.parametrize("tile_rows", [64, 128, 256])
@pytest.mark.parametrize("T", [1, 16, 300])
def test_split_gate_up_matches_store(dev, T, tile_rows):
    """Mode 3 (64-row tiles: the thin kernel) against the fp16 store of mode 0 on a 128-row table."""
    L, cfg = layer_case("layer1k")
    TL = device_layer("layer1k")
    x, ids, w, (ts, ws, eor, counts, row0), be, br = sorted_case(cfg, T, 11, dev, tile_rows)
    _, _, _, _, be128, br128 = sorted_case(cfg, T, 11, dev, 128)
    R, I, H = ids.size, cfg["I"], cfg["H"]
    h13 = torch.empty(gp.t16_rows(R), H, dtype=torch.float16, device=dev)
    gp.row_had(dt(x, dev).half(), h13, ts, eor, TL.w13_suh[:, 0], True, dst_layout=1, rows=R)
    weights = (TL.w13_trellis[:, 0], TL.w13_trellis[:, 1], TL.w13_svh[:, 0], TL.w13_svh[:, 1])
    args = (h13, *weights, be, br, counts, row0, None, None)
    gu16 = torch.empty(R, 2 * I, dtype=torch.float16, device=dev)
    gp.grouped_gemm(h13, *weights, be128, br128, counts, row0, None, None, gu16, 0, tile_rows=128, a_layout=1, a_rows=R)
    one = torch.zeros(R, 2 * I, dtype=torch.float32, device=dev)
    gp.grouped_gemm(*args, one, 3, tile_rows=tile_rows, a_layout=1, a_rows=R, k_split=1)
    torch.cuda.synchronize()
    # One slice: 0 + y is y, so the fp32 rows hold the store path's products before its fp16 rounding. The store path
    # may round the exact product once (mixed-precision multiply) where one.half() rounds the fp32 product again:
    # exact fp16 ties then go one step apart, nothing else.
    g = gu16.float()
    assert ((one - g).abs() <= g.abs() * 2.0 ** -11 + 2.0 ** -24).all()
    assert (one.half() != gu16).float().mean().item() < 1e-3
    for ks in (2, 5, 64):
        acc = torch.zeros_like(one)
        gp.grouped_gemm(*args, acc, 3, tile_rows=tile_rows, a_layout=1, a_rows=R, k_split=ks)
        torch.cuda.synchronize()
        assert ((acc - one).norm() / one.norm()).item() < 1e-6, ks      # fp32 sums in another order


@pytest.mark.parametrize("tile_rows", [64, 128])
@pytest.mark.parametrize("T", [1, 40])
def test_split_down_scatter_matches_unsplit(dev, T, tile_rows):
    L, cfg = layer_case("layer1k")
    TL = device_layer("layer1k")
    x, ids, w, (ts, ws, eor, counts, row0), be, br = sorted_case(cfg, T, 12, dev, tile_rows)
    R, I, H = ids.size, cfg["I"], cfg["H"]
    rng = np.random.default_rng(5)
    act = dt((rng.standard_normal((gp.t16_rows(R), I)) * 3).astype(np.float16), dev)
    outs = []
    for ks in (1, 2, 12):
        out = torch.zeros(T, H, dtype=torch.float32, device=dev)
        gp.grouped_gemm(act, TL.w2_trellis, None, TL.w2_svh, None, be, br, counts, row0, ts, ws, out, 1,
                        a_layout=1, a_rows=R, k_split=ks, tile_rows=tile_rows)
        torch.cuda.synchronize()
        outs.append(out)
    for o in outs[1:]:
        assert ((o - outs[0]).norm() / outs[0].norm()).item() < 1e-6


def test_split_rejections(dev):
    L, cfg = layer_case("tiny")
    TL = device_layer("tiny")
    x, ids, w, (ts, ws, eor, counts, row0), be, br = sorted_case(cfg, 4, 1, dev)
    R, I, H = ids.size, cfg["I"], cfg["H"]
    a = torch.zeros(gp.t16_rows(R), H, dtype=torch.float16, device=dev)
    args = (a, TL.w13_trellis[:, 0], TL.w13_trellis[:, 1], TL.w13_svh[:, 0], TL.w13_svh[:, 1], be, br, counts, row0,
            None, None)
    with pytest.raises(RuntimeError, match="k_split"):
        gp.grouped_gemm(*args, torch.zeros(R, 2 * I, dtype=torch.float16, device=dev), 0, a_layout=1, a_rows=R,
                        k_split=2)                                # a storing mode cannot take slices
    with pytest.raises(RuntimeError, match="k_split"):
        gp.grouped_gemm(*args, torch.zeros(R, 2 * I, device=dev), 3, a_layout=1, a_rows=R, k_split=H // 64 + 1)
    with pytest.raises(RuntimeError, match="mode 3"):
        gp.grouped_gemm(*args, torch.zeros(R, 2 * I, device=dev), 3, a_layout=1, a_rows=R, tile_rows=512)
    with pytest.raises(RuntimeError, match="tile_rows must be 64, 128, 256 or 512"):
        gp.grouped_gemm(*args, torch.zeros(R, I, device=dev), 2, a_layout=1, a_rows=R, tile_rows=96)


# ------------------------------------------------------------------------------------------- the decode op
@pytest.mark.parametrize("T", [1, 2, 7, 16, 24])
def test_decode_vs_expert_loop_layer1k(dev, T):
    L, cfg = layer_case("layer1k", svh_scale=1 / 64)
    TL = device_layer("layer1k", svh_scale=1 / 64)
    x, ids, w = inputs(cfg, T, 100 + T)
    got = decode(TL, x, ids, w, dev).cpu().numpy()
    ref = O.expert_loop(x, ids, w, to_np_layer(L), LIMIT)
    assert O.rel_l2(got, ref) < 1e-3
    prefill = rt.grouped_prefill(dt(x, dev), dt(ids, dev), dt(w, dev), TL, LIMIT).cpu().numpy()
    assert O.rel_l2(got, prefill) < 1e-3


@pytest.mark.parametrize("svh_scale", [1.0, 1 / 64])
@pytest.mark.parametrize("T", [1, 128])
def test_decode_vs_expert_loop_tiny(dev, T, svh_scale):
    L, cfg = layer_case("tiny", svh_scale=svh_scale)
    TL = device_layer("tiny", svh_scale=svh_scale)
    x, ids, w = inputs(cfg, T, 7)
    got = decode(TL, x, ids, w, dev).cpu().numpy()
    ref = O.expert_loop(x, ids, w, to_np_layer(L), LIMIT)
    assert O.rel_l2(got, ref) < 1e-3


@pytest.mark.parametrize("T", [1, 4])
@pytest.mark.parametrize("bits", [3, 2])
def test_decode_low_bits(dev, bits, T):
    """2/3-bit trellis through both placements of the activation pass: inside the down launch (one token, 8 routes)
    and at the end of the gate|up launch (four tokens, 32 routes)."""
    L, cfg = layer_case("layer1k", bits=bits, svh_scale=1 / 64)
    TL = device_layer("layer1k", bits=bits, svh_scale=1 / 64)
    x, ids, w = inputs(cfg, T, 20 + bits)
    got = decode(TL, x, ids, w, dev).cpu().numpy()
    assert O.rel_l2(got, O.expert_loop(x, ids, w, to_np_layer(L), LIMIT)) < 1e-3


def test_decode_skewed_rows_span_tiles(dev):
    """Every token on the same 8 experts: 200 rows per expert, two 128-row tiles each."""
    L, cfg = layer_case("layer1k", svh_scale=1 / 64)
    TL = device_layer("layer1k", svh_scale=1 / 64)
    T = 200
    x = synth.make_x(T, cfg["H"], 3)
    ids = np.tile(np.array([5, 77, 140, 141, 200, 3, 9, 287], np.int64), (T, 1))
    w = np.random.default_rng(2).random((T, 8)).astype(np.float32)
    w /= w.sum(1, keepdims=True)
    got = decode(TL, x, ids, w, dev).cpu().numpy()
    tokens = np.random.default_rng(4).choice(T, 12, replace=False)
    ref = O.expert_loop(x[tokens], ids[tokens], w[tokens], to_np_layer(L), LIMIT)
    assert O.rel_l2(got[tokens], ref) < 1e-3
    prefill = rt.grouped_prefill(dt(x, dev), dt(ids, dev), dt(w, dev), TL, LIMIT).cpu().numpy()
    assert O.rel_l2(got, prefill) < 1e-3


def test_decode_past_the_one_launch_route_prep(dev):
    """More than 2048 routes: the decode op falls back to the three-pass sort, a separate clear and the tile table."""
    L, cfg = layer_case("tiny", svh_scale=1 / 64)
    TL = device_layer("tiny", svh_scale=1 / 64)
    T = 1100                                                        # 2200 routes at top-2
    x, ids, w = inputs(cfg, T, 13)
    got = decode(TL, x, ids, w, dev).cpu().numpy()
    assert O.rel_l2(got, O.expert_loop(x, ids, w, to_np_layer(L), LIMIT)) < 1e-3
    prefill = rt.grouped_prefill(dt(x, dev), dt(ids, dev), dt(w, dev), TL, LIMIT).cpu().numpy()
    assert O.rel_l2(got, prefill) < 1e-3


def test_decode_dropped_ids_and_dtypes(dev):
    L, cfg = layer_case("tiny")
    TL = device_layer("tiny")
    x, ids, w = inputs(cfg, 24, 9)
    ids = ids.copy()
    ids[3, 1] = -1
    ids[10, 0] = cfg["E"] + 4                                       # outside [0, E): dropped like the reference loop
    wb = torch.from_numpy(w).to(torch.bfloat16)
    got = gp.moe_decode(dt(x, dev).half(), dt(ids, dev).to(torch.int32), wb.to(dev), TL.w13_trellis, TL.w13_suh,
                        TL.w13_svh, TL.w2_trellis, TL.w2_suh, TL.w2_svh, LIMIT).cpu().numpy()
    ref = O.expert_loop(x, ids, wb.float().numpy(), to_np_layer(L), LIMIT)
    assert O.rel_l2(got, ref) < 1e-3


def test_decode_empty_and_workspace_checks(dev):
    L, cfg = layer_case("tiny")
    TL = device_layer("tiny")
    H = cfg["H"]
    out = gp.moe_decode(torch.zeros(0, H, dtype=torch.float16, device=dev), torch.zeros(0, 2, dtype=torch.int64,
                        device=dev), torch.zeros(0, 2, device=dev), TL.w13_trellis, TL.w13_suh, TL.w13_svh,
                        TL.w2_trellis, TL.w2_suh, TL.w2_svh, LIMIT)
    assert out.shape == (0, H)
    x, ids, w = inputs(cfg, 3, 1)
    small = torch.empty(256, dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError, match="workspace"):
        gp.moe_decode(dt(x, dev).half(), dt(ids, dev), dt(w, dev), TL.w13_trellis, TL.w13_suh, TL.w13_svh,
                      TL.w2_trellis, TL.w2_suh, TL.w2_svh, LIMIT, workspace=small)


def test_decode_reuses_workspace_and_overwrites_out(dev):
    """Calls of different sizes on one workspace, and an out buffer holding garbage: every call starts clean."""
    L, cfg = layer_case("layer1k", svh_scale=1 / 64)
    TL = device_layer("layer1k", svh_scale=1 / 64)
    ws = torch.empty(gp.moe_decode_workspace_bytes(64, 8, cfg["E"], cfg["H"], cfg["I"]), dtype=torch.uint8,
                     device=dev)
    for T, seed in ((64, 1), (3, 2), (64, 1)):
        x, ids, w = inputs(cfg, T, seed)
        out = torch.full((T, cfg["H"]), 1e30, dtype=torch.float32, device=dev)
        got = decode(TL, x, ids, w, dev, out=out, workspace=ws)
        fresh = decode(TL, x, ids, w, dev)
        assert got.data_ptr() == out.data_ptr()
        assert ((got - fresh).norm() / fresh.norm()).item() < RERUN_TOL


def test_decode_graph_capture_replays(dev):
    """Capture one decode call in a graph; replay it on new inputs copied into the captured buffers, with eager calls
    in between, and compare every replay with an eager call on the same inputs."""
    L, cfg = layer_case("layer1k", svh_scale=1 / 64)
    TL = device_layer("layer1k", svh_scale=1 / 64)
    T, k, H = 8, cfg["topk"], cfg["H"]
    sx = torch.empty(T, H, dtype=torch.float16, device=dev)
    sids = torch.empty(T, k, dtype=torch.int64, device=dev)
    sw = torch.empty(T, k, dtype=torch.float32, device=dev)
    sout = torch.empty(T, H, dtype=torch.float32, device=dev)
    ws = torch.empty(gp.moe_decode_workspace_bytes(T, k, cfg["E"], H, cfg["I"]), dtype=torch.uint8, device=dev)

    def load(seed):
        x, ids, w = inputs(cfg, T, seed)
        sx.copy_(dt(x, dev).half())
        sids.copy_(dt(ids, dev))
        sw.copy_(dt(w, dev))
        return x, ids, w

    def call():
        gp.moe_decode(sx, sids, sw, TL.w13_trellis, TL.w13_suh, TL.w13_svh, TL.w2_trellis, TL.w2_suh, TL.w2_svh,
                      LIMIT, out=sout, workspace=ws)

    load(1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()                                                    # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for seed in (2, 3, 1, 2):
        x, ids, w = load(seed)
        g.replay()
        torch.cuda.synchronize()
        replay = sout.clone()
        eager = decode(TL, x, ids, w, dev)
        assert ((replay - eager).norm() / eager.norm()).item() < RERUN_TOL, seed
    ref = O.expert_loop(x, ids, w, to_np_layer(L), LIMIT)
    assert O.rel_l2(replay.cpu().numpy(), ref) < 1e-3


def test_runtime_decode_workspace_survives_larger_calls_after_capture(dev):
    """The runtime's decode workspace is one per device, sized on the first call for the row cap and never replaced:
    capture a call at T=8, make an eager call at a larger T <= cap, replay the graph with new inputs, and check that
    the workspace kept its address and the replay matches an eager call. A call beyond the reserved size raises."""
    L, cfg = layer_case("layer1k", svh_scale=1 / 64)
    TL = device_layer("layer1k", svh_scale=1 / 64)
    cap, T, k, H = 32, 8, cfg["topk"], cfg["H"]
    rt._decode_ws.clear()                                  # a fresh device workspace for this test
    sx = torch.empty(T, H, dtype=torch.float16, device=dev)
    sids = torch.empty(T, k, dtype=torch.int64, device=dev)
    sw = torch.empty(T, k, dtype=torch.float32, device=dev)
    sout = torch.empty(T, H, dtype=torch.float32, device=dev)

    def load(seed):
        x, ids, w = inputs(cfg, T, seed)
        sx.copy_(dt(x, dev).half())
        sids.copy_(dt(ids, dev))
        sw.copy_(dt(w, dev).float())
        return x, ids, w

    load(1)
    rt.moe_decode(sx, sids, sw, TL, LIMIT, out=sout, cap=cap)          # first call: sizes the workspace for cap
    ws_ptr = rt._decode_ws[torch.cuda.current_device()].data_ptr()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rt.moe_decode(sx, sids, sw, TL, LIMIT, out=sout, cap=cap)
    xb, idsb, wb = inputs(cfg, 24, 9)                                  # eager, larger than the captured batch
    big = rt.moe_decode(dt(xb, dev).half(), dt(idsb, dev), dt(wb, dev), TL, LIMIT, cap=cap)
    assert rt._decode_ws[torch.cuda.current_device()].data_ptr() == ws_ptr
    assert O.rel_l2(big.cpu().numpy(), O.expert_loop(xb, idsb, wb, to_np_layer(L), LIMIT)) < 1e-3
    for seed in (3, 4):
        load(seed)
        g.replay()
        torch.cuda.synchronize()
        replay = sout.clone()
        eager = rt.moe_decode(sx, sids, sw, TL, LIMIT, cap=cap)
        torch.cuda.synchronize()
        assert ((replay - eager).norm() / eager.norm()).item() < RERUN_TOL
    xc, idsc, wc = inputs(cfg, cap + 8, 5)
    with pytest.raises(RuntimeError, match="never reallocated"):
        rt.moe_decode(dt(xc, dev).half(), dt(idsc, dev), dt(wc, dev), TL, LIMIT)
    assert rt._decode_ws[torch.cuda.current_device()].data_ptr() == ws_ptr
    del g
    rt._decode_ws.clear()                                  # later tests size their own


def test_install_routes_decode_calls(dev, monkeypatch):
    L, cfg = layer_case("tiny")
    TL = device_layer("tiny")

    class Ov:
        SWIGLU_LIMIT_DEFAULT = LIMIT

        @staticmethod
        def apply_exl3_experts(*a, **k):
            return "original"

    rt.install(Ov)
    rt._decode_ws.clear()                                  # sized by this test's first decode call (cap 64)
    TL._exl3_fused_temps = [torch.zeros(1, 64)]
    x, ids, w = inputs(cfg, 48, 5)
    xb = dt(x, dev).to(torch.bfloat16)
    got = Ov.apply_exl3_experts(xb, dt(ids, dev), dt(w, dev), TL, limit=LIMIT)
    assert got.dtype == torch.bfloat16 and TL._exl3_last_apply == "decode"
    ref = rt.grouped_prefill(xb, dt(ids, dev), dt(w, dev), TL, LIMIT)
    assert O.rel_l2(got.float().cpu().numpy(), ref.to(torch.bfloat16).float().cpu().numpy()) < 1e-2
    monkeypatch.setenv("EXL3_GROUPED_DECODE", "0")
    assert Ov.apply_exl3_experts(xb, dt(ids, dev), dt(w, dev), TL) == "original"
