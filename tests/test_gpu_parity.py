"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle on the same seeded inputs.

Bars: bit-exact for integer / byte work (decode, reconstruct, route sort, block table); for floating point the
north-star tolerance rel L2 <= 1e-3 against the oracle (tighter bars are asserted where the arithmetic allows:
fp16 stage outputs may differ from the float64 oracle by one fp16 rounding step, fp32 GEMM outputs by fp32
accumulation order). At the headline size, where the full CPU loop is too slow for a test, parity is checked on
sampled tokens plus size-independent properties (linearity in the route weights, token-permutation
equivariance).
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


def to_np_layer(L):
    return O.Layer(L.w13_trellis, L.w13_suh, L.w13_svh, L.w2_trellis, L.w2_suh, L.w2_svh)


def t16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def within_f16_steps(got, ref, steps=1, frac=0.999):
    """Fraction of elements within `steps` fp16 spacings of the reference (fp16 outputs)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    spacing = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    ok = np.abs(got - ref) <= steps * spacing + 1e-7
    return ok.mean() >= frac


def to_t16(a):
    """Row-major [R, W] -> the T16 layout as a [t16_rows(R), W] array (include/exl3_grouped.h EXL3_LAYOUT_T16)."""
    R, W = a.shape
    Rp = (R + 15) // 16 * 16
    pad = np.zeros((Rp, W), a.dtype)
    pad[:R] = a
    return pad.reshape(Rp // 16, 16, W // 8, 8).transpose(0, 2, 1, 3).reshape(Rp, W)


def from_t16(t, R):
    Rp, W = t.shape
    return t.reshape(Rp // 16, W // 8, 16, 8).transpose(0, 2, 1, 3).reshape(Rp, W)[:R]


# ------------------------------------------------------------------------------------------- decode
def test_decode_states_all_65536_bit_exact(dev):
    states = torch.arange(65536, dtype=torch.int32).to(torch.int16).to(dev)
    out = torch.empty(65536, dtype=torch.int16, device=dev)
    gp.decode_states(states, out)
    got = out.cpu().numpy().view(np.uint16)
    assert np.array_equal(got, O.decode_lut())


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_reconstruct_bit_exact(dev, bits):
    rng = np.random.default_rng(100 + bits)
    for tk, tn in [(1, 1), (3, 8), (64, 48)]:
        pk = rng.integers(0, 65536, (tk, tn, 16 * bits), dtype=np.uint16).view(np.int16)
        w = torch.empty(tk * 16, tn * 16, dtype=torch.float16, device=dev)
        gp.reconstruct(w, t16(pk, dev), bits, True, False)
        assert np.array_equal(w.cpu().numpy().view(np.uint16), O.reconstruct(pk).view(np.uint16)), (tk, tn)


# ------------------------------------------------------------------------------------------- routing
ROUTINGS = [("softmax", 128, 8, 2), ("softmax", 1024, 288, 8), ("zipf", 8192, 288, 8), ("thin", 7168, 288, 8),
            ("skewed", 2048, 288, 8), ("softmax", 1, 288, 8), ("softmax", 3000, 1024, 6)]


def gpu_sort(ids_t, w_t, E, with_route_index=False):
    dev = ids_t.device
    R = ids_t.numel()
    ts = torch.empty(R, dtype=torch.int64, device=dev)
    ws = torch.empty(R, dtype=torch.float16, device=dev)
    eor = torch.empty(R, dtype=torch.int32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    row0 = torch.empty(E, dtype=torch.int32, device=dev)
    ri = torch.empty(R, dtype=torch.int32, device=dev) if with_route_index else None
    work = gp.sort_routes(ids_t, w_t, E, ts, ws, eor, counts, row0, route_index=ri)
    dropped = int(work[:4].view(torch.int32).item())
    res = (ts.cpu().numpy(), ws.cpu().numpy(), eor.cpu().numpy(), counts.cpu().numpy(), row0.cpu().numpy(), dropped)
    return res + (ri.cpu().numpy(),) if with_route_index else res


@pytest.mark.parametrize("kind,T,E,k", ROUTINGS)
def test_sort_routes_bit_exact(dev, kind, T, E, k):
    ids, w = synth.make_routing(kind, T, E, k, seed=T)
    ref = O.sort_routes(ids, w, E)
    for ids_dt in (torch.int64, torch.int32):
        got = gpu_sort(torch.from_numpy(ids).to(ids_dt).to(dev), torch.from_numpy(w).to(dev), E, True)
        assert got[5] == 0
        for g, r in zip(got[:5], ref):
            assert np.array_equal(np.asarray(g).view(np.uint8), np.asarray(r).view(np.uint8))
        assert np.array_equal(got[6], np.argsort(ids.reshape(-1), kind="stable"))       # route_index


@pytest.mark.parametrize("wdt", [torch.float16, torch.bfloat16])
def test_sort_routes_weight_dtypes(dev, wdt):
    ids, w = synth.make_routing("softmax", 500, 64, 8, seed=5)
    wt = torch.from_numpy(w).to(wdt)
    ref = O.sort_routes(ids, wt.float().numpy(), 64)
    got = gpu_sort(torch.from_numpy(ids).to(dev), wt.to(dev), 64)
    assert np.array_equal(got[1].view(np.uint16), ref[1].view(np.uint16))


def test_sort_routes_empty_and_dropped(dev):
    got = gpu_sort(torch.zeros(0, 8, dtype=torch.int64, device=dev), torch.zeros(0, 8, device=dev), 16)
    assert got[3].tolist() == [0] * 16 and got[4].tolist() == [0] * 16 and got[5] == 0
    ids = np.array([[0, 3], [20, 1], [-1, 3]], np.int64)
    w = np.full((3, 2), 0.5, np.float32)
    ts, ws, eor, counts, row0, dropped = gpu_sort(torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev), 4)
    assert dropped == 2 and counts.tolist() == [1, 1, 0, 2] and row0.tolist() == [0, 1, 2, 2]
    assert ts[:4].tolist() == [0, 1, 0, 2] and eor[:4].tolist() == [0, 1, 3, 3]
    assert ts[4:].tolist() == [0, 0] and eor[4:].tolist() == [0, 0] and ws[4:].tolist() == [0, 0]


@pytest.mark.parametrize("tile_rows", [128, 64, 256, 512])
@pytest.mark.parametrize("kind,T,E,k", ROUTINGS)
def test_build_blocks_bit_exact(dev, kind, T, E, k, tile_rows):
    ids, w = synth.make_routing(kind, T, E, k, seed=T + 1)
    counts = np.bincount(ids.ravel(), minlength=E).astype(np.int32)
    R = ids.size
    for max_blocks in (R // tile_rows + E, max(1, R // 512)):
        rbe, rbr, rmeta = O.build_blocks(counts, max_blocks, init=-7, tile_rows=tile_rows)
        be = torch.full((max_blocks,), -7, dtype=torch.int32, device=dev)
        br = torch.full((max_blocks,), -7, dtype=torch.int32, device=dev)
        meta = torch.zeros(2, dtype=torch.int32, device=dev)
        if tile_rows == 128:
            gp.build_blocks(t16(counts, dev), be, br, meta)
        else:
            gp.build_tiles(t16(counts, dev), be, br, meta, tile_rows)
        assert np.array_equal(be.cpu().numpy(), rbe) and np.array_equal(br.cpu().numpy(), rbr)
        assert np.array_equal(meta.cpu().numpy(), rmeta)


# ------------------------------------------------------------------------------------------- router top-k
def split_tables(counts, tile_rows, thin_rows=64):
    """Closed form of exl3_build_tiles_split: tile_rows-row tiles, an expert's last tile of <= thin_rows rows in a
    second table."""
    full, thin, row = [], [], 0
    for e, c in enumerate(counts.tolist()):
        nf, rem = divmod(c, tile_rows)
        full += [(e, row + i * tile_rows) for i in range(nf)]
        if rem > thin_rows:
            full.append((e, row + nf * tile_rows))
        elif rem > 0:
            thin.append((e, row + nf * tile_rows))
        row += c
    return full, thin, row


@pytest.mark.parametrize("tile_rows", [128, 256, 512])
@pytest.mark.parametrize("kind,T,E,k", ROUTINGS)
def test_build_tiles_split_bit_exact(dev, kind, T, E, k, tile_rows):
    ids, w = synth.make_routing(kind, T, E, k, seed=T + 2)
    counts = np.bincount(ids.ravel(), minlength=E).astype(np.int32)
    R = ids.size
    mf, mt = R // tile_rows + E, min(E, R)
    full, thin, rows = split_tables(counts, tile_rows)
    # the two tables hold exactly the tiles of the one-table schedule (oracle build_blocks), small last tiles moved
    rbe, rbr, rmeta = O.build_blocks(counts, mf, init=-7, tile_rows=tile_rows)
    n = int(rmeta[0])
    assert sorted(full + thin) == sorted(zip(rbe[:n].tolist(), rbr[:n].tolist()))
    t = [torch.full((m,), -7, dtype=torch.int32, device=dev) for m in (mf, mf, mt, mt)]
    meta = torch.full((3,), -5, dtype=torch.int32, device=dev)
    zero = torch.full((T * 37 * 4 + 8,), float("nan"), dtype=torch.float32, device=dev)     # the fused output clear
    gp.build_tiles_split(t16(counts, dev), *t, meta, tile_rows, 64, zero=zero[4:-4])
    torch.cuda.synchronize()
    assert (zero[4:-4] == 0).all() and zero[:4].isnan().all() and zero[-4:].isnan().all()   # exactly the range
    fe, fr, te, tr_ = (x.cpu().numpy() for x in t)
    assert meta.tolist() == [len(full), rows, len(thin)]
    assert list(zip(fe[:len(full)].tolist(), fr[:len(full)].tolist())) == full
    assert list(zip(te[:len(thin)].tolist(), tr_[:len(thin)].tolist())) == thin
    assert (fe[len(full):] == -1).all() and (te[len(thin):] == -1).all()


def fused_prep(ids_t, w_t, E, tile_rows, fused, zero_n=0):
    """The prefill preparation as sort_routes + build_tiles_split (fused=False) or as sort_routes_split_tiles: every
    output, from buffers pre-filled with sentinels."""
    dev = ids_t.device
    R = ids_t.numel()
    mf, mt = R // tile_rows + E, min(E, R)
    out = dict(ts=torch.full((R,), -3, dtype=torch.int64, device=dev),
               ws=torch.full((R,), 7.0, dtype=torch.float16, device=dev),
               eor=torch.full((R,), -3, dtype=torch.int32, device=dev),
               counts=torch.full((E,), -3, dtype=torch.int32, device=dev),
               row0=torch.full((E,), -3, dtype=torch.int32, device=dev),
               ri=torch.full((R,), -3, dtype=torch.int32, device=dev),
               fe=torch.full((mf,), -7, dtype=torch.int32, device=dev),
               fr=torch.full((mf,), -7, dtype=torch.int32, device=dev),
               te=torch.full((mt,), -7, dtype=torch.int32, device=dev),
               tr=torch.full((mt,), -7, dtype=torch.int32, device=dev),
               meta=torch.full((3,), -5, dtype=torch.int32, device=dev),
               zero=torch.full((zero_n + 8,), float("nan"), dtype=torch.float32, device=dev))
    o = out
    z = o["zero"][4:-4] if zero_n else None
    if fused:
        work = gp.sort_routes_split_tiles(ids_t, w_t, E, o["ts"], o["ws"], o["eor"], o["counts"], o["row0"], o["fe"],
                                          o["fr"], o["te"], o["tr"], o["meta"], tile_rows, 64, zero=z,
                                          route_index=o["ri"])
    else:
        work = gp.sort_routes(ids_t, w_t, E, o["ts"], o["ws"], o["eor"], o["counts"], o["row0"], route_index=o["ri"])
        gp.build_tiles_split(o["counts"], o["fe"], o["fr"], o["te"], o["tr"], o["meta"], tile_rows, 64, zero=z)
    torch.cuda.synchronize()
    res = {n: t.cpu().numpy() for n, t in out.items()}
    res["dropped"] = int(work[:4].view(torch.int32).item())
    return res


# every routing at the default 256-row tiles; 128- and 512-row tiles on two of them
SPLIT_TILE_CASES = ([r + (256,) for r in ROUTINGS] +
                    [r + (tr,) for tr in (128, 512) for r in ROUTINGS if r[0] in ("zipf", "softmax")])


@pytest.mark.parametrize("kind,T,E,k,tile_rows", SPLIT_TILE_CASES)
def test_sort_routes_split_tiles_matches_two_ops(dev, kind, T, E, k, tile_rows):
    """The prefill path's two-launch preparation (histogram; scatter with per-workgroup cursors + tile tables +
    output clear) writes exactly what sort_routes followed by build_tiles_split writes (kernel/exl3_grouped_runtime.py
    :59-68, kernel/exl3_grouped_prefill.cu:63-96), bit for bit, with int64 and int32 ids; the clear covers exactly the
    given range."""
    ids, w = synth.make_routing(kind, T, E, k, seed=T + 9)
    wt = torch.from_numpy(w).to(dev)
    for ids_dt in (torch.int64, torch.int32):
        it = torch.from_numpy(ids).to(ids_dt).to(dev)
        a = fused_prep(it, wt, E, tile_rows, fused=False, zero_n=T * 4 * 37)
        b = fused_prep(it, wt, E, tile_rows, fused=True, zero_n=T * 4 * 37)
        for n in a:
            assert np.array_equal(np.atleast_1d(a[n]).view(np.uint8), np.atleast_1d(b[n]).view(np.uint8)), n
        assert (b["zero"][4:-4] == 0).all() and np.isnan(b["zero"][:4]).all() and np.isnan(b["zero"][-4:]).all()
    ref = O.sort_routes(ids, w, E)                      # and both against the oracle
    for g, r in zip((b["ts"], b["ws"], b["eor"], b["counts"], b["row0"]), ref):
        assert np.array_equal(np.asarray(g).view(np.uint8), np.asarray(r).view(np.uint8))


def test_sort_routes_split_tiles_empty_and_dropped(dev):
    """No routes (tables all -1, meta zero) and dropped ids (the tail rows, the dropped count), as the two ops give."""
    a = fused_prep(torch.zeros(0, 8, dtype=torch.int64, device=dev), torch.zeros(0, 8, device=dev), 16, 256, False)
    b = fused_prep(torch.zeros(0, 8, dtype=torch.int64, device=dev), torch.zeros(0, 8, device=dev), 16, 256, True)
    assert b["meta"].tolist() == [0, 0, 0] and (b["fe"] == -1).all() and b["counts"].tolist() == [0] * 16
    for n in a:
        assert np.array_equal(np.atleast_1d(a[n]).view(np.uint8), np.atleast_1d(b[n]).view(np.uint8)), n
    rng = np.random.default_rng(4)
    ids = rng.integers(0, 40, (3000, 8)).astype(np.int64)
    ids[::7, 3] = -1                                    # dropped: negative and out-of-range ids
    ids[5::11, 6] = 40
    w = rng.random((3000, 8)).astype(np.float32)
    args = (torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev), 40, 256)
    a = fused_prep(*args, fused=False, zero_n=64)
    b = fused_prep(*args, fused=True, zero_n=64)
    assert b["dropped"] == int((ids < 0).sum() + (ids >= 40).sum()) > 0
    for n in a:
        assert np.array_equal(np.atleast_1d(a[n]).view(np.uint8), np.atleast_1d(b[n]).view(np.uint8)), n


def test_prefill_thin_tiles_match_one_table(dev):
    """Each expert's small last tile on the thin kernel gives the one-table result (the per-row arithmetic is the
    same; the down scatter's atomics may add in another order)."""
    L, x, ids, w, cfg = synth.make_config("headline", seed=3, T=2048)
    TL = synth.to_device(L, dev)
    args = (t16(x, dev), t16(ids, dev), t16(w, dev), TL, LIMIT)
    a = rt.grouped_prefill(*args, scatter="atomic", thin_tiles=True)
    b = rt.grouped_prefill(*args, scatter="atomic", thin_tiles=False)
    torch.cuda.synchronize()
    assert ((a - b).norm() / b.norm()).item() < 1e-6
    # the combine mode sums each token's route rows in a fixed order, so there the two schedules agree bit for bit
    c = rt.grouped_prefill(*args, scatter="combine", thin_tiles=True)
    d = rt.grouped_prefill(*args, scatter="combine", thin_tiles=False)
    assert torch.equal(c.view(torch.int32), d.view(torch.int32))
    assert ((c - b).norm() / b.norm()).item() < 1e-6


def test_prefill_tile_heights_agree_bitwise(dev):
    """128-, 256- and 512-row expert tiles (the 4-wave kernel, and the 8-wave kernel with its interleaved row groups)
    give the same output bit for bit with the combine output: a row's sums over K run in the same order whatever the
    tile height or the wave that multiplies it."""
    L, x, ids, w, cfg = synth.make_config("headline", seed=5, T=2048)
    TL = synth.to_device(L, dev)
    args = (t16(x, dev), t16(ids, dev), t16(w, dev), TL, LIMIT)
    outs = [rt.grouped_prefill(*args, scatter="combine", rows_per_tile=tr) for tr in (128, 256, 512)]
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int32), outs[0].view(torch.int32))


def _margins(logits, bias, k):
    """Per token: is the chosen set unambiguous (k-th and (k+1)-th selection scores more than 1e-5 apart), and is the
    order too (every adjacent pair among the first k + 1 apart)? fp32 sigmoids may differ by an ulp between devices."""
    s = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    sel = np.sort(s + (bias if bias is not None else 0), axis=1)[:, ::-1][:, :k + 1]
    gaps = sel[:, :-1] - sel[:, 1:]
    clear = (gaps > 1e-5) | (gaps == 0)              # exact ties (equal logits) break by expert id on both sides
    set_ok = clear[:, k - 1] if sel.shape[1] > k else np.ones(sel.shape[0], bool)
    return set_ok, set_ok & clear[:, :k - 1].all(axis=1)


@pytest.mark.parametrize("T,E,k,dt,ids_dt,renorm,with_bias", [
    (8192, 288, 8, torch.float32, torch.int64, True, True),         # the headline router (GLM-5.3-Flash)
    (1000, 288, 8, torch.bfloat16, torch.int32, True, True),
    (777, 1024, 16, torch.float16, torch.int64, False, False),
    (64, 8, 1, torch.float32, torch.int32, True, True),
    (0, 288, 8, torch.float32, torch.int64, True, True)])
def test_route_topk(dev, T, E, k, dt, ids_dt, renorm, with_bias):
    rng = np.random.default_rng(T + E)
    lg = torch.from_numpy((rng.standard_normal((T, E)) * 2).astype(np.float32)).to(dt)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if with_bias else None
    ids, w = gp.route_topk(lg.to(dev), t16(bias, dev) if with_bias else None, k, 2.5, renorm, ids_dt)
    assert ids.dtype == ids_dt and w.dtype == torch.float32 and tuple(ids.shape) == (T, k)
    if T == 0:
        return
    lg32 = lg.float().numpy()
    rid, rw = O.route_topk(lg32, bias, k, 2.5, renorm)
    set_ok, order_ok = _margins(lg32, bias, k)
    assert set_ok.mean() > 0.95 and order_ok.mean() > 0.8
    gid = ids.cpu().numpy().astype(np.int64)
    gw = w.cpu().numpy()
    assert np.array_equal(gid[order_ok], rid[order_ok])                 # same experts in the same order
    # same experts with the same weights wherever the chosen set is unambiguous (pair weights with ids)
    gi, ri = np.argsort(gid[set_ok], axis=1), np.argsort(rid[set_ok], axis=1)
    assert np.array_equal(np.take_along_axis(gid[set_ok], gi, 1), np.take_along_axis(rid[set_ok], ri, 1))
    assert np.allclose(np.take_along_axis(gw[set_ok], gi, 1), np.take_along_axis(rw[set_ok], ri, 1), rtol=2e-6,
                       atol=1e-7)


def test_route_topk_nan_and_feeds_sort(dev):
    T, E, k = 300, 64, 8
    rng = np.random.default_rng(3)
    lg = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    lg[7, :] = np.nan
    lg[7, [3, 5]] = 1.0                                             # only two finite candidates
    ids, w = gp.route_topk(t16(lg, dev), None, k, 1.0)
    gid = ids.cpu().numpy()
    assert gid[7, :2].tolist() == [3, 5] and (gid[7, 2:] == -1).all() and (w.cpu().numpy()[7, 2:] == 0).all()
    assert not np.isnan(w.cpu().numpy()).any()
    # the ids and weights go straight into the sort; the dropped -1 routes are counted, not placed
    R = T * k
    ts = torch.empty(R, dtype=torch.int64, device=dev)
    ws = torch.empty(R, dtype=torch.float16, device=dev)
    eor = torch.empty(R, dtype=torch.int32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    row0 = torch.empty(E, dtype=torch.int32, device=dev)
    gp.sort_routes(ids, w, E, ts, ws, eor, counts, row0)
    assert int(counts.sum()) == R - 6


def test_prefill_from_router_logits(dev):
    """Router top-k on the GPU feeding the grouped path equals the staged oracle on the oracle's routing."""
    L, x, _, _, cfg = synth.make_config("tiny", seed=4)
    rng = np.random.default_rng(4)
    lg = (rng.standard_normal((cfg["T"], cfg["E"])) * 2).astype(np.float32)
    bias = (rng.standard_normal(cfg["E"]) * 0.1).astype(np.float32)
    rid, rw = O.route_topk(lg, bias, cfg["topk"], 2.5)
    set_ok, order_ok = _margins(lg, bias, cfg["topk"])
    assert order_ok.all()
    TL = synth.to_device(L, dev)
    got = rt.grouped_prefill_from_logits(t16(x, dev), t16(lg, dev), TL, LIMIT, t16(bias, dev), cfg["topk"], 2.5)
    ref = O.grouped_prefill(x, rid, rw, to_np_layer(L), LIMIT)
    assert O.rel_l2(got.cpu().numpy(), ref) < 1e-4


def test_checkpoint_tp_ranks_on_gpu(dev, tmp_path):
    """A layer written in the EXL3 checkpoint layout, loaded for two tensor-parallel ranks straight onto the GPU:
    the ranks' grouped_prefill outputs sum to the unsliced layer's (the all-reduce), and match the oracle."""
    from exl3_grouped import checkpoint as C
    L = synth.make_layer(E=8, H=512, I=512, bits=4, seed=21, svh_scale=1 / 16)
    C.write_moe_layer(str(tmp_path), 5, L.w13_trellis, L.w13_suh, L.w13_svh, L.w2_trellis, L.w2_suh, L.w2_svh)
    x = synth.make_x(256, 512, 21)
    ids, w = synth.routing_softmax(256, 8, 4, 21)
    xt, it, wt = t16(x, dev), t16(ids, dev), t16(w, dev)
    full = rt.grouped_prefill(xt, it, wt, C.load_moe_layer(str(tmp_path), 5, device=dev), LIMIT)
    parts = [rt.grouped_prefill(xt, it, wt, C.load_moe_layer(str(tmp_path), 5, tp_rank=r, tp=2, device=dev), LIMIT)
             for r in range(2)]
    assert O.rel_l2((parts[0] + parts[1]).cpu().numpy(), full.cpu().numpy()) < 1e-5
    assert O.rel_l2(full.cpu().numpy(), O.expert_loop(x, ids, w, to_np_layer(L), LIMIT)) < 1e-3


# ------------------------------------------------------------------------------------------- Hadamard passes
@pytest.mark.parametrize("gather", [True, False])
def test_row_had(dev, gather):
    rng = np.random.default_rng(7)
    T, H, E, R = 300, 4096, 20, 1200
    x = rng.standard_normal((T if gather else R, H)).astype(np.float16)
    tok = rng.integers(0, T, R).astype(np.int64)
    eor = np.sort(rng.integers(0, E, R)).astype(np.int32)
    suh2 = synth._signs(rng, (E, 2, H))
    dst = torch.empty(R, H, dtype=torch.float16, device=dev)
    suh_t = t16(suh2, dev)
    gp.row_had(t16(x, dev), dst, t16(tok, dev) if gather else None, t16(eor, dev), suh_t[:, 0], gather)
    ref = O.row_had(x, tok if gather else None, eor, suh2[:, 0], gather)
    got = dst.cpu().numpy()
    assert O.rel_l2(got, ref) < 1e-4 and within_f16_steps(got, ref)
    dst16 = torch.full((gp.t16_rows(R), H), float("nan"), dtype=torch.float16, device=dev)
    gp.row_had(t16(x, dev), dst16, t16(tok, dev) if gather else None, t16(eor, dev), suh_t[:, 0], gather, dst_layout=1,
               rows=R)
    assert np.array_equal(from_t16(dst16.cpu().numpy(), R).view(np.uint16), got.view(np.uint16))     # same values, T16


@pytest.mark.parametrize("scale", [1.0, 12.0])
def test_act_had(dev, scale):
    rng = np.random.default_rng(8)
    R, I, E = 2000, 768, 30
    gu = (rng.standard_normal((R, 2 * I)) * scale).astype(np.float16)     # scale 12 drives the clamp
    eor = np.sort(rng.integers(0, E, R)).astype(np.int32)
    suh = synth._signs(rng, (E, I))
    act = torch.empty(R, I, dtype=torch.float16, device=dev)
    gp.act_had(t16(gu, dev), act, t16(eor, dev), t16(suh, dev), LIMIT)
    ref = O.act_had(gu, eor, suh, LIMIT)
    got = act.cpu().numpy()
    act16 = torch.full((gp.t16_rows(R), I), float("nan"), dtype=torch.float16, device=dev)
    gp.act_had(t16(gu, dev), act16, t16(eor, dev), t16(suh, dev), LIMIT, dst_layout=1)
    assert np.array_equal(from_t16(act16.cpu().numpy(), R).view(np.uint16), got.view(np.uint16))
    act_t = torch.full((gp.t16_rows(R), I), float("nan"), dtype=torch.float16, device=dev)   # gu in T16 too
    gp.act_had(t16(to_t16(gu), dev), act_t, t16(eor, dev), t16(suh, dev), LIMIT, dst_layout=1, gu_layout=1, rows=R)
    assert np.array_equal(from_t16(act_t.cpu().numpy(), R).view(np.uint16), got.view(np.uint16))
    # fp16 rounding of the SwiGLU output can land one step apart (fast exp vs libm exp) before the Hadamard
    assert O.rel_l2(got, ref) < 1e-3 and within_f16_steps(got, ref, steps=2, frac=0.99)


# ------------------------------------------------------------------------------------------- grouped GEMM
@functools.lru_cache(maxsize=4)
def stage_inputs(name, seed, T=None, bits=None, svh_scale=1.0):
    L, x, ids, w, cfg = synth.make_config(name, seed=seed, T=T, bits=bits, svh_scale=svh_scale)
    layer = to_np_layer(L)
    ts, ws, eor, counts, row0 = O.sort_routes(ids, w, cfg["E"])
    return L, layer, x, ids, w, cfg, (ts, ws, eor, counts, row0)


# Oracle results are shared by the tile sizes of one case (the expert loop dominates the test time).
@functools.lru_cache(maxsize=2)
def gate_up_case(name, T, bits):
    L, layer, x, ids, w, cfg, (ts, ws, eor, counts, row0) = stage_inputs(name, 1, T=T, bits=bits)
    h13 = O.row_had(x.astype(np.float16), ts, eor, L.w13_suh[:, 0], True)
    return h13, O.grouped_gemm_mode0(h13, O.WeightCache(layer), counts, row0)


@functools.lru_cache(maxsize=2)
def down_case(name, T, bits, seed, act_seed):
    L, layer, x, ids, w, cfg, (ts, ws, eor, counts, row0) = stage_inputs(name, seed, T=T, bits=bits)
    rng = np.random.default_rng(act_seed)
    act = (rng.standard_normal((ids.size, cfg["I"])) * 3).astype(np.float16)
    return act, O.grouped_gemm_mode1(act, O.WeightCache(layer), counts, row0, ts, ws, cfg["T"])


def gpu_blocks(counts, R, E, dev, tile_rows=128):
    mb = R // tile_rows + E
    be = torch.empty(mb, dtype=torch.int32, device=dev)
    br = torch.empty(mb, dtype=torch.int32, device=dev)
    meta = torch.zeros(2, dtype=torch.int32, device=dev)
    gp.build_tiles(t16(counts, dev), be, br, meta, tile_rows)
    return be, br


@pytest.mark.parametrize("tile_rows", [128, 256, 512])
@pytest.mark.parametrize("name,T,bits", [("tiny", None, 4), ("layer1k", None, 4), ("headline", 256, 4),
                                         ("thin", 1024, 4), ("thin", 1024, 3), ("thin", 1024, 2)])
def test_grouped_gemm_gate_up(dev, name, T, bits, tile_rows):
    L, layer, x, ids, w, cfg, (ts, ws, eor, counts, row0) = stage_inputs(name, 1, T=T, bits=bits)
    R = ids.size
    h13, ref = gate_up_case(name, T, bits)
    TL = synth.to_device(L, dev)
    be, br = gpu_blocks(counts, R, cfg["E"], dev, tile_rows)
    gu = torch.empty(R, 2 * cfg["I"], dtype=torch.float16, device=dev)
    gp.grouped_gemm(t16(h13, dev), TL.w13_trellis[:, 0], TL.w13_trellis[:, 1], TL.w13_svh[:, 0], TL.w13_svh[:, 1],
                    be, br, t16(counts, dev), t16(row0, dev), None, None, gu, 0, tile_rows=tile_rows)
    got = gu.cpu().numpy()
    assert O.rel_l2(got, ref) < 1e-4 and within_f16_steps(got, ref)
    gu16 = torch.empty_like(gu)
    gp.grouped_gemm(t16(to_t16(h13), dev), TL.w13_trellis[:, 0], TL.w13_trellis[:, 1], TL.w13_svh[:, 0],
                    TL.w13_svh[:, 1], be, br, t16(counts, dev), t16(row0, dev), None, None, gu16, 0, tile_rows=tile_rows,
                    a_layout=1, a_rows=R)
    assert torch.equal(gu16, gu)                                  # T16 activations: identical arithmetic
    gut = torch.full((gp.t16_rows(R), 2 * cfg["I"]), float("nan"), dtype=torch.float16, device=dev)
    gp.grouped_gemm(t16(to_t16(h13), dev), TL.w13_trellis[:, 0], TL.w13_trellis[:, 1], TL.w13_svh[:, 0],
                    TL.w13_svh[:, 1], be, br, t16(counts, dev), t16(row0, dev), None, None, gut, 4, tile_rows=tile_rows,
                    a_layout=1, a_rows=R)
    assert np.array_equal(from_t16(gut.cpu().numpy(), R).view(np.uint16), gu.cpu().numpy().view(np.uint16))   # mode 4
    # the same launch clearing a buffer on the side (the prefill path's down scatter output): same gu, exactly the range
    zero = torch.full((4 * 1237 + 8,), float("nan"), dtype=torch.float32, device=dev)
    gz = torch.full_like(gut, float("nan"))
    gp.grouped_gemm(t16(to_t16(h13), dev), TL.w13_trellis[:, 0], TL.w13_trellis[:, 1], TL.w13_svh[:, 0],
                    TL.w13_svh[:, 1], be, br, t16(counts, dev), t16(row0, dev), None, None, gz, 4, tile_rows=tile_rows,
                    a_layout=1, a_rows=R, zero=zero[4:-4])
    torch.cuda.synchronize()
    assert torch.equal(gz.view(torch.int16), gut.view(torch.int16))
    assert (zero[4:-4] == 0).all() and zero[:4].isnan().all() and zero[-4:].isnan().all()


@pytest.mark.parametrize("tile_rows", [128, 256, 512])
@pytest.mark.parametrize("name,T,bits", [("tiny", None, 4), ("layer1k", None, 4), ("thin", 512, 4), ("thin", 512, 3),
                                         ("thin", 512, 2)])
def test_grouped_gemm_down_scatter(dev, name, T, bits, tile_rows):
    L, layer, x, ids, w, cfg, (ts, ws, eor, counts, row0) = stage_inputs(name, 2, T=T, bits=bits)
    R = ids.size
    act, ref = down_case(name, T, bits, 2, 9)
    TL = synth.to_device(L, dev)
    be, br = gpu_blocks(counts, R, cfg["E"], dev, tile_rows)
    out = torch.zeros(cfg["T"], cfg["H"], dtype=torch.float32, device=dev)
    gp.grouped_gemm(t16(act, dev), TL.w2_trellis, None, TL.w2_svh, None, be, br, t16(counts, dev), t16(row0, dev),
                    t16(ts, dev), t16(ws, dev), out, 1, tile_rows=tile_rows)
    assert O.rel_l2(out.cpu().numpy(), ref) < 1e-5
    out16 = torch.zeros_like(out)
    gp.grouped_gemm(t16(to_t16(act), dev), TL.w2_trellis, None, TL.w2_svh, None, be, br, t16(counts, dev),
                    t16(row0, dev), t16(ts, dev), t16(ws, dev), out16, 1, tile_rows=tile_rows, a_layout=1, a_rows=R)
    assert O.rel_l2(out16.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("tile_rows", [64, 128, 256, 512])
@pytest.mark.parametrize("name,T", [("tiny", None), ("layer1k", None)])
def test_grouped_gemm_down_routes_and_combine(dev, name, T, tile_rows):
    L, layer, x, ids, w, cfg, (ts, ws, eor, counts, row0) = stage_inputs(name, 3, T=T)
    R = ids.size
    act, ref = down_case(name, T, None, 3, 10)
    TL = synth.to_device(L, dev)
    be, br = gpu_blocks(counts, R, cfg["E"], dev, tile_rows)
    ri = torch.from_numpy(np.argsort(ids.reshape(-1), kind="stable").astype(np.int32)).to(dev)
    outs = []
    for _ in range(2):
        partial = torch.full((R, cfg["H"]), float("nan"), dtype=torch.float32, device=dev)
        gp.grouped_gemm(t16(act, dev), TL.w2_trellis, None, TL.w2_svh, None, be, br, t16(counts, dev),
                        t16(row0, dev), None, t16(ws, dev), partial, 2, route_index=ri, tile_rows=tile_rows)
        assert not torch.isnan(partial).any()                      # every route row written exactly
        out = torch.full((cfg["T"], cfg["H"]), float("nan"), dtype=torch.float32, device=dev)
        gp.combine_routes(partial, out, cfg["topk"], t16(ids, dev), cfg["E"])
        outs.append(out.cpu().numpy())
    assert O.rel_l2(outs[0], ref) < 1e-5
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))      # deterministic


@pytest.mark.parametrize("k,N,id_dtype", [(3, 16, torch.int64), (8, 16, torch.int64), (8, 1024, torch.int64),
                                          (8, 4096, torch.int32), (8, 2048, torch.int64)])
def test_combine_skips_invalid_routes(dev, k, N, id_dtype):
    """Dropped routes' rows (never written by mode 2: NaN here) are skipped; the rest add in route order. k = 8 runs
    the unrolled kernels, which load every row and discard the dropped ones by a select (rows of a multiple of 1024
    floats: one workgroup per token and 1024 columns)."""
    T = 5
    partial = torch.arange(T * k * N, dtype=torch.float32, device=dev).reshape(T * k, N)
    ids = torch.from_numpy(np.random.default_rng(k + N).integers(-1, 6, (T, k))).to(device=dev, dtype=id_dtype)
    ids[0] = torch.arange(k, device=dev) % 4                                     # ids 4 and 5 out of range
    keep = ((ids >= 0) & (ids < 4)).cpu()
    partial.view(T, k, N)[~keep.to(dev)] = float("nan")
    out = torch.empty(T, N, device=dev)
    gp.combine_routes(partial, out, k, ids, 4)
    p = partial.cpu().reshape(T, k, N)
    ref = torch.where(keep[:, :, None], p, torch.zeros(())).sum(1)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("N", [4096, 48])
def test_combine_order_is_route_order(dev, N):
    """Random fp32 rows add in route order j = 0 .. 7 exactly (a sequential fp32 sum on the CPU, bit for bit), for the
    per-token-column kernel (N = 4096) and the general one (N = 48)."""
    T, k = 37, 8
    rng = np.random.default_rng(N)
    partial = torch.from_numpy(rng.standard_normal((T * k, N)).astype(np.float32) * 1e3).to(dev)
    ids = torch.from_numpy(rng.integers(-1, 9, (T, k))).to(dev)                       # 8 out of range
    out = torch.empty(T, N, device=dev)
    gp.combine_routes(partial, out, k, ids, 8)
    p = partial.cpu().reshape(T, k, N)
    keep = ((ids >= 0) & (ids < 8)).cpu()
    ref = torch.zeros(T, N)
    for j in range(k):
        ref = ref + torch.where(keep[:, j, None], p[:, j], torch.zeros(()))
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("N", [4096, 48])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_combine_into_half_dtypes_is_the_cast(dev, N, dtype):
    """combine_routes writing bf16 / fp16 gives exactly the fp32 combine followed by torch's cast: one rounding to nearest
    even, NaN and infinities, fp16 overflow to infinity, bf16 ties."""
    T, k = 19, 8
    rng = np.random.default_rng(N + 7)
    partial = torch.from_numpy(rng.standard_normal((T * k, N)).astype(np.float32) * 300).to(dev)
    partial[3, :8] = torch.tensor([float("nan"), float("inf"), -float("inf"), 7e4, -7e4, 1e-8, -0.0, 3.0], device=dev)
    bf_tie = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x7F7FFFFF], dtype=np.uint32).view(np.float32)
    partial[k * 5, :4] = torch.from_numpy(bf_tie).to(dev)         # token 5: ties and the largest finite fp32
    partial[k * 5 + 1:k * 6, :4] = 0.0
    ids = torch.from_numpy(rng.integers(-1, 9, (T, k))).to(dev)
    ids[5] = torch.arange(k, device=dev)
    ref32 = torch.empty(T, N, device=dev)
    gp.combine_routes(partial, ref32, k, ids, 8)
    out = torch.full((T, N), 1.0, dtype=dtype, device=dev)
    gp.combine_routes(partial, out, k, ids, 8)
    assert torch.equal(out.view(torch.int16), ref32.to(dtype).view(torch.int16))


@pytest.mark.parametrize("scatter", ["atomic", "combine"])
def test_prefill_out_dtype(dev, scatter):
    """grouped_prefill(out_dtype=bf16) is grouped_prefill(...).to(bf16) bit for bit (the combine method writes it
    directly; the atomic scatter casts its fp32 target)."""
    L, x, ids, w, cfg = synth.make_config("tiny", seed=12)
    TL = synth.to_device(L, dev)
    args = (t16(x, dev).to(torch.bfloat16), t16(ids, dev), t16(w, dev), TL, LIMIT)
    ref = rt.grouped_prefill(*args, scatter=scatter)
    got = rt.grouped_prefill(*args, scatter=scatter, out_dtype=torch.bfloat16)
    assert got.dtype == torch.bfloat16 and ref.dtype == torch.float32
    if scatter == "combine":
        assert torch.equal(got.view(torch.int16), ref.to(torch.bfloat16).view(torch.int16))
    else:                                                          # atomic order may differ between the two calls
        assert torch.allclose(got.float(), ref.to(torch.bfloat16).float(), rtol=1e-2, atol=1e-2)


# ------------------------------------------------------------------------------------------- dense EXL3 linear
@pytest.mark.parametrize("M,K,N,bits", [(1, 4096, 1536, 4), (300, 768, 4096, 4), (4096, 4096, 1536, 4),
                                        (200, 4096, 1536, 3), (70, 1024, 512, 2), (0, 512, 256, 4),
                                        (4096, 2048, 1536, 3), (3072, 4096, 2048, 2)])     # the last two: K-pair
def test_linear_exl3(dev, M, K, N, bits):
    rng = np.random.default_rng(M + K + bits)
    x = rng.standard_normal((M, K)).astype(np.float16)
    packed = synth._random_words(rng, (K // 16, N // 16, 16 * bits))
    suh = synth._signs(rng, (K,))
    svh = synth._svh(rng, (N,))
    y32 = gp.linear_exl3(t16(x, dev), t16(packed, dev), t16(suh, dev), t16(svh, dev), bits, out_dtype=torch.float32)
    y16 = gp.linear_exl3(t16(x, dev), t16(packed, dev), t16(suh, dev), t16(svh, dev), bits)
    assert y32.shape == (M, N) and y16.dtype == torch.float16
    if M == 0:
        return
    ref = O.linear(x, packed, suh, svh)
    got = y32.cpu().numpy()
    assert O.rel_l2(got, ref) < 1e-4
    assert within_f16_steps(y16.cpu().numpy(), got.astype(np.float16))      # fp16 store = rounded fp32 result
    again = gp.linear_exl3(t16(x, dev), t16(packed, dev), t16(suh, dev), t16(svh, dev), bits, out_dtype=torch.float32)
    assert torch.equal(again, y32)                                          # the same summation order every run


# ------------------------------------------------------------------------------------------- fat GEMM (config 2)
@pytest.mark.parametrize("M", [300, 4096])
def test_fat_gemm_config2(dev, M):
    a, packed, svh = synth.make_fat(0, M=M)
    ref = O.fat_gemm(a, packed, svh, dtype=np.float32)
    outs = []
    for v in range(4):
        out = torch.empty(M, 1536, dtype=torch.float32, device=dev)
        gp.fat_gemm_v2(t16(a, dev), t16(packed, dev), out, t16(svh, dev), 4, True, False, v)
        outs.append(out.cpu().numpy())
    assert O.rel_l2(outs[0], ref) < 1e-5
    # max-abs difference against the fp32-accumulate reference (only the order of the fp32 additions differs)
    max_abs, scale = float(np.abs(outs[0] - ref).max()), float(np.abs(ref).max())
    print(f"fat GEMM config 2, M={M}: max |out - ref| = {max_abs:.3e} (max |ref| = {scale:.3e})")
    assert max_abs <= 1e-5 * scale
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])                                # variants are bit-identical
    alias = torch.empty(M, 1536, dtype=torch.float32, device=dev)
    gp.exl3_fat_gemm(t16(a, dev), t16(packed, dev), alias, t16(svh, dev), 4, True, False)   # PR77's name and order
    assert np.array_equal(alias.cpu().numpy(), outs[1])


@pytest.mark.parametrize("M,bits", [(4090, 4), (4090, 3), (3600, 2)])
def test_fat_gemm_kpair_shapes(dev, M, bits):
    """The K-pair schedule (192 or more 256-row tiles x 128 columns at K = 4096, both K halves in one workgroup) on
    row counts that are not a multiple of 16 (a partial last row group) and 2/3/4-bit tiles, against the oracle, with
    every variant bit-identical and every output written."""
    a, packed, svh = synth.make_fat(5, M=M, K=4096, N=1536, bits=bits)
    ref = O.fat_gemm(a, packed, svh, dtype=np.float32)
    outs = []
    for v in range(4):
        out = torch.full((M, 1536), float("nan"), dtype=torch.float32, device=dev)
        gp.fat_gemm_v2(t16(a, dev), t16(packed, dev), out, t16(svh, dev), bits, True, False, v)
        outs.append(out.cpu().numpy())
    assert np.isfinite(outs[0]).all()
    assert O.rel_l2(outs[0], ref) < 1e-5
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])


def test_fat_gemm_scatter(dev):
    M, T = 300, 4096
    a, packed, svh = synth.make_fat(1, M=M, K=1024, N=4096)
    rng = np.random.default_rng(11)
    tok = rng.permutation(T)[:M].astype(np.int64)
    rw = (rng.random(M) * 0.5 + 0.25).astype(np.float16)
    out0 = np.zeros((T, 4096), np.float32)
    ref = O.fat_gemm_scatter(a, packed, svh, tok, rw, out0, dtype=np.float32)
    outs = []
    for v in range(4):
        out = torch.zeros(T, 4096, dtype=torch.float32, device=dev)
        gp.fat_gemm_v2_scatter(t16(a, dev), t16(packed, dev), out, t16(svh, dev), t16(tok, dev), t16(rw, dev), 4,
                               True, False, v)
        outs.append(out.cpu().numpy())
    assert O.rel_l2(outs[1], ref) < 1e-5
    for o in outs:                          # each token receives one row: the schedules are bit-identical
        assert np.array_equal(o, outs[1])
    alias = torch.zeros(T, 4096, dtype=torch.float32, device=dev)
    gp.exl3_fat_gemm_scatter(t16(a, dev), t16(packed, dev), alias, t16(svh, dev), t16(tok, dev), t16(rw, dev), 4,
                             True, False)                              # PR77's name and argument order
    assert np.array_equal(alias.cpu().numpy(), outs[1])


@pytest.mark.parametrize("M,K", [(300, 64), (300, 192), (300, 320), (10, 4096), (40, 4096), (270, 4096)])
@pytest.mark.parametrize("bits", [4, 3, 2])
def test_fat_gemm_short_k(dev, M, K, bits):
    """K/32 stages not a multiple of the mainloop's 4-stage trip (tail of 2 stages; K=64 is the tail alone), and
    row counts that leave waves with <= 16 rows or none (the thin-expert variants) over long K."""
    a, packed, svh = synth.make_fat(3, M=M, K=K, N=256, bits=bits)
    ref = O.fat_gemm(a, packed, svh)
    out = torch.empty(M, 256, dtype=torch.float32, device=dev)
    gp.fat_gemm_v2(t16(a, dev), t16(packed, dev), out, t16(svh, dev), bits, True, False, 1)
    assert O.rel_l2(out.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_thin_tile_epilogues_bit_identical(dev, bits):
    """Thin tiles of at most 16 rows (the column-split loop, its results gathered in LDS for wave 0's epilogue; one-row
    tiles in the fp32 atomic modes take a one-row epilogue, two columns per lane) must give the shared loop's outputs
    bit for bit. Dense calls of 1, 2, 5 and 16 rows (thin tiles) against the same rows of a 20-row call (the shared
    loop), for the fp32 store (K = 1024), the K-split fp32 atomic store (K = 4096: two slices added onto zero) and the
    routed scatter (one add per token), and against the oracle."""
    M = 20
    tok = np.random.default_rng(bits).permutation(40)[:M].astype(np.int64)
    rw = (np.random.default_rng(bits + 1).random(M) * 0.5 + 0.25).astype(np.float16)
    for K in (1024, 4096):
        a, packed, svh = synth.make_fat(7 + K, M=M, K=K, N=256, bits=bits)
        ref = O.fat_gemm(a, packed, svh, dtype=np.float32)
        outs, scat = {}, {}
        for m in (1, 2, 5, 16, M):
            out = torch.full((m, 256), float("nan"), dtype=torch.float32, device=dev)
            gp.fat_gemm_v2(t16(a[:m], dev), t16(packed, dev), out, t16(svh, dev), bits, True, False, 1)
            outs[m] = out.cpu().numpy()
            sc = torch.zeros(40, 256, dtype=torch.float32, device=dev)
            gp.fat_gemm_v2_scatter(t16(a[:m], dev), t16(packed, dev), sc, t16(svh, dev), t16(tok[:m], dev),
                                   t16(rw[:m], dev), bits, True, False, 1)
            scat[m] = sc.cpu().numpy()
        assert O.rel_l2(outs[M], ref) < 1e-5
        assert O.rel_l2(scat[M][tok], ref * rw[:, None].astype(np.float32)) < 1e-5
        for m in (1, 2, 5, 16):
            assert np.array_equal(outs[m].view(np.uint32), outs[M][:m].view(np.uint32)), (K, m)
            assert np.array_equal(scat[m][tok[:m]].view(np.uint32), scat[M][tok[:m]].view(np.uint32)), (K, m)
            assert not np.delete(scat[m], tok[:m], axis=0).any()


def test_thin_tile_epilogue_grouped_bit_identical(dev):
    """The grouped GEMM's thin tiles (64-row tables: the thin kernel, experts of 1-16 rows on the column-split loop)
    against the same rows on 256-row tiles (the shared loop): the fp16 gate|up rows and the down projection's per-route
    fp32 rows bit for bit, at the headline routing over 256 tokens."""
    L, x, ids, w, cfg = synth.make_config("headline", seed=4, T=256)
    E, H, I = cfg["E"], cfg["H"], cfg["I"]
    ts, ws, eor, counts, row0 = O.sort_routes(ids, w, E)
    R = ids.size
    assert ((counts >= 2) & (counts <= 16)).any() and (counts == 1).any()
    TL = synth.to_device(L, dev)
    rng = np.random.default_rng(3)
    h13 = t16(to_t16(rng.standard_normal((R, H)).astype(np.float16)), dev)
    act = t16(to_t16(rng.standard_normal((R, I)).astype(np.float16)), dev)
    ri = torch.from_numpy(np.argsort(ids.reshape(-1), kind="stable").astype(np.int32)).to(dev)
    res = {}
    for tr in (64, 256):
        be, br = gpu_blocks(counts, R, E, dev, tr)
        gu = torch.full((R, 2 * I), float("nan"), dtype=torch.float16, device=dev)
        gp.grouped_gemm(h13, TL.w13_trellis[:, 0], TL.w13_trellis[:, 1], TL.w13_svh[:, 0], TL.w13_svh[:, 1], be, br,
                        t16(counts, dev), t16(row0, dev), None, None, gu, 0, tile_rows=tr, a_layout=1, a_rows=R)
        part = torch.full((R, H), float("nan"), dtype=torch.float32, device=dev)
        gp.grouped_gemm(act, TL.w2_trellis, None, TL.w2_svh, None, be, br, t16(counts, dev), t16(row0, dev), None,
                        t16(ws, dev), part, 2, route_index=ri, tile_rows=tr, a_layout=1, a_rows=R)
        res[tr] = (gu.cpu().numpy().view(np.uint16), part.cpu().numpy().view(np.uint32))
    assert not np.isnan(res[64][1].view(np.float32)).any()
    assert np.array_equal(res[64][0], res[256][0])
    assert np.array_equal(res[64][1], res[256][1])


@pytest.mark.parametrize("bits", [2, 3])
def test_fat_gemm_low_bits(dev, bits):
    a, packed, svh = synth.make_fat(2, M=200, K=1024, N=768, bits=bits)
    ref = O.fat_gemm(a, packed, svh)
    out = torch.empty(200, 768, dtype=torch.float32, device=dev)
    gp.fat_gemm_v2(t16(a, dev), t16(packed, dev), out, t16(svh, dev), bits, True, False, 1)
    assert O.rel_l2(out.cpu().numpy(), ref) < 1e-5


# ------------------------------------------------------------------------------------------- full layer
class Fake:
    pass


def run_layer(L, x, ids, w, dev, scatter=None):
    """One grouped_prefill call; scatter None is the shipped default (EXL3_GROUPED_SCATTER, else "auto")."""
    TL = synth.to_device(L, dev)
    out = rt.grouped_prefill(t16(x, dev), t16(ids, dev), t16(w, dev), TL, LIMIT, scatter=scatter)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("scatter", ["atomic", "combine"])
@pytest.mark.parametrize("name,svh_scale", [("tiny", 1.0), ("tiny", 1 / 64), ("layer1k", 1.0), ("layer1k", 1 / 64)])
def test_layer_vs_expert_loop(dev, name, svh_scale, scatter):
    L, x, ids, w, cfg = synth.make_config(name, seed=4, svh_scale=svh_scale)
    got = run_layer(L, x, ids, w, dev, scatter).cpu().numpy()
    layer = to_np_layer(L)
    ref = O.expert_loop(x, ids, w, layer, LIMIT)
    assert O.rel_l2(got, ref) < 1e-3
    staged = O.grouped_prefill(x, ids, w, layer, LIMIT)
    assert O.rel_l2(got, staged) < 1e-4


def sampled_loop(L, x, ids, w, tokens):
    layer = to_np_layer(L)
    return O.expert_loop(x[tokens], ids[tokens], w[tokens], layer, LIMIT)


@pytest.mark.parametrize("scatter", ["atomic", "combine"])
def test_headline_sampled_tokens_and_properties(dev, scatter):
    L, x, ids, w, cfg = synth.make_config("headline", seed=0)
    out = run_layer(L, x, ids, w, dev, scatter)
    if scatter == "combine":                           # the fixed-order sum: bit-reproducible at full size
        again = run_layer(L, x, ids, w, dev, scatter)
        assert torch.equal(out.view(torch.int32), again.view(torch.int32))
    tokens = np.random.default_rng(0).choice(cfg["T"], 128, replace=False)
    ref = sampled_loop(L, x, ids, w, tokens)
    assert O.rel_l2(out.cpu().numpy()[tokens], ref) < 1e-3
    # linearity in the route weights (x2 is exact in fp16)
    out2 = run_layer(L, x, ids, 2 * w, dev, scatter)
    assert (out2 - 2 * out).norm().item() <= 1e-6 * out.norm().item()
    # token permutation equivariance
    perm = np.random.default_rng(1).permutation(cfg["T"])
    outp = run_layer(L, x[perm], ids[perm], w[perm], dev, scatter)
    assert (outp - out[torch.from_numpy(perm).to(dev)]).norm().item() <= 1e-6 * out.norm().item()
    if scatter == "combine":      # every route's row is computed position-independently and summed in slot order
        assert torch.equal(outp.view(torch.int32), out[torch.from_numpy(perm).to(dev)].view(torch.int32))


@pytest.mark.parametrize("scatter", [None, "atomic"])
@pytest.mark.parametrize("T", [1024, 2048, 4096])
def test_headline_routing_sweep_sampled_tokens(dev, T, scatter):
    """The headline layer and Zipf routing at the sweep's smaller chunks, sampled tokens
    against the expert loop, through the shipped output method (None: "auto", the combine from 16384 routes) and the
    atomic scatter."""
    L, x, ids, w, cfg = synth.make_config("headline", seed=0, T=T)
    out = run_layer(L, x, ids, w, dev, scatter).cpu().numpy()
    tokens = np.random.default_rng(T).choice(cfg["T"], 64, replace=False)
    assert O.rel_l2(out[tokens], sampled_loop(L, x, ids, w, tokens)) < 1e-3


@pytest.mark.parametrize("name,T,bits", [("headline", 2048, None), ("headline", 8192, None), ("repro", 256, None),
                                         ("repro", 2048, None), ("headline", 2048, 3), ("headline", 2048, 2)])
def test_full_output_vs_expert_loop(dev, name, T, bits):
    """Every token of the output through the shipped output method (scatter None: "auto") against the expert loop,
    as the reference checks its grouped path (kernel/test_grouped.py:148-155: the whole output at 256 and 2048 tokens,
    skewed routing, which the repro config restates): the headline layer and Zipf routing at 2048 tokens and at the
    full 8192-token chunk, the reference's own shape (I = 1024, skewed routing), and the
    headline layer with 3- and 2-bit trellis codes (configs[4] repeats the hot path at those widths)."""
    L, x, ids, w, cfg = synth.make_config(name, seed=0, T=T, bits=bits)
    out = run_layer(L, x, ids, w, dev).cpu().numpy()
    ref = O.expert_loop(x, ids, w, to_np_layer(L), LIMIT)
    err = O.rel_l2(out, ref)
    print(f"{name} T={T} bits={cfg['bits']} scatter={rt.resolve_scatter(None, T * cfg['topk'])}: rel L2 vs expert "
          f"loop {err:.3e} over {T} tokens", flush=True)
    assert np.isfinite(out).all()
    assert err < 1e-3


def test_repro_config_sampled_tokens(dev):
    """The reference's published shape (I = 1024 per rank, skewed routing) at 1024 tokens, sampled tokens against
    the expert loop."""
    L, x, ids, w, cfg = synth.make_config("repro", seed=0, T=1024)
    out = run_layer(L, x, ids, w, dev).cpu().numpy()
    tokens = np.random.default_rng(7).choice(cfg["T"], 16, replace=False)
    assert O.rel_l2(out[tokens], sampled_loop(L, x, ids, w, tokens)) < 1e-3


@pytest.mark.parametrize("scatter", [None, "atomic"])       # None: the shipped "auto" (combine at 57344 routes)
@pytest.mark.parametrize("svh_scale", [1.0, 1 / 64])          # 1/64: pre-activations inside the clamp (SiLU region)
@pytest.mark.parametrize("bits", [4, 3, 2])
def test_thin_config_all_bits(dev, bits, svh_scale, scatter):
    L, x, ids, w, cfg = synth.make_config("thin", seed=0, bits=bits, svh_scale=svh_scale)
    out = run_layer(L, x, ids, w, dev, scatter).cpu().numpy()
    tokens = np.random.default_rng(bits).choice(cfg["T"], 16, replace=False)
    assert O.rel_l2(out[tokens], sampled_loop(L, x, ids, w, tokens)) < 1e-3


def test_prefill_workspace_reuse(dev, monkeypatch):
    """The prefill intermediates come from one per-device buffer reused across calls of different sizes (grown when a
    call needs more, the outgrown buffer released unless kept for captured graphs): results match the per-call-allocation
    path up to the atomic summation order."""
    L, x, ids, w, cfg = synth.make_config("layer1k", seed=3, svh_scale=1 / 64)
    TL = synth.to_device(L, dev)
    xt, it, wt = t16(x, dev), t16(ids, dev), t16(w, dev)
    rt._prefill_ws.clear()
    rt._prefill_ws_outgrown.clear()
    rt.keep_outgrown_prefill_workspaces(False)
    key = torch.cuda.current_device()
    sizes = (300, 1024, 300, 1024, 700)
    got = [rt.grouped_prefill(xt[:sizes[0]], it[:sizes[0]], wt[:sizes[0]], TL, LIMIT)]
    for n in sizes[1:]:
        got.append(rt.grouped_prefill(xt[:n], it[:n], wt[:n], TL, LIMIT))
    ws = rt._prefill_ws[key]
    assert not rt._prefill_ws_outgrown.get(key) and rt.live_prefill_workspaces(dev) == 1   # outgrown: released
    got.append(rt.grouped_prefill(xt[:500], it[:500], wt[:500], TL, LIMIT))
    assert rt._prefill_ws[key].data_ptr() == ws.data_ptr()                     # no growth for smaller calls
    # kept for captured graphs on request
    big = rt.reserve_prefill_workspace(dev, 2 * x.shape[0], cfg["topk"], cfg["E"], cfg["H"], cfg["I"],
                                       keep_outgrown=True)
    assert big.numel() > ws.numel() and rt._prefill_ws[key].data_ptr() == big.data_ptr()
    assert [b.data_ptr() for b in rt._prefill_ws_outgrown[key]] == [ws.data_ptr()]
    rt.release_outgrown_prefill_workspaces()
    rt.keep_outgrown_prefill_workspaces(False)
    assert not rt._prefill_ws_outgrown and rt.live_prefill_workspaces(dev) == 1
    del ws
    rt.grouped_prefill(xt, it, wt, TL, LIMIT)
    assert rt._prefill_ws[key].data_ptr() == big.data_ptr()                    # reserved: the full chunk fits
    sizes = sizes + (500,)
    monkeypatch.setenv("EXL3_GROUPED_WORKSPACE", "0")
    for n, g in zip(sizes, got):
        ref = rt.grouped_prefill(xt[:n], it[:n], wt[:n], TL, LIMIT)
        assert ((g - ref).norm() / ref.norm()).item() < 1e-6, n


@pytest.mark.parametrize("scatter", ["atomic", "combine"])
def test_prefill_graph_capture_replays(dev, scatter):
    """grouped_prefill captured in a HIP graph (the prefill workspace already sized; the output clear is a kernel, no
    memset node): replays with fresh inputs in the captured buffers match eager calls, with eager work between the
    replays, for both down-projection output methods."""
    L, x, ids, w, cfg = synth.make_config("tiny", seed=11)
    TL = synth.to_device(L, dev)
    xs, it, wt = t16(x, dev), t16(ids, dev), t16(w, dev)
    rt.grouped_prefill(xs, it, wt, TL, LIMIT, scatter=scatter)
    torch.cuda.synchronize()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            out = rt.grouped_prefill(xs, it, wt, TL, LIMIT, scatter=scatter)
    torch.cuda.current_stream().wait_stream(cap)
    for seed in (1, 2, 3):
        ids2, w2 = synth.make_routing(cfg["routing"], cfg["T"], cfg["E"], cfg["topk"], seed=seed)
        xs.copy_(t16(synth.make_x(cfg["T"], cfg["H"], seed), dev))
        it.copy_(t16(ids2, dev))
        wt.copy_(t16(w2, dev))
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        ref = rt.grouped_prefill(xs.clone(), it.clone(), wt.clone(), TL, LIMIT, scatter=scatter)
        torch.cuda.synchronize()
        assert ((got - ref).norm() / ref.norm()).item() < 1e-6, seed
        if scatter == "combine":                                  # fixed summation order: bit-identical
            assert torch.equal(got, ref), seed


def test_install_engages_grouped_path(dev, monkeypatch):
    L, x, ids, w, cfg = synth.make_config("tiny", seed=5)
    ov = Fake()
    ov.SWIGLU_LIMIT_DEFAULT = LIMIT
    ov.apply_exl3_experts = lambda *a, **k: "original"
    rt.install(ov)
    TL = synth.to_device(L, dev)
    TL._exl3_fused_temps = [torch.zeros(1, 64)]
    xb = t16(x, dev).to(torch.bfloat16)
    got = ov.apply_exl3_experts(xb, t16(ids, dev).to(torch.int32), t16(w, dev), TL, limit=LIMIT)
    assert got.dtype == torch.bfloat16 and TL._exl3_last_apply == "grouped"
    ref = rt.grouped_prefill(xb, t16(ids, dev), t16(w, dev), TL, LIMIT)
    assert torch.allclose(got.float(), ref.to(torch.bfloat16).float())
    small = ov.apply_exl3_experts(xb[:64], t16(ids, dev)[:64], t16(w, dev)[:64], TL)   # tokens <= cap: decode path
    assert small.dtype == torch.bfloat16 and TL._exl3_last_apply == "decode"
    monkeypatch.setenv("EXL3_GROUPED_DECODE", "0")
    assert ov.apply_exl3_experts(xb[:64], t16(ids, dev)[:64], t16(w, dev)[:64], TL) == "original"
