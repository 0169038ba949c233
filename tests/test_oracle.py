"""Pins the CPU oracle (oracle/exl3_oracle.{c,py}) before it is trusted as the checker.

Every check compares the oracle with something it did not compute itself: numpy / scipy library routines,
closed forms worked by hand, brute force over the abstract definition, or invariants a plausible slip
(wrong shift, transposed index, dropped term, wrong sign) would break. The committed fixtures in
tests/golden/ (made by tests/golden/make_golden.py) pin the oracle and the generators across rounds.
"""
import hashlib
import json
import math
import os

import numpy as np
import pytest
import scipy.linalg

import exl3_oracle as O
from exl3_grouped import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ------------------------------------------------------------------------------------------- fp16
def test_f16_to_f32_all_patterns_match_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.empty(65536, np.float32)
    O.lib().orc_f16_to_f32_array(O._p(bits), O._p(got), 65536)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(np.isinf(got), np.isinf(ref))


def test_f32_to_f16_rne_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 200000),
        # exact ties between fp16 neighbours (round half to even), subnormal range, overflow edge
        (np.arange(1, 4000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),
        np.float32(2.0 ** -24) * (np.arange(0, 3000, dtype=np.float32) / 4),
        np.array([65504, 65519.99, 65520, 65536, 1e9, -65520, 2 ** -25, 2 ** -25 * 1.0001, 0.0, -0.0],
                 dtype=np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f32_to_f16(x), ref)


# ------------------------------------------------------------------------------------------- trellis decode
def _numpy_decode(states: np.ndarray) -> np.ndarray:
    """decode() written again with numpy integer and float16 arithmetic (independent of the C code)."""
    x = (states.astype(np.uint64) * 0xCBAC1FED) & 0xFFFFFFFF
    y = (x & 0x8FFF8FFF) ^ 0x3B603B60
    lo = (y & 0xFFFF).astype(np.uint16).view(np.float16)
    hi = (y >> 16).astype(np.uint16).view(np.float16)
    return (lo + hi).view(np.uint16)


def test_decode_worked_examples():
    # state 0: x = 0 -> both halves 0x3B60 = 0.921875 -> 1.84375 = 0x3F60
    assert O.lib().orc_decode_state_mcg(0) == 0x3F60
    # state 1: x = 0xCBAC1FED -> y = (0x8BAC0FED ^ 0x3B603B60) = 0xB0CC348D
    #   lo 0x348D = 0.28448..., hi 0xB0CC = -0.14990... -> fp16 sum
    lo = np.array([0x348D], np.uint16).view(np.float16)[0]
    hi = np.array([0xB0CC], np.uint16).view(np.float16)[0]
    assert O.lib().orc_decode_state_mcg(1) == np.float16(lo + hi).view(np.uint16)


def test_decode_lut_matches_independent_numpy():
    lut = O.decode_lut()
    assert np.array_equal(lut, _numpy_decode(np.arange(65536, dtype=np.uint32)))
    v = lut.view(np.float16).astype(np.float64)
    assert np.all(np.isfinite(v)) and np.abs(v).max() < 4.0        # each half is in +-[1/8, 2)
    assert abs(v.mean()) < 0.05 and 0.8 < v.std() < 1.6


def test_tile_position_map_is_a_bijection_and_matches_the_fragment_layout():
    seen = set()
    for p in range(256):
        k, n = O.tile_pos_to_kn(p)
        assert 0 <= k < 16 and 0 <= n < 16
        seen.add((k, n))
        l, j = divmod(p, 8)
        r0 = 2 * (l % 4)
        assert k == [r0, r0 + 1, r0 + 8, r0 + 9][j % 4]
        assert n == l // 4 + (8 if j >= 4 else 0)
    assert len(seen) == 256
    assert [O.tile_pos_to_kn(p) for p in (0, 1, 2, 3, 4, 8, 32)] == [(0, 0), (1, 0), (8, 0), (9, 0), (0, 8),
                                                                     (2, 0), (0, 1)]


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_trellis_is_a_tail_biting_shift_register(bits):
    """state[p] = ((state[p-1] >> K) | (sym[p] << (16 - K))) & 0xFFFF for every p, p - 1 taken mod 256."""
    rng = np.random.default_rng(bits)
    for _ in range(20):
        sym = rng.integers(0, 1 << bits, 256, dtype=np.uint8)
        st = O.tile_states(O.pack_tile(sym, bits), bits).astype(np.int64)
        assert np.array_equal(st >> (16 - bits), sym)
        prev = np.roll(st, 1)
        assert np.array_equal(st, ((prev >> bits) | (sym.astype(np.int64) << (16 - bits))) & 0xFFFF)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_state_window_reads_little_endian_dwords(bits):
    """A single set bit at stream position b shows up in exactly the states whose window covers b."""
    L = 256 * bits
    for b in (0, 1, 15, 16, 31, 32, 33, L - 17, L - 1):
        w = np.zeros(16 * bits, np.uint16)
        w[b // 16] = 1 << (b % 16)
        st = O.tile_states(w, bits)
        for p in range(256):
            start = (p + 1) * bits - 16
            off = (b - start) % L
            expect = (1 << off) if off < 16 else 0
            assert st[p] == expect, (bits, b, p)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_reconstruct_matches_spec_composition(bits):
    rng = np.random.default_rng(10 + bits)
    pk = rng.integers(0, 65536, (3, 5, 16 * bits), dtype=np.uint16)
    W = O.reconstruct(pk).view(np.uint16)
    lut = O.decode_lut()
    for tk in range(3):
        for tn in range(5):
            st = O.tile_states(pk[tk, tn], bits)
            for p in range(256):
                k, n = O.tile_pos_to_kn(p)
                assert W[16 * tk + k, 16 * tn + n] == lut[st[p]]


def test_decode_golden_fixture():
    g = json.load(open(os.path.join(GOLDEN, "decode.json")))
    lut = O.decode_lut()
    assert hashlib.sha256(lut.tobytes()).hexdigest() == g["lut_sha"]
    assert lut[::64].tolist() == g["lut_sample_every_64"]
    for bits, t in g["tiles"].items():
        pk = np.array(t["packed"], np.uint16).reshape(t["shape"])
        assert hashlib.sha256(O.reconstruct(pk).view(np.uint16).tobytes()).hexdigest() == t["w_sha"]


# ------------------------------------------------------------------------------------------- routing
def test_sort_routes_matches_numpy_stable_argsort():
    rng = np.random.default_rng(3)
    for T, k, E in [(1, 1, 1), (7, 2, 3), (128, 8, 288), (1000, 8, 16), (333, 6, 1024)]:
        ids = rng.integers(0, E, (T, k))
        w = rng.random((T, k)).astype(np.float32)
        ts, ws, eor, counts, row0 = O.sort_routes(ids, w, E)
        order = np.argsort(ids.reshape(-1), kind="stable")
        assert np.array_equal(ts, np.repeat(np.arange(T), k)[order])
        assert np.array_equal(ws.view(np.uint16), w.reshape(-1)[order].astype(np.float16).view(np.uint16))
        assert np.array_equal(eor, ids.reshape(-1)[order])
        assert np.array_equal(counts, np.bincount(ids.reshape(-1), minlength=E))
        assert np.array_equal(row0, np.cumsum(counts) - counts)


def test_sort_routes_edges():
    ts, ws, eor, counts, row0 = O.sort_routes(np.zeros((0, 8), np.int64), np.zeros((0, 8), np.float32), 4)
    assert ts.size == 0 and counts.tolist() == [0, 0, 0, 0] and row0.tolist() == [0, 0, 0, 0]
    with pytest.raises(ValueError):
        O.sort_routes(np.array([[0, 5]]), np.ones((1, 2), np.float32), 4)


def _brute_blocks(counts, max_blocks, tile_rows=128):
    be, br = [], []
    row = 0
    for e, c in enumerate(counts):
        for i in range(math.ceil(c / tile_rows)):
            be.append(e)
            br.append(row + tile_rows * i)
        row += c
    return be, br, len(be), row


@pytest.mark.parametrize("tile_rows", [128, 64, 256, 512])
@pytest.mark.parametrize("seed", range(5))
def test_build_blocks_brute_force(seed, tile_rows):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(1, 300))
    counts = rng.integers(0, 700, E).astype(np.int32) * (rng.random(E) < 0.7)
    R = int(counts.sum())
    for max_blocks in (R // tile_rows + E, max(1, R // 512)):
        be, br, meta = O.build_blocks(counts, max_blocks, init=-7, tile_rows=tile_rows)
        rbe, rbr, nb, nrows = _brute_blocks(counts, max_blocks, tile_rows)
        assert meta.tolist() == [nb, nrows]
        m = min(nb, max_blocks)
        assert be[:m].tolist() == rbe[:m] and br[:m].tolist() == rbr[:m]
        assert np.all(be[m:] == -1) and np.all(br[m:] == -7)        # tail expert -1, row0 left unwritten
    assert nb <= R // tile_rows + E


# ------------------------------------------------------------------------------------------- Hadamard / act
def test_had128_is_scipy_hadamard_and_an_involution():
    H = scipy.linalg.hadamard(128).astype(np.float64) / math.sqrt(128)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 384))
    ref = np.concatenate([x[:, i * 128:(i + 1) * 128] @ H for i in range(3)], axis=1)
    assert np.allclose(O.had128(x), ref, rtol=1e-10, atol=1e-10)
    assert np.allclose(O.had128(O.had128(x)), x, rtol=1e-9, atol=1e-9)


def test_swiglu_clamped_closed_form():
    L = 10.0
    g = np.array([0.0, 1.0, -3.0, 25.0, -40.0, 10.0], np.float32)
    u = np.array([2.0, -20.0, 0.5, 3.0, 1.0, 11.0], np.float32)
    ref = [0.0, (1 / (1 + math.exp(-1))) * -10.0, (-3 / (1 + math.exp(3))) * 0.5,
           (10 / (1 + math.exp(-10))) * 3.0, (-40 / (1 + math.exp(40))) * 1.0, (10 / (1 + math.exp(-10))) * 10.0]
    assert np.allclose(O.swiglu_clamped(g, u, L), ref, rtol=1e-6, atol=1e-12)


# ------------------------------------------------------------------------------------------- layer
def _micro(seed=0, svh_scale=1.0):
    L = synth.make_layer(3, 256, 128, 4, seed, svh_scale)
    layer = O.Layer(L.w13_trellis, L.w13_suh, L.w13_svh, L.w2_trellis, L.w2_suh, L.w2_svh)
    x = synth.make_x(16, 256, seed)
    ids, w = synth.routing_softmax(16, 3, 2, seed)
    return layer, x, ids, w


def _real_weight(t, suh, svh):
    """W = diag(suh) H W' H diag(svh) with scipy's Hadamard, built explicitly (harness/proto_fp8.py:66-76)."""
    H = scipy.linalg.hadamard(128).astype(np.float64) / math.sqrt(128)
    Wp = O.reconstruct(t).astype(np.float64)
    K, N = Wp.shape
    Hk = np.kron(np.eye(K // 128), H)
    Hn = np.kron(np.eye(N // 128), H)
    return np.diag(suh.astype(np.float64)) @ Hk @ Wp @ Hn @ np.diag(svh.astype(np.float64))


@pytest.mark.parametrize("svh_scale", [1.0, 1.0 / 16])
def test_expert_loop_equals_token_major_brute_force(svh_scale):
    layer, x, ids, w = _micro(1, svh_scale)
    got = O.expert_loop(x, ids, w, layer, 10.0)
    E = layer.n_experts
    Wg = [_real_weight(layer.w13_trellis[e, 0], layer.w13_suh[e, 0], layer.w13_svh[e, 0]) for e in range(E)]
    Wu = [_real_weight(layer.w13_trellis[e, 1], layer.w13_suh[e, 1], layer.w13_svh[e, 1]) for e in range(E)]
    Wd = [_real_weight(layer.w2_trellis[e], layer.w2_suh[e], layer.w2_svh[e]) for e in range(E)]
    ref = np.zeros((x.shape[0], x.shape[1]))
    for t in range(x.shape[0]):
        h = x[t].astype(np.float64)
        for j in range(ids.shape[1]):
            e = ids[t, j]
            g = O.round_f16(h @ Wg[e])
            u = O.round_f16(h @ Wu[e])
            a = O.round_f16(O.swiglu_clamped(g, u, 10.0))
            ref[t] += (a.astype(np.float64) @ Wd[e]) * float(np.float16(w[t, j]))
    assert O.rel_l2(got, ref) < 1e-4


@pytest.mark.parametrize("svh_scale", [1.0, 1.0 / 16])
def test_staged_oracle_tracks_expert_loop(svh_scale):
    layer, x, ids, w = _micro(2, svh_scale)
    staged = O.grouped_prefill(x, ids, w, layer, 10.0)
    loop = O.expert_loop(x, ids, w, layer, 10.0)
    assert O.rel_l2(staged, loop) < 1e-3


@pytest.mark.parametrize("svh_scale", [1.0, 1.0 / 64])
def test_staged_distance_from_loop_is_its_two_rounding_points(svh_scale):
    """The staged path (the grouped kernels' stages) differs from the real-domain loop only by its two extra fp16
    rounding points, the rotated input rows and the rotated activation: the loop with both added equals the staged
    oracle (both with fp64 GEMMs), and the rotated input's rounding carries most of the distance."""
    from exl3_grouped import synth
    L, x, ids, w, cfg = synth.make_config("tiny", seed=0, svh_scale=svh_scale)
    layer = O.Layer(L.w13_trellis, L.w13_suh, L.w13_svh, L.w2_trellis, L.w2_suh, L.w2_svh)
    cache = O.WeightCache(layer)
    loop = O.expert_loop(x, ids, w, layer, 10.0, cache=cache)
    both = O.expert_loop(x, ids, w, layer, 10.0, cache=cache, dtype=np.float64, round_h13=True, round_act=True)
    h13 = O.expert_loop(x, ids, w, layer, 10.0, cache=cache, round_h13=True)
    act = O.expert_loop(x, ids, w, layer, 10.0, cache=cache, round_act=True)
    staged = O.grouped_prefill(x, ids, w, layer, 10.0)
    assert O.rel_l2(both, staged) < 1e-6
    d = O.rel_l2(staged, loop)
    assert 2e-4 < d < 1e-3
    assert O.rel_l2(h13, loop) > 0.8 * d > O.rel_l2(act, loop)


def test_gemm_stage_commutes_with_real_domain_weight():
    """mode-0 stage on H(x*suh) equals x @ W_real before rounding: pins the Hadamard side and the svh axis."""
    layer, x, ids, w = _micro(3)
    e = 1
    Wg = _real_weight(layer.w13_trellis[e, 0], layer.w13_suh[e, 0], layer.w13_svh[e, 0])
    h = O.had128(x.astype(np.float64) * layer.w13_suh[e, 0].astype(np.float64))
    y = O.expert_gemm(h, O.reconstruct(layer.w13_trellis[e, 0]).astype(np.float64), layer.w13_svh[e, 0])
    assert np.allclose(y, x.astype(np.float64) @ Wg, rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_linear_is_x_times_real_domain_weight(bits):
    """The dense linear equals x @ diag(suh) H W' H diag(svh) up to the fp16 rounding of h."""
    rng = np.random.default_rng(bits)
    K, N, M = 256, 384, 24
    x = rng.standard_normal((M, K)).astype(np.float16)
    packed = synth._random_words(rng, (K // 16, N // 16, 16 * bits))
    suh = synth._signs(rng, (K,))
    svh = synth._svh(rng, (N,))
    got = O.linear(x, packed, suh, svh)
    ref = x.astype(np.float64) @ _real_weight(packed, suh, svh)
    assert O.rel_l2(got, ref) < 1e-3
    # the same without rounding h to fp16 matches to float64 accuracy: only that rounding separates the two
    h = O.had128(x.astype(np.float64) * suh.astype(np.float64))
    exact = O.expert_gemm(h, O.reconstruct(packed).astype(np.float64), svh)
    assert np.allclose(exact, ref, rtol=1e-9, atol=1e-9)


def test_fat_scatter_is_index_add_of_store():
    a, packed, svh = synth.make_fat(0, M=40, K=128, N=128)
    y = O.fat_gemm(a, packed, svh)
    tok = np.array([(7 * i) % 50 for i in range(40)])
    rw = (np.arange(40) % 5 + 1).astype(np.float16) / 8
    out0 = np.random.default_rng(0).standard_normal((50, 128)).astype(np.float32)
    got = O.fat_gemm_scatter(a, packed, svh, tok, rw, out0)
    ref = out0.astype(np.float64).copy()
    for i in range(40):
        ref[tok[i]] += float(rw[i]) * y[i].astype(np.float64)
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-5)


def test_tiny_golden_fixture():
    g = np.load(os.path.join(GOLDEN, "tiny.npz"))
    L, x, ids, w, cfg = synth.make_config("tiny", seed=0)
    hashes = json.loads(str(g["input_sha"]))
    arrays = dict(w13_trellis=L.w13_trellis, w13_suh=L.w13_suh, w13_svh=L.w13_svh, w2_trellis=L.w2_trellis,
                  w2_suh=L.w2_suh, w2_svh=L.w2_svh, x=x)
    for k, v in arrays.items():
        assert hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest() == hashes[k], k
    assert np.array_equal(ids, g["ids"]) and np.array_equal(w, g["weights"])
    layer = O.Layer(L.w13_trellis, L.w13_suh, L.w13_svh, L.w2_trellis, L.w2_suh, L.w2_svh)
    out, st = O.grouped_prefill(x, ids, w, layer, 10.0, return_stages=True)
    for k in ("token_sorted", "expert_of_row", "counts", "expert_row0"):
        assert np.array_equal(st[k], g[k]), k
    assert np.array_equal(st["weight_sorted"].view(np.uint16), g["weight_sorted"].view(np.uint16))
    be, br, meta = O.build_blocks(st["counts"], ids.size // 128 + cfg["E"], init=-7)
    assert np.array_equal(be, g["block_expert"]) and np.array_equal(br, g["block_row0"])
    assert np.array_equal(meta, g["meta"])
    for k in ("h13", "gu", "act"):          # fp16 stages: at most one fp16 ulp from BLAS summation order
        d = np.abs(st[k].astype(np.float32) - g[k].astype(np.float32))
        assert np.all(d <= np.abs(g[k].astype(np.float32)) * 2 ** -10 + 1e-6), k
    assert O.rel_l2(out, g["out"]) < 1e-5
    assert O.rel_l2(O.expert_loop(x, ids, w, layer, 10.0), g["loop"]) < 1e-5


# ------------------------------------------------------------------------------------------- router top-k
def test_route_topk_brute_force():
    rng = np.random.default_rng(5)
    T, E, k = 40, 37, 5
    logits = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    logits[3] = -5.0
    logits[3, [20, 9, 4]] = 1.25                                   # exact ties: lower expert id first
    bias = (rng.standard_normal(E) * 0.2).astype(np.float32)
    bias[[4, 9, 20]] = 0
    ids, w = O.route_topk(logits, bias, k, 2.5)
    for t in range(T):
        s = [1.0 / (1.0 + math.exp(-float(v))) for v in logits[t]]
        sel = [float(np.float32(np.float32(s[e]) + bias[e])) for e in range(E)]
        want = sorted(range(E), key=lambda e: (-sel[e], e))[:k]
        assert ids[t].tolist() == want
        sc = np.float32([s[e] for e in want])
        assert abs(float(w[t].sum()) - 2.5) < 1e-5                     # renormalised un-biased scores
        assert np.allclose(w[t], sc / sc.sum() * 2.5, rtol=1e-6)
    assert ids[3, :3].tolist() == [4, 9, 20]
    _, w_raw = O.route_topk(logits, bias, k, 2.5, renorm=False)
    s_sel = 1.0 / (1.0 + np.exp(-np.take_along_axis(logits.astype(np.float64), ids, 1)))
    assert np.allclose(w_raw, s_sel * 2.5, rtol=1e-6)                  # the bias only selects, never weighs
