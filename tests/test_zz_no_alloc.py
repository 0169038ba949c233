"""GPU test of exl3_moe_decode_noalloc, the decode entry point that allocates nothing (its workspace is the library's
fixed per-GPU scratch array): called through the C ABI, its output must equal exl3_moe_decode's (the same kernels on a
caller workspace) up to the fp32 atomic summation order, and meet the north-star rel L2 <= 1e-3 against the oracle
expert loop -- on two calls in a row, the second with fewer tokens (the scratch keeps the first call's contents)."""
import ctypes

import numpy as np
import pytest
import torch

import exl3_grouped as gp
import exl3_oracle as O
from exl3_grouped import _lib, synth

pytestmark = pytest.mark.gpu
LIMIT = 10.0
# Same kernels, same inputs: only the order of the fp32 atomic additions (K slices, scatter) differs between the two
# entry points, which can flip an fp16 rounding of gate|up by one step (about 1e-5 relative in the output).
RERUN_TOL = 1e-4


def noalloc(x, ids, w, TL, out):
    g, u = TL.w13_trellis[:, 0], TL.w13_trellis[:, 1]
    words = TL.w13_trellis.size(4)
    T, H = x.shape
    E, inter = TL.w13_trellis.size(0), TL.w13_trellis.size(3) * 16
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = _lib.load().exl3_moe_decode_noalloc(
        P(x), T, H, P(ids), _lib.DTYPE_I64, P(w), _lib.DTYPE_F32, ids.size(1), E, inter, words // 16, P(g), P(u),
        g.stride(0), P(TL.w13_suh[:, 0]), TL.w13_suh.stride(0), P(TL.w13_svh[:, 0]), P(TL.w13_svh[:, 1]),
        TL.w13_svh.stride(0), P(TL.w2_trellis), TL.w2_trellis.stride(0), P(TL.w2_suh), TL.w2_suh.stride(0),
        P(TL.w2_svh), TL.w2_svh.stride(0), ctypes.c_float(LIMIT), P(out), stream)
    return rc


def test_noalloc_matches_workspace_entry_point(dev):
    L, x_all, _, _, cfg = synth.make_config("layer1k", seed=0, T=1, svh_scale=1 / 64)
    TL = synth.to_device(L, dev)
    layer = O.Layer(L.w13_trellis, L.w13_suh, L.w13_svh, L.w2_trellis, L.w2_suh, L.w2_svh)
    for T, seed in ((96, 11), (5, 12), (2, 13)):         # each call smaller than the one before
        print(f"noalloc decode: T={T} seed={seed}", flush=True)
        x = synth.make_x(T, cfg["H"], seed)
        ids, w = synth.make_routing("softmax", T, cfg["E"], cfg["topk"], seed=seed)
        xt = torch.from_numpy(x).to(dev).half().contiguous()
        it = torch.from_numpy(ids).to(dev).contiguous()
        wt = torch.from_numpy(w).to(dev).float().contiguous()
        out = torch.full((T, cfg["H"]), float("nan"), dtype=torch.float32, device=dev)
        rc = noalloc(xt, it, wt, TL, out)
        assert rc == 0, _lib.load().exl3_last_error()
        ws = torch.empty(gp.moe_decode_workspace_bytes(T, cfg["topk"], cfg["E"], cfg["H"], cfg["I"]),
                         dtype=torch.uint8, device=dev)          # exl3_moe_decode: any workspace contents
        ref = gp.moe_decode(xt, it, wt, TL.w13_trellis, TL.w13_suh, TL.w13_svh, TL.w2_trellis, TL.w2_suh, TL.w2_svh,
                            LIMIT, workspace=ws)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.isfinite(got).all()
        assert O.rel_l2(got, ref.cpu().numpy()) < RERUN_TOL
        assert O.rel_l2(got, O.expert_loop(x, ids, w, layer, LIMIT)) < 1e-3


def test_noalloc_rejects_calls_beyond_its_scratch(dev):
    L, _, _, _, cfg = synth.make_config("layer1k", seed=0, T=1)
    TL = synth.to_device(L, dev)
    T = 512                                             # 512 tokens x top-8 at H=4096, I=768: ~62 MiB > 32 MiB
    x = torch.zeros(T, cfg["H"], dtype=torch.float16, device=dev)
    ids = torch.zeros(T, cfg["topk"], dtype=torch.int64, device=dev)
    w = torch.zeros(T, cfg["topk"], dtype=torch.float32, device=dev)
    out = torch.zeros(T, cfg["H"], dtype=torch.float32, device=dev)
    assert noalloc(x, ids, w, TL, out) == _lib.EXL3_ERR_ARG
    assert b"scratch" in _lib.load().exl3_last_error()
