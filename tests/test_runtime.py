"""Host-side logic that needs no GPU: the serving wrapper's pass-through rules
(kernel/exl3_grouped_runtime.py:91-107), the idempotent overlay hook (kernel/patch_exl3_grouped.py:6-22) and the
synthetic generators."""
import types

import numpy as np
import pytest
import torch

import exl3_grouped_runtime as rt
import patch_exl3_grouped as patcher
from exl3_grouped import synth


class FakeLayer(torch.nn.Module):
    pass


def fake_overlay():
    calls = []

    def original(x, topk_ids, topk_weights, layer, *, limit=10.0, fused=None):
        calls.append(dict(tokens=x.shape[-2], limit=limit, fused=fused))
        return "original"

    ov = types.SimpleNamespace(apply_exl3_experts=original, SWIGLU_LIMIT_DEFAULT=10.0)
    return ov, calls


def test_install_passes_through_decode_ep_and_non_trellis_layers(monkeypatch):
    ov, calls = fake_overlay()
    rt.install(ov)
    assert ov.apply_exl3_experts is not None and ov.apply_exl3_experts.__name__ == "apply_exl3_experts_grouped"
    x = torch.zeros(64, 512, dtype=torch.float16)
    ids = torch.zeros(64, 8, dtype=torch.long)
    w = torch.zeros(64, 8)
    # decode-sized call: tokens <= cap (cap = layer._exl3_fused_temps[0].shape[1]) goes to moe_decode, or to the
    # original path with EXL3_GROUPED_DECODE=0
    layer = FakeLayer()
    layer.w13_trellis = torch.zeros(4, 2, 32, 16, 64, dtype=torch.int16)
    layer._exl3_fused_temps = [torch.zeros(1, 128)]
    layer.expert_map = None
    decoded = []

    def fake_decode(x2d, ids2d, w2d, lay, limit, out=None, cap=None):
        decoded.append((tuple(x2d.shape), ids2d.dtype, limit, cap))
        return torch.ones(x2d.shape, dtype=torch.float32)

    monkeypatch.setattr(rt, "moe_decode", fake_decode)
    got = ov.apply_exl3_experts(x, ids.to(torch.int32), w, layer, limit=7.0, fused="f")
    assert got.dtype == torch.float16 and decoded == [((64, 512), torch.int64, 7.0, 128)]   # sized for the cap
    assert layer._exl3_last_apply == "decode" and not calls
    monkeypatch.setenv("EXL3_GROUPED_DECODE", "0")
    assert ov.apply_exl3_experts(x, ids, w, layer, limit=7.0, fused="f") == "original"
    assert calls[-1] == dict(tokens=64, limit=7.0, fused="f")
    # expert-parallel layer
    layer2 = FakeLayer()
    layer2.w13_trellis = layer.w13_trellis
    layer2.expert_map = torch.arange(4)
    assert ov.apply_exl3_experts(torch.zeros(300, 512), ids, w, layer2) == "original"
    # layer without trellis weights
    layer3 = FakeLayer()
    layer3.expert_map = None
    assert ov.apply_exl3_experts(torch.zeros(300, 512), ids, w, layer3) == "original"
    assert len(calls) == 3


def test_patch_hook_is_idempotent(tmp_path):
    target = tmp_path / "exl3.py"
    target.write_text("SWIGLU_LIMIT_DEFAULT = 10.0\n")
    assert patcher.patch(target, "/opt/somewhere") is True
    text = target.read_text()
    assert patcher.MARKER in text and "EXL3_GROUPED_PREFILL" in text and "/opt/somewhere" in text
    assert patcher.patch(target, "/opt/somewhere") is False
    assert target.read_text() == text
    compile(text, str(target), "exec")


def test_scatter_mode_resolution(monkeypatch):
    """"auto" (the default) takes the deterministic combine method from COMBINE_MIN_ROUTES routes up, the atomic scatter
    below; explicit modes pass through; anything else is rejected like the reference's checks."""
    monkeypatch.delenv("EXL3_GROUPED_SCATTER", raising=False)
    assert rt.scatter_mode() == "auto"
    n = rt.COMBINE_MIN_ROUTES
    assert rt.resolve_scatter(None, n) == "combine" and rt.resolve_scatter(None, n - 1) == "atomic"
    assert rt.resolve_scatter("auto", 8192 * 8) == "combine" and rt.resolve_scatter("auto", 1024 * 8) == "atomic"
    assert rt.resolve_scatter("atomic", 10 ** 6) == "atomic" and rt.resolve_scatter("combine", 8) == "combine"
    monkeypatch.setenv("EXL3_GROUPED_SCATTER", "atomic")
    assert rt.resolve_scatter(None, 10 ** 6) == "atomic"
    monkeypatch.setenv("EXL3_GROUPED_SCATTER", "bogus")
    with pytest.raises(RuntimeError, match="EXL3_GROUPED_SCATTER"):
        rt.resolve_scatter(None, 8)
    with pytest.raises(RuntimeError, match="scatter must be one of"):
        rt.resolve_scatter("sum", 8)
    monkeypatch.setenv("EXL3_GROUPED_SCATTER", "auto")
    monkeypatch.setenv("EXL3_GROUPED_COMBINE_MIN_ROUTES", "64")
    assert rt.resolve_scatter(None, 64) == "combine" and rt.resolve_scatter(None, 63) == "atomic"
    monkeypatch.setenv("EXL3_GROUPED_COMBINE_MIN_ROUTES", "-3")
    with pytest.raises(RuntimeError, match="COMBINE_MIN_ROUTES"):
        rt.resolve_scatter(None, 8)


def test_prefill_workspace_holds_the_combine_rows(monkeypatch):
    """The prefill plan sized for a chunk that "auto" sends down the combine path holds the per-route fp32 rows
    (routes x hidden) and the route index on top of what the atomic path needs; below the threshold it does not."""
    monkeypatch.delenv("EXL3_GROUPED_SCATTER", raising=False)
    gp = rt._load_ext()

    def size(T, scatter):
        c = rt._Carve()
        rt._prefill_plan(gp, T, 4096, 8, 288, 768, 256, rt.resolve_scatter(scatter, T * 8), True)(c)
        return c.off

    T = rt.COMBINE_MIN_ROUTES // 8
    extra = size(T, "auto") - size(T, "atomic")
    assert T * 8 * 4096 * 4 + T * 8 * 4 <= extra <= T * 8 * 4096 * 4 + T * 8 * 4 + 2 * 256
    assert size(T - 1, "auto") == size(T - 1, "atomic")


def test_prefill_workspace_is_bounded():
    """Twenty calls of rising size leave one live workspace per device: each growth takes at least WS_GROWTH times the
    old size and releases the outgrown buffer (kernel/exl3_grouped_runtime.py:69-80 allocates per call; the buffer here
    is reused). Kept outgrown buffers (graph-capture safety, on request) are freed by
    release_outgrown_prefill_workspaces."""
    dev = torch.device("cpu")
    rt._prefill_ws.clear()
    rt._prefill_ws_outgrown.clear()
    rt.keep_outgrown_prefill_workspaces(False)
    try:
        sizes = [int(1e6 * (1 + 0.1 * i)) for i in range(20)]
        grows, last = 0, None
        for n in sizes:
            ws = rt._prefill_workspace(dev, n)
            assert ws.numel() >= n and rt.live_prefill_workspaces(dev) == 1
            if last is not None and ws.numel() != last:
                assert ws.numel() >= rt.WS_GROWTH * last
                grows += 1
            last = ws.numel()
            del ws
        assert grows <= 6                     # 1e6 -> 2.9e6 in steps of >= 1.25x from a 2 MiB-aligned start
        assert not rt._prefill_ws_outgrown
        small = rt._prefill_workspace(dev, 1000)
        assert small.numel() == last          # never shrinks
        rt.keep_outgrown_prefill_workspaces(True)
        big = rt._prefill_workspace(dev, 4 * last)
        assert rt.live_prefill_workspaces(dev) == 2 and rt._prefill_ws_outgrown[-1][0] is small
        rt.release_outgrown_prefill_workspaces()
        assert rt.live_prefill_workspaces(dev) == 1 and rt._prefill_ws[-1] is big
    finally:
        rt.keep_outgrown_prefill_workspaces(False)
        rt._prefill_ws.clear()
        rt._prefill_ws_outgrown.clear()


def test_generators_are_deterministic():
    a = synth.make_config("tiny", seed=3)
    b = synth.make_config("tiny", seed=3)
    for u, v in zip(a[:4], b[:4]):
        if isinstance(u, np.ndarray):
            assert np.array_equal(u, v)
    assert np.array_equal(a[0].w13_trellis, b[0].w13_trellis)
    assert np.array_equal(a[0].w13_suh[:, 0], a[0].w13_suh[:, 1])       # gate/up share suh
    c = synth.make_config("tiny", seed=4)
    assert not np.array_equal(a[0].w13_trellis, c[0].w13_trellis)


@pytest.mark.parametrize("kind", ["softmax", "zipf", "thin", "skewed"])
def test_routing_shapes_and_distinct_ids(kind):
    ids, w = synth.make_routing(kind, 512, 288, 8, seed=1)
    assert ids.shape == (512, 8) and w.shape == (512, 8)
    assert ids.min() >= 0 and ids.max() < 288
    assert all(len(set(r)) == 8 for r in ids.tolist())
    assert np.allclose(w.sum(1), 1.0, atol=1e-5) and (w > 0).all()


def test_zipf_and_thin_skews():
    ids, _ = synth.routing_zipf(8192, 288, 8, 1.1, 0)
    c = np.sort(np.bincount(ids.ravel(), minlength=288))[::-1]
    assert c[0] > 0.9 * 8192 and c[:16].sum() > 0.7 * c.sum()
    ids, _ = synth.routing_thin(7168, 288, 8, 0)
    c = np.bincount(ids.ravel(), minlength=288)
    cs = np.sort(c)[::-1]
    assert 0.5 < cs[:16].sum() / c.sum() < 0.65          # 16 hot experts take ~60%
    assert 180 <= int((c <= 16).sum()) <= 220            # ~200 experts with <= 16 rows
    ids, _ = synth.routing_skewed(8192, 288, 8, 0)         # the reference's routing_skewed(hot=12, share=0.55)
    c = np.bincount(ids.ravel(), minlength=288)
    assert 0.48 < c[:12].sum() / c.sum() < 0.56            # 55% of draws go to the 12 hot experts, fewer slots after
    assert c[:12].min() > 10 * c[12:].max()                # duplicates within a token are redrawn
