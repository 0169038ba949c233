"""EXL3 checkpoint ingest and tensor-parallel slicing (exl3_grouped/checkpoint.py), on the CPU.

The reference's loaders (kernel/test_grouped.py:52-81) read a real GLM-5.3-Flash EXL3 checkpoint, which is not
available here; these tests write synthetic layers in the same per-expert key layout and check the round trip, the
slicing geometry, and the property the slicing must have: the tensor-parallel ranks' outputs sum to the unsliced
layer's output.
"""
import json
import os

import numpy as np
import pytest
import torch

import exl3_oracle as O
from exl3_grouped import checkpoint as C
from exl3_grouped import synth


def _write(tmp_path, L, layer=3, **kw):
    C.write_moe_layer(str(tmp_path), layer, L.w13_trellis, L.w13_suh, L.w13_svh, L.w2_trellis, L.w2_suh, L.w2_svh,
                      **kw)
    return str(tmp_path)


def _np_layer(W):
    return O.Layer(*(t.numpy() for t in (W.w13_trellis, W.w13_suh, W.w13_svh, W.w2_trellis, W.w2_suh, W.w2_svh)))


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_round_trip_unsliced(tmp_path, bits):
    L = synth.make_layer(E=5, H=256, I=256, bits=bits, seed=bits)
    d = _write(tmp_path, L, experts_per_shard=2)
    W = C.load_moe_layer(d, 3)
    for name in ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh", "w2_svh"):
        assert np.array_equal(getattr(W, name).numpy(), getattr(L, name)), name
    assert W._exl3_bits == bits and W._exl3_hidden_size == 256 and W._exl3_intermediate_local == 256
    index = json.load(open(os.path.join(d, "model.safetensors.index.json")))["weight_map"]
    assert len({v for v in index.values()}) == 3                         # 5 experts over shards of 2
    assert "model.layers.3.mlp.experts.4.down_proj.trellis" in index


def test_tp_slices_tile_the_unsliced_layer(tmp_path):
    L = synth.make_layer(E=3, H=512, I=512, bits=4, seed=7)
    d = _write(tmp_path, L)
    W = [C.load_moe_layer(d, 3, tp_rank=r, tp=2) for r in range(2)]
    assert W[0].w13_trellis.shape == (3, 2, 32, 16, 64) and W[0].w2_trellis.shape == (3, 16, 32, 64)
    assert W[0]._exl3_intermediate_local == 256 and W[0]._exl3_hidden_size == 512
    # column-parallel gate|up: output features (I) split; row-parallel down: input features (I) split
    assert np.array_equal(torch.cat([w.w13_trellis for w in W], dim=3).numpy(), L.w13_trellis)
    assert np.array_equal(torch.cat([w.w13_svh for w in W], dim=2).numpy(), L.w13_svh)
    assert all(np.array_equal(w.w13_suh.numpy(), L.w13_suh) for w in W)
    assert np.array_equal(torch.cat([w.w2_trellis for w in W], dim=1).numpy(), L.w2_trellis)
    assert np.array_equal(torch.cat([w.w2_suh for w in W], dim=1).numpy(), L.w2_suh)
    assert all(np.array_equal(w.w2_svh.numpy(), L.w2_svh) for w in W)


@pytest.mark.parametrize("tp", [2, 4])
def test_tp_ranks_sum_to_the_unsliced_layer(tmp_path, tp):
    """Every rank runs the whole op on its slice; the all-reduce of their outputs is the unsliced layer's output."""
    L = synth.make_layer(E=4, H=256, I=512, bits=4, seed=11, svh_scale=1 / 16)
    d = _write(tmp_path, L)
    x = synth.make_x(24, 256, 5)
    ids, w = synth.routing_softmax(24, 4, 2, 5)
    full = O.expert_loop(x, ids, w, _np_layer(C.load_moe_layer(d, 3)), 10.0)
    parts = [O.expert_loop(x, ids, w, _np_layer(C.load_moe_layer(d, 3, tp_rank=r, tp=tp)), 10.0) for r in range(tp)]
    assert O.rel_l2(np.sum(parts, axis=0), full) < 1e-6


def test_language_model_prefix_and_layer_filter(tmp_path):
    L = synth.make_layer(E=2, H=128, I=128, bits=4, seed=1)
    d = str(tmp_path)
    C.write_moe_layer(d, 7, L.w13_trellis, L.w13_suh, L.w13_svh, L.w2_trellis, L.w2_suh, L.w2_svh,
                      prefix="model.language_model.layers")
    L2 = synth.make_layer(E=2, H=128, I=128, bits=4, seed=2)
    C.write_moe_layer(d, 8, L2.w13_trellis, L2.w13_suh, L2.w13_svh, L2.w2_trellis, L2.w2_suh, L2.w2_svh)
    assert np.array_equal(C.load_moe_layer(d, 7).w2_trellis.numpy(), L.w2_trellis)
    assert np.array_equal(C.load_moe_layer(d, 8).w2_trellis.numpy(), L2.w2_trellis)
    with pytest.raises(ValueError, match="no routed-expert"):
        C.load_moe_layer(d, 9)


def _edit(d, fn):
    from safetensors.torch import load_file, save_file
    index = json.load(open(os.path.join(d, "model.safetensors.index.json")))["weight_map"]
    for shard in sorted(set(index.values())):
        path = os.path.join(d, shard)
        t = load_file(path)
        fn(t)
        save_file(t, path)


def test_rejections(tmp_path):
    L = synth.make_layer(E=2, H=256, I=256, bits=4, seed=3)
    d = _write(tmp_path / "a", L)
    with pytest.raises(ValueError, match="128-feature blocks"):
        C.load_moe_layer(d, 3, tp_rank=0, tp=4)                        # I = 256 is 2 blocks, not 4
    with pytest.raises(ValueError, match="rank"):
        C.load_moe_layer(d, 3, tp_rank=2, tp=2)

    def bad_mcg(t):
        t["model.layers.3.mlp.experts.1.up_proj.mcg"] = torch.tensor(12345, dtype=torch.int32)
    _edit(d, bad_mcg)
    with pytest.raises(ValueError, match="MCG multiplier"):
        C.load_moe_layer(d, 3)

    d2 = _write(tmp_path / "b", L)

    def split_suh(t):
        t["model.layers.3.mlp.experts.0.up_proj.suh"] = -t["model.layers.3.mlp.experts.0.up_proj.suh"]
    _edit(d2, split_suh)
    with pytest.raises(ValueError, match="share their input sign"):
        C.load_moe_layer(d2, 3)

    d3 = _write(tmp_path / "c", L)
    idx = os.path.join(d3, "model.safetensors.index.json")
    j = json.load(open(idx))
    del j["weight_map"]["model.layers.3.mlp.experts.1.down_proj.svh"]
    json.dump(j, open(idx, "w"))
    with pytest.raises(ValueError, match="missing down_proj.svh"):
        C.load_moe_layer(d3, 3)
