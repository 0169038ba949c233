"""EXL3 checkpoint ingest for the grouped MoE path: the per-expert safetensors tensors of one layer become the stacked
layer layout the grouped ops read, sliced for one tensor-parallel rank.

The reference's tests load a layer this way (kernel/test_grouped.py:52-81, harness/test_exl3_moe_op.py:80-90,
harness/proto_fp8.py:40-50): keys `model.[language_model.]layers.L.mlp.experts.e.{gate,up,down}_proj.{trellis,suh,svh,
mcg}` found through `model.safetensors.index.json`, gate/up sliced column-parallel and down row-parallel with the
overlay's `shard_exl3_col` / `shard_exl3_row`, then stacked:
  w13_trellis [E, 2, H/16, I/16, 16*bits]   w13_suh [E, 2, H]   w13_svh [E, 2, I]
  w2_trellis  [E, I/16, H/16, 16*bits]      w2_suh  [E, I]      w2_svh  [E, H]
(kernel/test_grouped.py:76-81), with gate.suh == up.suh required (:84).

The slicing rules here follow from the weight convention y = H128(H128(x * suh) . W') * svh: the Hadamards act on
128-feature blocks, so a rank takes whole 128-feature blocks. Column-parallel (gate/up) splits the output features:
the trellis along its N-tile axis and svh; suh is kept whole. Row-parallel (down) splits the input features: the trellis
along its K-tile axis and suh; svh is kept whole, and the ranks' partial outputs sum to the full output (the
all-reduce). The overlay's own functions are not available here; these are this build's restatement.
"""
from __future__ import annotations

import json
import os
import re
from dataclasses import dataclass, field

import numpy as np
import torch

KEY = re.compile(r"^model\.(?:language_model\.)?layers\.(\d+)\.mlp\.experts\.(\d+)\."
                 r"(gate_proj|up_proj|down_proj)\.(trellis|suh|svh|mcg|mul1)$")
MCG_MULT = 0xCBAC1FED                      # the MCG codebook multiplier the decoder implements
PROJS = ("gate_proj", "up_proj", "down_proj")


def _split(n: int, rank: int, tp: int, what: str) -> slice:
    if tp < 1 or not 0 <= rank < tp:
        raise ValueError(f"bad tensor-parallel rank {rank} of {tp}")
    if n % (128 * tp):
        raise ValueError(f"{what} ({n}) must split into whole 128-feature blocks over {tp} ranks")
    step = n // tp
    return slice(rank * step, (rank + 1) * step)


def shard_exl3_col(t: torch.Tensor, suffix: str, rank: int, tp: int) -> torch.Tensor:
    """Column-parallel slice of one EXL3 tensor (gate/up): output features split over `tp` ranks."""
    if tp == 1 or suffix in ("suh", "mcg", "mul1"):
        return t
    if suffix == "trellis":
        sl = _split(t.shape[1] * 16, rank, tp, "output features")
        return t[:, sl.start // 16:sl.stop // 16].contiguous()
    if suffix == "svh":
        return t[_split(t.shape[0], rank, tp, "output features")].contiguous()
    raise ValueError(f"unknown EXL3 tensor suffix {suffix!r}")


def shard_exl3_row(t: torch.Tensor, suffix: str, rank: int, tp: int) -> torch.Tensor:
    """Row-parallel slice of one EXL3 tensor (down): input features split over `tp` ranks."""
    if tp == 1 or suffix in ("svh", "mcg", "mul1"):
        return t
    if suffix == "trellis":
        sl = _split(t.shape[0] * 16, rank, tp, "input features")
        return t[sl.start // 16:sl.stop // 16].contiguous()
    if suffix == "suh":
        return t[_split(t.shape[0], rank, tp, "input features")].contiguous()
    raise ValueError(f"unknown EXL3 tensor suffix {suffix!r}")


def _check_mcg(name: str, t: torch.Tensor) -> None:
    """The `mcg` tensor marks the MCG codebook. Accepted: a true flag, or the multiplier itself (as a signed or
    unsigned 32-bit pattern); anything else is a codebook this decoder does not implement."""
    v = int(t.reshape(-1)[0].item()) if t.numel() else 0
    if t.dtype == torch.bool and v == 1:
        return
    if v in (1, MCG_MULT, MCG_MULT - (1 << 32)):
        return
    raise ValueError(f"{name}: MCG multiplier {v:#x} is not {MCG_MULT:#x}; only the MCG codebook is supported")


@dataclass
class MoELayerWeights:
    """The attributes the grouped path reads from a vLLM EXL3 MoE layer (kernel/exl3_grouped_runtime.py:56-58,74-82),
    loaded for one tensor-parallel rank."""
    w13_trellis: torch.Tensor
    w13_suh: torch.Tensor
    w13_svh: torch.Tensor
    w2_trellis: torch.Tensor
    w2_suh: torch.Tensor
    w2_svh: torch.Tensor
    meta: dict = field(default_factory=dict)

    def __post_init__(self):
        self._exl3_hidden_size = self.w13_trellis.shape[2] * 16
        self._exl3_intermediate_local = self.w13_trellis.shape[3] * 16
        self._exl3_bits = self.w13_trellis.shape[4] // 16
        self.expert_map = None
        self._exl3_fused_temps = None


def expert_keys(index: dict, layer: int) -> dict:
    """{(expert, proj, suffix): (tensor name, shard file)} for one layer of a safetensors index's weight_map."""
    out = {}
    for name, shard in index.items():
        m = KEY.match(name)
        if m and int(m.group(1)) == layer:
            out[(int(m.group(2)), m.group(3), m.group(4))] = (name, shard)
    return out


def load_moe_layer(model_dir: str, layer: int, tp_rank: int = 0, tp: int = 1, n_experts: int | None = None,
                   device="cpu") -> MoELayerWeights:
    """Read one layer's routed experts from an EXL3 checkpoint directory (model.safetensors.index.json + shards),
    slice them for `tp_rank` of `tp` and stack them. Tensors are read with safetensors (no code runs from the files)."""
    from safetensors import safe_open

    with open(os.path.join(model_dir, "model.safetensors.index.json")) as f:
        index = json.load(f)["weight_map"]
    keys = expert_keys(index, layer)
    experts = sorted({e for (e, _, _) in keys})
    if not experts:
        raise ValueError(f"no routed-expert EXL3 tensors for layer {layer} in {model_dir}")
    E = n_experts if n_experts is not None else experts[-1] + 1
    for e in range(E):
        for proj in PROJS:
            for suf in ("trellis", "suh", "svh"):
                if (e, proj, suf) not in keys:
                    raise ValueError(f"layer {layer} expert {e}: missing {proj}.{suf}")
            if (e, proj, "mul1") in keys:
                raise ValueError(f"layer {layer} expert {e} {proj}: the mul1 codebook is not supported (MCG only)")
            if (e, proj, "mcg") not in keys:
                raise ValueError(f"layer {layer} expert {e} {proj}: no mcg tensor; only the MCG codebook is supported")
    by_shard = {}
    for (e, proj, suf), (name, shard) in keys.items():
        if e < E:
            by_shard.setdefault(shard, []).append((name, e, proj, suf))
    raw = {}
    for shard, items in sorted(by_shard.items()):
        with safe_open(os.path.join(model_dir, shard), framework="pt", device="cpu") as f:
            for name, e, proj, suf in items:
                t = f.get_tensor(name)
                if suf == "mcg":
                    _check_mcg(name, t)
                    continue
                shard_fn = shard_exl3_row if proj == "down_proj" else shard_exl3_col
                raw[(e, proj, suf)] = shard_fn(t, suf, tp_rank, tp)
    bits = {raw[(e, p, "trellis")].shape[2] // 16 for e in range(E) for p in PROJS}
    if len(bits) != 1 or bits.pop() not in (2, 3, 4):
        raise ValueError("the layer's trellis tensors must share one width of 2, 3 or 4 bits")

    def stack(f):
        return torch.stack([f(e) for e in range(E)]).contiguous().to(device)

    w13_trellis = stack(lambda e: torch.stack([raw[(e, "gate_proj", "trellis")], raw[(e, "up_proj", "trellis")]]))
    w13_suh = stack(lambda e: torch.stack([raw[(e, "gate_proj", "suh")], raw[(e, "up_proj", "suh")]]))
    w13_svh = stack(lambda e: torch.stack([raw[(e, "gate_proj", "svh")], raw[(e, "up_proj", "svh")]]))
    if not torch.equal(w13_suh[:, 0], w13_suh[:, 1]):
        raise ValueError("gate and up must share their input sign vector (suh) for the stacked gate|up GEMM")
    return MoELayerWeights(w13_trellis, w13_suh, w13_svh,
                           stack(lambda e: raw[(e, "down_proj", "trellis")]),
                           stack(lambda e: raw[(e, "down_proj", "suh")]),
                           stack(lambda e: raw[(e, "down_proj", "svh")]),
                           dict(layer=layer, tp_rank=tp_rank, tp=tp, experts=E))


def write_moe_layer(model_dir: str, layer: int, w13_trellis, w13_suh, w13_svh, w2_trellis, w2_suh, w2_svh,
                    experts_per_shard: int = 64, prefix: str = "model.layers") -> None:
    """Write a stacked (unsliced) layer as per-expert EXL3 tensors in the checkpoint layout load_moe_layer reads,
    merging its keys into model_dir's model.safetensors.index.json. Inputs are numpy arrays or CPU tensors."""
    from safetensors.torch import save_file

    os.makedirs(model_dir, exist_ok=True)
    as_t = lambda a: torch.as_tensor(np.ascontiguousarray(a))  # noqa: E731
    w13_trellis, w13_suh, w13_svh = as_t(w13_trellis), as_t(w13_suh), as_t(w13_svh)
    w2_trellis, w2_suh, w2_svh = as_t(w2_trellis), as_t(w2_suh), as_t(w2_svh)
    E = w13_trellis.shape[0]
    mcg = torch.tensor(MCG_MULT - (1 << 32), dtype=torch.int32)
    idx_path = os.path.join(model_dir, "model.safetensors.index.json")
    index = {"metadata": {}, "weight_map": {}}
    if os.path.exists(idx_path):
        with open(idx_path) as f:
            index = json.load(f)
    for s0 in range(0, E, experts_per_shard):
        shard = f"layer{layer}-experts{s0:04d}.safetensors"
        tensors = {}
        for e in range(s0, min(E, s0 + experts_per_shard)):
            base = f"{prefix}.{layer}.mlp.experts.{e}."
            parts = {"gate_proj": (w13_trellis[e, 0], w13_suh[e, 0], w13_svh[e, 0]),
                     "up_proj": (w13_trellis[e, 1], w13_suh[e, 1], w13_svh[e, 1]),
                     "down_proj": (w2_trellis[e], w2_suh[e], w2_svh[e])}
            for proj, (t, suh, svh) in parts.items():
                for suf, v in (("trellis", t), ("suh", suh), ("svh", svh), ("mcg", mcg)):
                    tensors[base + proj + "." + suf] = v.contiguous().clone()
        save_file(tensors, os.path.join(model_dir, shard))
        for name in tensors:
            index["weight_map"][name] = shard
    with open(idx_path, "w") as f:
        json.dump(index, f, indent=1)
