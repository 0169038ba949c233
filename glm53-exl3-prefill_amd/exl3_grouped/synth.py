"""Seeded synthetic inputs for the five BASELINE.json configs (numpy on the host; see to_device()).

A layer is one TP rank's share of a routed-expert MoE: trellis codes are uniform random 16-bit words,
suh are +-1 sign vectors (gate and up share theirs, as kernel/test_grouped.py:82-84 requires), svh are
+-1 * U(0.5, 1.5) in fp16. Activations are fp16 N(0, 1). Routing generators:
  softmax  router logits N(0,1) [T, E]; top-k, weights = softmax over the selected logits
  zipf     the same logits plus log p_zipf(rank_pi(e)), p_r ~ r^-s over a seeded permutation pi
  thin     explicit seeded allocation: 16 hot experts take ~60% of routes, ~200 experts get <= 16 rows
  skewed   kernel/test_grouped.py:95-106 routing_skewed(hot, share): weights U(0,1) normalised
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

CONFIGS = {
    # tiny layer, CPU-runnable
    "tiny": dict(E=8, H=512, I=256, bits=4, T=128, topk=2, routing="softmax"),
    # single-expert fat GEMM (exl3_fat_gemm drop-in), gate|up concatenated
    "fat": dict(M=4096, K=4096, N=1536, bits=4),
    # full 288-expert layer, 1024-token chunk
    "layer1k": dict(E=288, H=4096, I=768, bits=4, T=1024, topk=8, routing="softmax"),
    # headline, 8192 tokens, Zipf(1.1)-skewed top-8 (sweep 1K/2K/4K/8K)
    "headline": dict(E=288, H=4096, I=768, bits=4, T=8192, topk=8, routing="zipf", zipf_s=1.1),
    # thin-expert stress at 4 bpw (repeated at 3 and 2 bpw)
    "thin": dict(E=288, H=4096, I=768, bits=4, T=7168, topk=8, routing="thin"),
    # the shape of the reference's own published grouped-path numbers (README.md:41-44: I = 1024 per rank,
    # routing_skewed(hot=12, share=0.55), T = 1K / 2K / 4K / 8K), with synthetic codes in place of the checkpoint
    "repro": dict(E=288, H=4096, I=1024, bits=4, T=8192, topk=8, routing="skewed"),
}


@dataclass
class LayerNP:
    w13_trellis: np.ndarray   # int16 [E, 2, H/16, I/16, 16*bits]
    w13_suh: np.ndarray       # fp16 [E, 2, H]
    w13_svh: np.ndarray       # fp16 [E, 2, I]
    w2_trellis: np.ndarray    # int16 [E, I/16, H/16, 16*bits]
    w2_suh: np.ndarray        # fp16 [E, I]
    w2_svh: np.ndarray        # fp16 [E, H]
    bits: int = 4
    meta: dict = field(default_factory=dict)


def _random_words(rng: np.random.Generator, shape) -> np.ndarray:
    n = int(np.prod(shape))
    return np.frombuffer(rng.bytes(2 * n), dtype=np.int16).reshape(shape).copy()


def _signs(rng, shape) -> np.ndarray:
    return (rng.integers(0, 2, size=shape, dtype=np.int8) * 2 - 1).astype(np.float16)


def _svh(rng, shape, scale=1.0) -> np.ndarray:
    s = rng.integers(0, 2, size=shape, dtype=np.int8).astype(np.float32) * 2 - 1
    return (s * rng.uniform(0.5, 1.5, size=shape).astype(np.float32) * scale).astype(np.float16)


def make_layer(E: int, H: int, I: int, bits: int = 4, seed: int = 0, svh_scale: float = 1.0) -> LayerNP:
    """Stacked layer tensors from a seed. svh_scale < 1 (e.g. 1/sqrt(K)) keeps gate/up pre-activations O(1)
    so the SwiGLU clamp is actually exercised."""
    assert H % 128 == 0 and I % 128 == 0 and bits in (2, 3, 4)
    rng = np.random.default_rng(seed)
    w = 16 * bits
    w13 = _random_words(rng, (E, 2, H // 16, I // 16, w))
    w2 = _random_words(rng, (E, I // 16, H // 16, w))
    suh = _signs(rng, (E, H))
    w13_suh = np.stack([suh, suh], axis=1)
    w13_svh = _svh(rng, (E, 2, I), svh_scale)
    w2_suh = _signs(rng, (E, I))
    w2_svh = _svh(rng, (E, H), svh_scale)
    return LayerNP(w13, w13_suh, w13_svh, w2, w2_suh, w2_svh, bits, dict(E=E, H=H, I=I, seed=seed))


def make_x(T: int, H: int, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng(seed + 1000)
    return rng.standard_normal((T, H), dtype=np.float32).astype(np.float16)


def _topk_softmax(logits: np.ndarray, topk: int):
    idx = np.argpartition(-logits, topk - 1, axis=1)[:, :topk]
    sel = np.take_along_axis(logits, idx, axis=1)
    order = np.argsort(-sel, axis=1, kind="stable")
    idx = np.take_along_axis(idx, order, axis=1)
    sel = np.take_along_axis(sel, order, axis=1)
    w = np.exp(sel - sel.max(axis=1, keepdims=True))
    w = w / w.sum(axis=1, keepdims=True)
    return idx.astype(np.int64), w.astype(np.float32)


def routing_softmax(T: int, E: int, topk: int, seed: int = 0):
    rng = np.random.default_rng(seed + 2000)
    return _topk_softmax(rng.standard_normal((T, E), dtype=np.float32), topk)


def routing_zipf(T: int, E: int, topk: int, s: float = 1.1, seed: int = 0):
    rng = np.random.default_rng(seed + 3000)
    perm = rng.permutation(E)                       # expert e has popularity rank perm[e] + 1
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    bias = np.log(p[perm]).astype(np.float32)
    logits = rng.standard_normal((T, E), dtype=np.float32) + bias[None, :]
    return _topk_softmax(logits, topk)


def _distinct_draws(rng, T, topk, probs):
    E = probs.size
    ids = np.empty((T, topk), dtype=np.int64)
    cand = rng.choice(E, size=(T, 4 * topk + 16), p=probs)
    for t in range(T):
        seen = []
        for e in cand[t]:
            if e not in seen:
                seen.append(int(e))
                if len(seen) == topk:
                    break
        while len(seen) < topk:                      # vanishingly rare: top up uniformly
            e = int(rng.integers(0, E))
            if e not in seen:
                seen.append(e)
        ids[t] = seen
    return ids


def routing_thin(T: int, E: int, topk: int, seed: int = 0, n_hot: int = 16, hot_share: float = 0.60,
                 n_thin: int = 200, thin_rows: float = 8.0):
    """Config 5: hot experts share `hot_share` of the routes, `n_thin` experts get ~Poisson(thin_rows) rows
    (<= 16 for nearly all), the remaining experts share the rest."""
    rng = np.random.default_rng(seed + 4000)
    perm = rng.permutation(E)
    hot, thin, warm = perm[:n_hot], perm[n_hot:n_hot + n_thin], perm[n_hot + n_thin:]
    R = T * topk
    thin_share = n_thin * thin_rows / R
    p = np.zeros(E)
    p[hot] = hot_share / n_hot
    p[thin] = thin_share / n_thin
    p[warm] = (1.0 - hot_share - thin_share) / max(len(warm), 1)
    ids = _distinct_draws(rng, T, topk, p / p.sum())
    w = rng.random((T, topk)).astype(np.float32)
    return ids, (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


def routing_skewed(T: int, E: int, topk: int, seed: int = 0, hot: int = 12, share: float = 0.55):
    """kernel/test_grouped.py:95-106: with probability `share` a slot draws from the first `hot` experts,
    otherwise from all E; ids distinct per token; weights U(0,1) normalised."""
    rng = np.random.default_rng(seed + 5000)
    ids = np.empty((T, topk), dtype=np.int64)
    for t in range(T):
        pool = []
        while len(pool) < topk:
            e = int(rng.integers(0, hot)) if rng.random() < share else int(rng.integers(0, E))
            if e not in pool:
                pool.append(e)
        ids[t] = pool
    w = rng.random((T, topk)).astype(np.float32)
    return ids, (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


def make_routing(kind: str, T: int, E: int, topk: int, seed: int = 0, **kw):
    if kind == "softmax":
        return routing_softmax(T, E, topk, seed)
    if kind == "zipf":
        return routing_zipf(T, E, topk, kw.get("zipf_s", 1.1), seed)
    if kind == "thin":
        return routing_thin(T, E, topk, seed)
    if kind == "skewed":
        return routing_skewed(T, E, topk, seed)
    raise ValueError(f"unknown routing {kind}")


def make_config(name: str, seed: int = 0, T: int | None = None, bits: int | None = None, svh_scale: float = 1.0):
    """(layer, x, ids, weights, cfg) for a layer config; T / bits override the config's."""
    cfg = dict(CONFIGS[name])
    if T is not None:
        cfg["T"] = T
    if bits is not None:
        cfg["bits"] = bits
    layer = make_layer(cfg["E"], cfg["H"], cfg["I"], cfg["bits"], seed, svh_scale)
    x = make_x(cfg["T"], cfg["H"], seed)
    ids, w = make_routing(cfg["routing"], cfg["T"], cfg["E"], cfg["topk"], seed, zipf_s=cfg.get("zipf_s", 1.1))
    return layer, x, ids, w, cfg


def make_fat(seed: int = 0, M: int = 4096, K: int = 4096, N: int = 1536, bits: int = 4):
    """Config 2: a [M, K] fp16 rows (already rotated), packed [K/16, N/16, 16 bits], svh [N]."""
    rng = np.random.default_rng(seed + 6000)
    a = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    packed = _random_words(rng, (K // 16, N // 16, 16 * bits))
    svh = _svh(rng, (N,))
    return a, packed, svh


class TorchLayer:
    """The attributes the reference's wrapper reads from a vLLM EXL3 MoE layer (kernel/test_grouped.py:89-91),
    as torch tensors on one device."""

    def __init__(self, L: LayerNP, device):
        import torch
        self.w13_trellis = torch.from_numpy(L.w13_trellis).to(device)
        self.w13_suh = torch.from_numpy(L.w13_suh).to(device)
        self.w13_svh = torch.from_numpy(L.w13_svh).to(device)
        self.w2_trellis = torch.from_numpy(L.w2_trellis).to(device)
        self.w2_suh = torch.from_numpy(L.w2_suh).to(device)
        self.w2_svh = torch.from_numpy(L.w2_svh).to(device)
        self._exl3_hidden_size = L.w13_trellis.shape[2] * 16
        self._exl3_intermediate_local = L.w13_trellis.shape[3] * 16
        self._exl3_bits = L.bits
        self.expert_map = None
        self._exl3_fused_temps = None


def to_device(L: LayerNP, device) -> TorchLayer:
    return TorchLayer(L, device)
