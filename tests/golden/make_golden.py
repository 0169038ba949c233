#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/ from this repo's own CPU oracle and generators.

The reference ships no vectors, KATs or fixtures for this path (its tests need exllamav3, the vLLM overlay, a
real checkpoint and CUDA), so these fixtures pin the GPU <-> oracle relation and the generators across
rounds, not the oracle <-> exllamav3 relation (that stays "parity unpinned").

  tiny.npz      config 1: sha256 of every generated input, the routing, sort and
                block-table outputs (bit-exact), the stage outputs h13 / gu / act (fp16) and the layer output
                of both the staged oracle and the expert loop (fp32).
  decode.json   sha256 of the 65536-entry decode table, a 1024-entry sample, and decoded tiles of a fixed
                packed tensor at 2/3/4 bits.

Run: python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "glm53-exl3-prefill_amd")]

import exl3_oracle as O  # noqa: E402
from exl3_grouped import synth  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def tiny_case():
    L, x, ids, w, cfg = synth.make_config("tiny", seed=0)
    layer = O.Layer(L.w13_trellis, L.w13_suh, L.w13_svh, L.w2_trellis, L.w2_suh, L.w2_svh)
    return L, layer, x, ids, w, cfg


def main():
    L, layer, x, ids, w, cfg = tiny_case()
    out, st = O.grouped_prefill(x, ids, w, layer, O.SWIGLU_LIMIT_DEFAULT, return_stages=True)
    loop = O.expert_loop(x, ids, w, layer, O.SWIGLU_LIMIT_DEFAULT)
    R = ids.size
    be, br, meta = O.build_blocks(st["counts"], R // 128 + cfg["E"], init=-7)
    hashes = {k: sha(v) for k, v in dict(w13_trellis=L.w13_trellis, w13_suh=L.w13_suh, w13_svh=L.w13_svh,
                                         w2_trellis=L.w2_trellis, w2_suh=L.w2_suh, w2_svh=L.w2_svh, x=x).items()}
    np.savez_compressed(
        os.path.join(HERE, "tiny.npz"), input_sha=json.dumps(hashes), ids=ids, weights=w,
        token_sorted=st["token_sorted"], weight_sorted=st["weight_sorted"], expert_of_row=st["expert_of_row"],
        counts=st["counts"], expert_row0=st["expert_row0"], block_expert=be, block_row0=br, meta=meta,
        h13=st["h13"], gu=st["gu"], act=st["act"], out=out, loop=loop)

    lut = O.decode_lut()
    rng = np.random.default_rng(123)
    tiles = {}
    for bits in (2, 3, 4):
        pk = rng.integers(0, 65536, (2, 3, 16 * bits), dtype=np.uint16)
        tiles[str(bits)] = dict(packed=pk.reshape(-1).tolist(), shape=list(pk.shape),
                                w_sha=sha(O.reconstruct(pk).view(np.uint16)))
    with open(os.path.join(HERE, "decode.json"), "w") as f:
        json.dump(dict(lut_sha=sha(lut), lut_sample_every_64=lut[::64].tolist(), tiles=tiles), f)
    print("wrote tiny.npz and decode.json")


if __name__ == "__main__":
    main()
