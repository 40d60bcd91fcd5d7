"""Synthetic sharded block-FP8 checkpoint for the weight-prep tests."""
from __future__ import annotations

import numpy as np

import oracle

PREFIX = "model.layers.3.mlp"


def synthetic_checkpoint(E: int, S: int, H: int, I: int, seed: int = 5):
    """numpy tensors {name: array or [shards]}: e4m3 codes as uint8, scales as
    bf16 bits (uint16) for even experts and fp32 for odd ones and the shared
    expert; gate/up/down of even experts split into two output shards."""
    rng = np.random.default_rng(seed)
    out = {}
    experts = list(range(E)) + [None] * S
    for e in experts:
        owner = "shared_expert" if e is None else f"experts.{e}"
        sharded = e is not None and e % 2 == 0
        for proj, (rows, cols) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            w = rng.integers(0, 256, size=(rows, cols), dtype=np.uint8)
            sc = (rng.random((rows // 128, cols // 128), dtype=np.float32) * 0.01 + 1e-4).astype(np.float32)
            if e is not None and e % 2 == 0:
                sc = oracle.bf16_from_f32(sc)  # uint16 bf16 bits
            key = f"{PREFIX}.{owner}.{proj}"
            if sharded:
                out[key + ".weight"] = [w[: rows // 2], w[rows // 2:]]
                out[key + ".weight_scale_inv"] = [sc[: rows // 256], sc[rows // 256:]] if rows >= 256 else sc
            else:
                out[key + ".weight"] = w
                out[key + ".weight_scale_inv"] = sc
    return out
