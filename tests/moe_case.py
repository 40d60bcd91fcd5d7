"""Shared set-up for GPU parity tests, smoke() and the CPU baseline: seeded
inputs for one configuration, the engine run with every intermediate exposed,
and the oracle's answer on the same bytes."""
from __future__ import annotations

import numpy as np
import torch

import oracle
from netra_moe.config import MoEConfig
from netra_moe.engine import resolve_front, resolve_path
from netra_moe.layer import MoELayer
from netra_moe import weights as W

ROUTING = ("logits", "topk_ids", "topk_weights", "x_q", "x_scale", "sorted_ids",
           "sorted_expert", "tile_map", "pair_map", "num_valid", "expert_counts", "partial")
PATH_INTERMEDIATES = {"fused": ("h_q", "h_scale", "ffn_counters"), "stream": ("h_q", "h_scale"), "tile": ("h_q", "h_scale")}
FRONT_INTERMEDIATES = {"exact": ("mask",), "screen": ()}


def intermediates(path: str, front: str) -> tuple[str, ...]:
    front_extra = () if path == "fused" else FRONT_INTERMEDIATES[front]  # the gate/up prologue keeps its bitmask in LDS
    return ROUTING + PATH_INTERMEDIATES[path] + front_extra
WEIGHT_SEED = 77


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def make_inputs(cfg: MoEConfig, device: torch.device, weights_on_gpu: bool | None = None):
    """Activations from the CPU generator; expert weights quantised by the
    oracle (small shapes) or by the GPU weight-prep kernel (full shapes)."""
    act = W.synthetic_activations(cfg, "cpu")
    if weights_on_gpu is None:
        weights_on_gpu = cfg.Etot * cfg.I * cfg.H > (1 << 24)
    if weights_on_gpu:
        wq = W.synthetic_expert_weights(cfg, WEIGHT_SEED, device, keep_row_major=True)
        torch.cuda.synchronize(device)
        rm13 = wq.pop("w13_row_major").cpu().numpy()
        rm2 = wq.pop("w2_row_major").cpu().numpy()
        s13, s2 = wq["w13_scale"].cpu().numpy(), wq["w2_scale"].cpu().numpy()
    else:
        w13, w2 = W.synthetic_expert_weights_f32(cfg, WEIGHT_SEED, "cpu")
        rm13, s13 = oracle.quant_blocks_f32(w13.numpy())
        rm2, s2 = oracle.quant_blocks_f32(w2.numpy())
        wq = {"w13": torch.from_numpy(W.pack_tiles_host(rm13, gate_up=True)).to(device),
              "w13_scale": torch.from_numpy(s13).to(device),
              "w2": torch.from_numpy(W.pack_tiles_host(rm2)).to(device),
              "w2_scale": torch.from_numpy(s2).to(device)}
    gpu = {"router_w": act["router_w"].to(device), "router_bias": act["router_bias"].to(device), **wq}
    host = {
        "x": bf16_bits(act["x"]),
        "router_w": bf16_bits(act["router_w"]),
        "router_bias": act["router_bias"].numpy(),
        "w13": rm13, "w13_scale": s13, "w2": rm2, "w2_scale": s2,
    }
    return act["x"].to(device), gpu, host


def run_gpu(cfg: MoEConfig, x: torch.Tensor, gpu_weights: dict, device: torch.device,
            expose=None, graph: bool = False, repeats: int = 1, path: str = "auto", front: str = "auto"):
    path = resolve_path(cfg, path)
    front = resolve_front(cfg, path, front)
    layer = MoELayer(cfg, gpu_weights, device=device.index or 0,
                     expose=expose or intermediates(path, front), graph=graph, path=path, front=front)
    expose = layer.expose
    outs = []
    for _ in range(repeats):
        layer.forward(x)
        torch.cuda.synchronize(device)
        outs.append(bf16_bits(layer.out))
    res = {"out": outs[-1], "runs": outs, "path": path, "front": front}
    for name in expose:
        t = layer.buffer(name).detach().cpu()
        if t.dtype == torch.bfloat16:
            res[name] = bf16_bits(t)
        else:
            res[name] = t.numpy().copy()
    layer.close()
    return res


def oracle_routing(cfg: MoEConfig, host: dict) -> dict:
    logits = oracle.router_logits(host["x"], host["router_w"])
    ids, wts = oracle.topk(logits, host["router_bias"], cfg.E, cfg.K, cfg.S)
    x_q, x_s = oracle.quant_rows_bf16(host["x"])
    sid, sexp, nv, counts, tmap, pmap = oracle.sort(ids, cfg.Etot, cfg.cap_blocks, with_tiles=True)
    return dict(logits=logits, topk_ids=ids, topk_weights=wts, x_q=x_q, x_scale=x_s,
                sorted_ids=sid, sorted_expert=sexp, num_valid=nv, expert_counts=counts,
                tile_map=tmap, pair_map=pmap)


def sample_tokens(cfg: MoEConfig, n: int) -> np.ndarray:
    if cfg.T <= n:
        return np.arange(cfg.T, dtype=np.int64)
    rng = np.random.default_rng(cfg.seed + 5)
    picks = rng.choice(cfg.T, size=n, replace=False)
    return np.unique(np.concatenate([[0, cfg.T - 1], picks]))[:n].astype(np.int64)
