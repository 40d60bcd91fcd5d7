"""Shared set-up of the bridge tests: the reference's Qwen3.6-35B-A3B layer
shape (hidden 2048, 256 routed experts + the shared expert as expert 256,
top-8 + 1, intermediate 512) with seeded weights quantised on the GPU, kept in
the AITER 16x16 shuffle for the kernels and row-major on the host for the
oracle, plus seeded tokens, their oracle routing and the prefill sorted
format."""
from __future__ import annotations

import ctypes

import numpy as np
import torch

import oracle
from moe_case import bf16_bits
from netra_moe import weights as W

DEV = torch.device("cuda", 0)
H, E, K, I = 2048, 256, 8, 512
ETOT, KTOT = E + 1, K + 1
SEED = 2024
M768 = 768


def capacity(rows: int) -> int:
    return (rows * KTOT + 63) // 64 + ETOT


def half_rows(rows: int) -> int:
    return rows * KTOT + capacity(rows)


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else None)


def stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)


def aiter(q: torch.Tensor) -> torch.Tensor:
    """Row-major e4m3 bytes [G, N, K] -> the AITER 16x16 shuffle [N/16][K/32][2][16][16] per group."""
    g, n, k = q.shape
    return q.view(g, n // 16, 16, k // 32, 2, 16).permute(0, 1, 3, 4, 2, 5).contiguous().view(g, n, k)


class _Shape:
    Etot, I, H = ETOT, I, H


def build_model() -> dict:
    gen = torch.Generator().manual_seed(SEED)
    router = (torch.randn((E + 1, H), generator=gen) * 0.02).to(torch.bfloat16)
    w13f, w2f = W.synthetic_expert_weights_f32(_Shape(), SEED, DEV)
    q13, s13 = W.quantize_blocks(w13f)
    q2, s2 = W.quantize_blocks(w2f)
    del w13f, w2f
    torch.cuda.synchronize()
    return {
        "router_w": router[:E].contiguous().to(DEV), "shared_w": router[E:].contiguous().to(DEV),
        "w13": aiter(q13), "w13_scale": s13, "w2": aiter(q2), "w2_scale": s2,
        "host": {"router": bf16_bits(router), "w13": q13.cpu().numpy(), "w13_scale": s13.cpu().numpy(),
                 "w2": q2.cpu().numpy(), "w2_scale": s2.cpu().numpy()},
    }


def tokens(rows: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((rows, H), generator=g).to(torch.bfloat16)
    return x, bf16_bits(x)


def routing(model: dict, xb: np.ndarray):
    """Oracle routing of the tokens: logits, top-8 + shared ids / weights."""
    logits = oracle.router_logits(xb, model["host"]["router"])
    ids, wts = oracle.topk(logits, None, E, K, 1)
    return logits, ids, wts


def prefill_inputs(model: dict, xb: np.ndarray) -> dict:
    """Quantised tokens, routing and the AITER sorted format for len(xb) tokens."""
    rows = xb.shape[0]
    _, ids, wts = routing(model, xb)
    x_q, x_s = oracle.quant_rows_bf16(xb)
    sid, sexp, nv, _ = oracle.sort(ids, ETOT, capacity(rows))
    return dict(rows=rows, xb=xb, x_q=x_q, x_s=x_s, ids=ids, wts=wts, sid=sid, sexp=sexp, nv=nv)


def prefill_buffers(inp: dict) -> dict:
    """Device inputs and fresh outputs of one prefill launch (outputs poisoned)."""
    rows = inp["rows"]
    d = {k: torch.from_numpy(np.ascontiguousarray(inp[k])).to(DEV) for k in ("x_q", "x_s", "sid", "sexp", "wts")}
    d["nv"] = torch.from_numpy(np.ascontiguousarray(inp["nv"][:1])).to(DEV)
    d["sorted_w"] = torch.zeros(inp["sid"].size, dtype=torch.float32, device=DEV)  # unused by the producer
    d["rs"] = torch.full((capacity(rows) * 64, I // 128), -1.0, dtype=torch.float32, device=DEV)
    d["parts"] = torch.full((2, half_rows(rows), H), float("nan"), dtype=torch.float16, device=DEV)
    d["out"] = torch.full((rows, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    return d


def prefill_args(model: dict, d: dict) -> tuple:
    return (ptr(d["x_q"]), ptr(d["x_s"]), ptr(model["w13"]), ptr(model["w13_scale"]), ptr(model["w2"]),
            ptr(model["w2_scale"]), ptr(d["sid"]), ptr(d["sorted_w"]), ptr(d["sexp"]), ptr(d["nv"]),
            ptr(d["wts"]), ptr(d["rs"]), ptr(d["parts"]), ptr(d["out"]))
