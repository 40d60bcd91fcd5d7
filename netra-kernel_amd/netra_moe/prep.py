"""Checkpoint weight preparation: per-expert FP8 tensors -> the layer's
stacked tile16x128 weights on the GPU.

A block-FP8 MoE checkpoint stores every expert separately: gate_proj and
up_proj weights [I, H], down_proj [H, I], as e4m3 codes with one scale per
128x128 block (``weight_scale_inv``, bf16 or fp32), and the shared expert under
its own name. A tensor may also arrive split into output shards (row blocks
of one logical tensor, as tensor-parallel checkpoints save them). The
reference plans these conversions as explicit steps
(compiler/netra_compiler/layouts.py:109-206): concatenate output shards along
axis 0, widen bf16 scales to fp32 exactly, then one layout transform. Here the
steps are:

  1. ``concatenate_output_shards`` (axis 0) for weights and scale grids;
  2. ``widen_bf16_to_fp32_exact`` for bf16 scales;
  3. ``stack_experts``: routed experts 0..E-1, the shared expert as expert E;
     W13 rows are gate then up ([E+S, 2I, H]), W2 is [E+S, H, I];
  4. ``tile16x128_gate_up_interleaved`` (W13) / ``tile16x128`` (W2) on the GPU
     by the library's packing kernels (netra_moe_pack_tiles_gate_up /
     netra_moe_pack_tiles).

Steps 1-3 are byte moves and exact widenings done with torch on the device;
step 4 is this build's HIP kernels. The result is what MoELayer binds as
w13 / w13_scale / w2 / w2_scale.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Mapping, Sequence, Union

import torch

from . import weights as W
from .config import MoEConfig

TensorOrShards = Union[torch.Tensor, Sequence[torch.Tensor]]
PROJECTIONS = ("gate_proj", "up_proj", "down_proj")


@dataclass(frozen=True)
class PrepStep:
    tensor: str
    transform: str
    parameters: tuple[tuple[str, int], ...] = ()

    def to_dict(self) -> dict:
        return {"tensor": self.tensor, "transform": self.transform, "parameters": dict(self.parameters)}


def checkpoint_name(prefix: str, expert: int | None, proj: str, scale: bool = False) -> str:
    """HF-style names: {prefix}.experts.{e}.{proj}.weight[_scale_inv], the
    shared expert (expert=None) as {prefix}.shared_expert.{proj}...."""
    owner = "shared_expert" if expert is None else f"experts.{expert}"
    return f"{prefix}.{owner}.{proj}.{'weight_scale_inv' if scale else 'weight'}"


def _pieces(tensors: Mapping[str, TensorOrShards], name: str) -> list[torch.Tensor]:
    if name not in tensors:
        raise KeyError(f"checkpoint tensor {name} is missing")
    v = tensors[name]
    return [v] if isinstance(v, torch.Tensor) else list(v)


def plan_checkpoint(cfg: MoEConfig, tensors: Mapping[str, TensorOrShards], prefix: str) -> list[PrepStep]:
    """The step list for this checkpoint (shard counts and scale dtype as found)."""
    steps: list[PrepStep] = []
    experts = list(range(cfg.E)) + ([None] * cfg.S)
    for kind, projs in (("w13", ("gate_proj", "up_proj")), ("w2", ("down_proj",))):
        shards = {len(_pieces(tensors, checkpoint_name(prefix, e, p))) for e in experts for p in projs}
        if max(shards) > 1:
            steps.append(PrepStep(kind, "concatenate_output_shards", (("axis", 0), ("shards", max(shards)))))
        sdt = {_pieces(tensors, checkpoint_name(prefix, e, p, True))[0].dtype for e in experts for p in projs}
        if torch.bfloat16 in sdt:
            steps.append(PrepStep(kind + "_scale", "widen_bf16_to_fp32_exact"))
        steps.append(PrepStep(kind, "stack_experts", (("routed", cfg.E), ("shared", cfg.S))))
        steps.append(PrepStep(kind, "tile16x128_gate_up_interleaved" if kind == "w13" else "tile16x128"))
    return steps


def _weight(tensors, name: str, rows: int, cols: int, device) -> torch.Tensor:
    parts = _pieces(tensors, name)
    for p in parts:
        if p.dim() != 2 or p.shape[1] != cols or p.dtype not in (torch.uint8, torch.float8_e4m3fn):
            raise ValueError(f"{name}: shards must be e4m3 (or uint8 codes) [rows, {cols}], got "
                             f"{tuple(p.shape)} {p.dtype}")
    if sum(p.shape[0] for p in parts) != rows:
        raise ValueError(f"{name}: shards hold {sum(p.shape[0] for p in parts)} rows, expected {rows}")
    return torch.cat([p.to(device).view(torch.uint8) for p in parts], dim=0)


def _scale(tensors, name: str, rows: int, cols: int, device) -> torch.Tensor:
    parts = _pieces(tensors, name)
    for p in parts:
        if p.dim() != 2 or p.shape[1] != cols or p.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError(f"{name}: scale shards must be bf16 or fp32 [rows, {cols}], got "
                             f"{tuple(p.shape)} {p.dtype}")
    if sum(p.shape[0] for p in parts) != rows:
        raise ValueError(f"{name}: scale shards hold {sum(p.shape[0] for p in parts)} block rows, expected {rows}")
    return torch.cat([p.to(device).to(torch.float32) for p in parts], dim=0)  # bf16 -> fp32 is exact


def stack_checkpoint(cfg: MoEConfig, tensors: Mapping[str, TensorOrShards], prefix: str,
                     device: torch.device) -> dict[str, torch.Tensor]:
    """Per-expert checkpoint tensors (host or device) -> the layer's weight
    bindings on ``device``: w13 [E+S, 2I, H] and w2 [E+S, H, I] e4m3 bytes in
    the kernels' tile layouts, fp32 block scales [E+S, 2I/128, H/128] and
    [E+S, H/128, I/128]. Every expected tensor is checked before any is moved."""
    if not torch.cuda.is_available():
        raise RuntimeError("stack_checkpoint packs on the GPU; there is no CPU path")
    H, I, kb, ki = cfg.H, cfg.I, cfg.H // 128, cfg.I // 128
    experts = list(range(cfg.E)) + ([None] * cfg.S)
    plan_checkpoint(cfg, tensors, prefix)  # raises on a missing tensor before anything moves
    w13 = torch.empty((cfg.Etot, 2 * I, H), dtype=torch.uint8, device=device)
    w2 = torch.empty((cfg.Etot, H, I), dtype=torch.uint8, device=device)
    s13 = torch.empty((cfg.Etot, 2 * ki, kb), dtype=torch.float32, device=device)
    s2 = torch.empty((cfg.Etot, kb, ki), dtype=torch.float32, device=device)
    for slot, e in enumerate(experts):
        w13[slot, :I] = _weight(tensors, checkpoint_name(prefix, e, "gate_proj"), I, H, device)
        w13[slot, I:] = _weight(tensors, checkpoint_name(prefix, e, "up_proj"), I, H, device)
        w2[slot] = _weight(tensors, checkpoint_name(prefix, e, "down_proj"), H, I, device)
        s13[slot, :ki] = _scale(tensors, checkpoint_name(prefix, e, "gate_proj", True), ki, kb, device)
        s13[slot, ki:] = _scale(tensors, checkpoint_name(prefix, e, "up_proj", True), ki, kb, device)
        s2[slot] = _scale(tensors, checkpoint_name(prefix, e, "down_proj", True), kb, ki, device)
    return {"w13": W.pack_tiles(w13, gate_up=True), "w13_scale": s13,
            "w2": W.pack_tiles(w2), "w2_scale": s2}
