"""Shape profiles: exact/bounded guards with priority-ordered selection.

Mirrors compiler/netra_compiler/profiles.py:12-77 (DimensionGuard, ShapeProfile,
select_profile) and the netra-profile-1 JSON files in
manifests/gfx950/profiles/*.json. A failed selection reports that the framework
fallback is required instead of guessing a neighbouring shape. These types,
their one-line bodies and select_profile's two reason strings are kept alike on
purpose: they are the netra-profile-1 interface a caller of the reference
reads and writes.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Mapping

from .config import MoEConfig


@dataclass(frozen=True)
class DimensionGuard:
    minimum: int
    maximum: int

    def __post_init__(self) -> None:
        if self.minimum < 0 or self.maximum < self.minimum:
            raise ValueError("invalid bounded dimension guard")

    @classmethod
    def exact(cls, value: int) -> "DimensionGuard":
        return cls(value, value)

    def matches(self, value: int) -> bool:
        return self.minimum <= value <= self.maximum

    def to_dict(self) -> dict[str, int]:
        return {"min": self.minimum, "max": self.maximum}


@dataclass(frozen=True)
class ShapeProfile:
    name: str
    guards: tuple[tuple[str, DimensionGuard], ...]
    quantization: str = "fp8_block128"
    tensor_parallel: int = 1
    priority: int = 0

    def __post_init__(self) -> None:
        if self.tensor_parallel <= 0:
            raise ValueError("tensor parallel degree must be positive")
        if len({k for k, _ in self.guards}) != len(self.guards):
            raise ValueError("duplicate profile guard")

    def guard(self, name: str) -> DimensionGuard:
        for k, g in self.guards:
            if k == name:
                return g
        raise KeyError(name)

    def matches(self, dims: Mapping[str, int], *, quantization: str, tensor_parallel: int) -> bool:
        return (quantization == self.quantization and tensor_parallel == self.tensor_parallel
                and all(k in dims and g.matches(dims[k]) for k, g in self.guards))

    def to_dict(self) -> dict[str, object]:
        return {"format": "netra-profile-1", "name": self.name,
                "guards": {k: g.to_dict() for k, g in self.guards},
                "quantization": self.quantization, "tensor_parallel": self.tensor_parallel,
                "priority": self.priority}

    @classmethod
    def from_dict(cls, d: Mapping[str, object]) -> "ShapeProfile":
        if d.get("format", "netra-profile-1") != "netra-profile-1":
            raise ValueError("not a netra-profile-1 document")
        guards = d["guards"]
        assert isinstance(guards, Mapping)
        tp = d.get("tensor_parallel", 1)
        return cls(str(d["name"]),
                   tuple((k, DimensionGuard(int(v["min"]), int(v["max"]))) for k, v in guards.items()),
                   str(d.get("quantization", "fp8_block128")),
                   int(tp) if not isinstance(tp, str) else 1,
                   int(d.get("priority", 0)))


@dataclass(frozen=True)
class ProfileSelection:
    supported: bool
    profile: ShapeProfile | None
    reason: str


def select_profile(profiles: tuple[ShapeProfile, ...], dims: Mapping[str, int], *,
                   quantization: str = "fp8_block128", tensor_parallel: int = 1) -> ProfileSelection:
    for p in sorted(profiles, key=lambda p: (-p.priority, p.name)):
        if p.matches(dims, quantization=quantization, tensor_parallel=tensor_parallel):
            return ProfileSelection(True, p, "all exact/bounded guards matched")
    return ProfileSelection(False, None, "unsupported contract/profile; framework fallback required")


def profile_for(cfg: MoEConfig) -> ShapeProfile:
    """Exact-m profile of one fixed-shape MoE engine (m = tokens per call)."""
    return ShapeProfile(
        name=f"moe_m{cfg.T}",
        guards=(("m", DimensionGuard.exact(cfg.T)), ("batch", DimensionGuard(1, 1 << 16)),
                ("sequence", DimensionGuard(0, 1 << 20))),
        priority=10,
    )


def load_profiles(directory: Path) -> tuple[ShapeProfile, ...]:
    out = []
    for path in sorted(Path(directory).glob("*.json")):
        out.append(ShapeProfile.from_dict(json.loads(path.read_text())))
    return tuple(out)
