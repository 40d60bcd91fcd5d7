"""Kernel contracts and their stable identities.

Identity rule follows the reference compiler: an ``nk_`` id is the first 24 hex
digits of sha256 over the canonical JSON (sorted keys, compact separators,
trailing newline) of the contract's identity fields; names of models and
symbols are not part of the identity
(compiler/netra_compiler/types.py:49-57, contracts.py:94-172).

The build's kernels are HIP code objects, so contracts carry
``artifact_kind: "hip_code_object"`` and the code object's sha256 (the
reference pins assembled artefacts the same way for golden operations,
contracts.py:418-501).
"""
from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass, field
from typing import Any


def canonical_json(value: Any) -> str:
    return json.dumps(value, sort_keys=True, separators=(",", ":"), ensure_ascii=False) + "\n"


def stable_hash(value: Any) -> str:
    return hashlib.sha256(canonical_json(value).encode("utf-8")).hexdigest()


@dataclass(frozen=True)
class Launch:
    grid: tuple[int, int, int]
    block: tuple[int, int, int]
    lds_bytes: int = 0
    dynamic_lds_bytes: int = 0

    def __post_init__(self) -> None:
        if len(self.grid) != 3 or len(self.block) != 3 or min(self.grid) < 1 or min(self.block) < 1:
            raise ValueError("launch grid/block need three positive dimensions")
        if self.block[0] * self.block[1] * self.block[2] > 1024:
            raise ValueError("workgroup exceeds 1024 threads")
        if self.lds_bytes + self.dynamic_lds_bytes > 160 * 1024:
            raise ValueError("LDS request exceeds 160 KiB")

    def to_dict(self) -> dict[str, Any]:
        return {"grid": list(self.grid), "block": list(self.block),
                "lds_bytes": self.lds_bytes, "dynamic_lds_bytes": self.dynamic_lds_bytes}


@dataclass(frozen=True)
class HipKernelContract:
    """One fixed-shape launch of a HIP kernel from a gfx950 code object."""

    operation: str
    family: str
    symbol: str
    constants: tuple[tuple[str, int], ...]
    semantics: tuple[tuple[str, str], ...]
    launch: Launch
    kernarg_size: int
    code_object_sha256: str
    target: str = "gfx950"
    wave_size: int = 64
    graph_capture: bool = True
    deterministic: bool = True
    source_refs: tuple[str, ...] = field(default=(), compare=False)

    def __post_init__(self) -> None:
        if self.target != "gfx950" or self.wave_size != 64:
            raise ValueError("gfx950 contracts require wave64")
        if self.kernarg_size <= 0 or self.kernarg_size % 4:
            raise ValueError("kernarg size must be positive and dword aligned")
        names = [n for n, _ in self.constants]
        if len(names) != len(set(names)) or any(v < 0 for _, v in self.constants):
            raise ValueError("constants need unique names and nonnegative values")

    def identity_dict(self) -> dict[str, Any]:
        return {
            "target": self.target,
            "wave_size": self.wave_size,
            "operation": self.operation,
            "family": self.family,
            "constants": dict(self.constants),
            "semantics": dict(self.semantics),
            "kernarg_size": self.kernarg_size,
            "launch": self.launch.to_dict(),
            "code_object_sha256": self.code_object_sha256,
            "graph_capture": self.graph_capture,
            "deterministic": self.deterministic,
        }

    @property
    def stable_id(self) -> str:
        return "nk_" + stable_hash(self.identity_dict())[:24]

    def to_dict(self) -> dict[str, Any]:
        d = self.identity_dict()
        d.update(id=self.stable_id, symbol=self.symbol, artifact_kind="hip_code_object",
                 source_refs=list(self.source_refs))
        return d
