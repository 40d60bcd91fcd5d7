"""Kernel contracts and their stable identities.

Identity rule follows the reference compiler: an ``nk_`` id is the first 24 hex
digits of sha256 over the canonical JSON (sorted keys, compact separators,
trailing newline) of the contract's identity fields; names of models and
symbols are not part of the identity
(compiler/netra_compiler/types.py:49-57, contracts.py:94-172).

The build's kernels are HIP code objects, so contracts carry
``artifact_kind: "hip_code_object"`` and the code object's sha256 (the
reference pins assembled artefacts the same way for golden operations,
contracts.py:418-501). Each contract also states the typed fields of the
reference's typed kernel contract (shape, dtypes, quantization, layouts,
epilogue, tactic, numerical, workspace, maturity, fallback; contracts.py:
176-285), which is the variant of schemas/netra-kernel-contract.schema.json a
contract that is neither a raw-assembly template, a golden external hsaco nor
a framework fallback must satisfy. A request no tactic serves gets a
``FallbackContract`` (``nkf_`` id, no launch, workspace or symbol; the rule of
contracts.py:288-375).
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


def _pairs(d: Any) -> tuple[tuple[str, Any], ...]:
    """A mapping frozen as sorted (key, value) pairs (lists become tuples)."""
    items = d.items() if isinstance(d, dict) else d
    return tuple(sorted((str(k), tuple(v) if isinstance(v, list) else v) for k, v in items))


def _thaw(pairs: tuple[tuple[str, Any], ...]) -> dict[str, Any]:
    return {k: list(v) if isinstance(v, tuple) else v for k, v in pairs}


MATURITIES = ("experiment", "verified", "accepted", "rejected")
EPILOGUES = ("identity", "bias", "silu", "gelu", "gated_silu")
DTYPES = ("fp8_e4m3", "fp16", "bf16", "fp32", "int32")


@dataclass(frozen=True)
class HipKernelContract:
    """One fixed-shape launch of a HIP kernel from a gfx950 code object.

    ``shape`` is the operation's [m, n, k], ``dtypes`` its [input, weight,
    accumulator, output] dtypes, ``layouts`` its [activation, weight, output]
    layouts, each in the reference's vocabulary (types.py:11-32)."""

    operation: str
    family: str
    symbol: str
    constants: tuple[tuple[str, int], ...]
    semantics: tuple[tuple[str, str], ...]
    launch: Launch
    kernarg_size: int
    code_object_sha256: str
    shape: tuple[int, int, int] = (1, 1, 1)
    dtypes: tuple[str, str, str, str] = ("fp8_e4m3", "fp8_e4m3", "fp32", "bf16")
    quantization: tuple[tuple[str, Any], ...] = ()
    layouts: tuple[str, str, str] = ("row_major", "row_major", "row_major")
    epilogue: str = "identity"
    tactic: str = ""
    numerical: tuple[tuple[str, Any], ...] = ()
    workspace_bytes: int = 0
    workspace_alignment: int = 256
    target: str = "gfx950"
    wave_size: int = 64
    graph_capture: bool = True
    deterministic: bool = True
    fallback: str = "framework"
    maturity: str = "accepted"
    source_refs: tuple[str, ...] = field(default=(), compare=False)
    evidence_refs: tuple[str, ...] = field(default=(), compare=False)

    def __post_init__(self) -> None:
        if self.target != "gfx950" or self.wave_size != 64:
            raise ValueError("gfx950 contracts require wave64")
        if self.kernarg_size <= 0 or self.kernarg_size % 4:
            raise ValueError("kernarg size must be positive and dword aligned")
        names = [n for n, _ in self.constants]
        if len(names) != len(set(names)) or any(v < 0 for _, v in self.constants):
            raise ValueError("constants need unique names and nonnegative values")
        if len(self.shape) != 3 or min(self.shape) <= 0:
            raise ValueError("shape needs three positive dimensions [m, n, k]")
        if len(self.dtypes) != 4 or any(d not in DTYPES for d in self.dtypes):
            raise ValueError(f"dtypes need four of {DTYPES}")
        if len(self.layouts) != 3 or not all(self.layouts):
            raise ValueError("layouts need [activation, weight, output]")
        if self.epilogue not in EPILOGUES:
            raise ValueError(f"epilogue must be one of {EPILOGUES}")
        if not self.tactic or not self.fallback:
            raise ValueError("a kernel contract names its tactic and its fallback")
        if self.maturity not in MATURITIES:
            raise ValueError(f"maturity must be one of {MATURITIES}")
        if self.workspace_bytes < 0 or self.workspace_alignment <= 0 or \
                self.workspace_alignment & (self.workspace_alignment - 1):
            raise ValueError("workspace needs nonnegative bytes and a power-of-two alignment")

    def identity_dict(self) -> dict[str, Any]:
        return {
            "target": self.target,
            "wave_size": self.wave_size,
            "operation": self.operation,
            "family": self.family,
            "constants": dict(self.constants),
            "semantics": dict(self.semantics),
            "shape": list(self.shape),
            "dtypes": list(self.dtypes),
            "quantization": _thaw(self.quantization),
            "layouts": list(self.layouts),
            "epilogue": self.epilogue,
            "tactic": self.tactic,
            "numerical": _thaw(self.numerical),
            "kernarg_size": self.kernarg_size,
            "launch": self.launch.to_dict(),
            "workspace": {"bytes": self.workspace_bytes, "alignment": self.workspace_alignment},
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
                 fallback=self.fallback, maturity=self.maturity,
                 source_refs=list(self.source_refs), evidence_refs=list(self.evidence_refs))
        return d


@dataclass(frozen=True)
class FallbackContract:
    """The requested computation when no tactic serves it: a stable ``nkf_``
    identity and no launch, workspace, symbol or tactic (those belong to the
    framework implementation that runs instead)."""

    operation: str
    shape: tuple[int, int, int]
    dtypes: tuple[str, str, str, str]
    quantization: tuple[tuple[str, Any], ...]
    layouts: tuple[str, str, str]
    epilogue: str
    numerical: tuple[tuple[str, Any], ...]
    fallback: str = "framework"
    target: str = "gfx950"
    wave_size: int = 64
    graph_capture: bool = True
    deterministic: bool = True

    def identity_dict(self) -> dict[str, Any]:
        return {
            "target": self.target,
            "wave_size": self.wave_size,
            "operation": self.operation,
            "shape": list(self.shape),
            "dtypes": list(self.dtypes),
            "quantization": _thaw(self.quantization),
            "layouts": list(self.layouts),
            "epilogue": self.epilogue,
            "graph_capture": self.graph_capture,
            "deterministic": self.deterministic,
            "numerical": _thaw(self.numerical),
        }

    @property
    def stable_id(self) -> str:
        return "nkf_" + stable_hash(self.identity_dict())[:24]

    def to_dict(self) -> dict[str, Any]:
        d = self.identity_dict()
        d.update(id=self.stable_id, artifact_kind="framework_fallback", fallback=self.fallback)
        return d
