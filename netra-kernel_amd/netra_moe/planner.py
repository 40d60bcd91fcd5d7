"""Tactic catalog, layer planning with fallback, and the workspace packer.

The reference compiler chooses a kernel per graph operation from a catalog of
fixed tactics: every tactic states the semantics it implements and the
compile-time constants it accepts, lists why it rejects a request, and the
planner takes the best-ranked tactic that rejects nothing or falls back to the
framework, recording every candidate's reasons in ``explain.json``
(compiler/netra_compiler/backends/gfx950/catalog.py:23-212, planner.py:139-266,
engine.py:435-440). Its workspace is interval-packed: temporaries whose
lifetimes do not overlap share bytes (memory.py:56-112).

Here the unit a tactic implements is the whole routed-MoE layer: the launches
of one GEMM path and one routing front end, built from this build's gfx950
code object (``artifact_kind: "hip_code_object"``). The reason strings are the
reference planner's vocabulary ("operation mismatch", "layouts semantic
mismatch", "<constant> mismatch", ...), so a caller that reads
``explain.json`` the reference's way finds the same words.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Mapping

from .config import MoEConfig

OPERATION = "moe.routed_layer"
FAMILY = "moe.fp8_block128.gfx950_hip"
TARGET = "gfx950"
MATURITIES = ("accepted", "experiment", "rejected")


@dataclass(frozen=True)
class HipCodeObjectTactic:
    """One way to run the layer: a GEMM path plus a routing front end.

    ``sets`` lists constants with their allowed values, ``ranges`` constants
    with an inclusive [lo, hi] bound, ``limits`` derived quantities with an
    upper bound (routes per token, experts incl. shared, capacity blocks)."""

    name: str
    path: str
    front: str
    semantics: tuple[tuple[str, str], ...]
    sets: tuple[tuple[str, tuple[int, ...]], ...]
    ranges: tuple[tuple[str, int, int], ...]
    limits: tuple[tuple[str, int], ...] = ()
    pairs: tuple[tuple[int, int], ...] = ()  # instantiated (H, I) pairs, when not every combination is
    rank: int = 100
    maturity: str = "accepted"
    graph_capture: bool = True
    deterministic: bool = True
    fallback: str = "framework"
    evidence_refs: tuple[str, ...] = field(default=(), compare=False)

    @property
    def artifact_kind(self) -> str:
        return "hip_code_object"

    def rejection_reasons(self, request: Mapping[str, Any], *, allow_experimental: bool = False) -> tuple[str, ...]:
        out: list[str] = []
        if request.get("family") not in (None, FAMILY):
            out.append("tactic-family mismatch")
        if request.get("operation") != OPERATION:
            out.append("operation mismatch")
        if request.get("target") != TARGET:
            out.append("target mismatch")
        if request.get("wave_size") != 64:
            out.append("wave-size mismatch")
        for key, mine in (("path", self.path), ("front", self.front)):
            want = request.get(key)
            if want not in (None, "auto") and want != mine:
                out.append(f"{'gemm-path' if key == 'path' else 'front-end'} mismatch")
        sem = request.get("semantics")
        if not isinstance(sem, Mapping):
            out.append("semantic contract missing")
        else:
            mine = dict(self.semantics)
            for key, value in mine.items():
                # numerical is optional in a request: absent means either front end will do
                if key == "numerical" and key not in sem:
                    continue
                if sem.get(key) != value:
                    out.append(f"{key} semantic mismatch")
            out.extend(f"undeclared semantic field {k}" for k in sorted(set(sem) - set(mine)))
        if self.maturity == "rejected":
            out.append("maturity is rejected")
        elif self.maturity == "experiment" and not allow_experimental:
            out.append("experimental tactics are disabled")
        if request.get("graph_capture", True) and not self.graph_capture:
            out.append("graph capture required")
        if request.get("deterministic", True) and not self.deterministic:
            out.append("determinism required")
        constants = request.get("constants")
        if not isinstance(constants, Mapping):
            out.append("compile-time constants missing")
            return tuple(out)
        declared = set()
        for key, allowed in self.sets:
            declared.add(key)
            if key not in constants:
                out.append(f"{key} missing")
            elif constants[key] not in allowed:
                out.append(f"{key} mismatch")
        for key, lo, hi in self.ranges:
            declared.add(key)
            v = constants.get(key)
            if v is None:
                out.append(f"{key} missing")
            elif not isinstance(v, int) or isinstance(v, bool) or not lo <= v <= hi:
                out.append(f"{key} mismatch")
        if self.pairs and (constants.get("H"), constants.get("I")) not in self.pairs:
            out.append("H/I pair mismatch")
        derived = request.get("derived", {})
        for key, hi in self.limits:
            if derived.get(key, 0) > hi:
                out.append(f"{key} exceeds {hi}")
        out.extend(f"undeclared compile-time constant {k}" for k in sorted(set(constants) - declared))
        return tuple(out)


# Layer-level semantics. The layouts a caller hands in: W13 gate/up-interleaved
# tile16x128 and W2 tile16x128 (netra_moe_pack_tiles*), e4m3 codes with fp32
# 128x128 block scales; routing and h stay inside the layer.
LAYER_ABI = "netra_moe_layer.engine_bindings.x_router_w_router_bias_w13_w13s_w2_w2s_out.v1"
LAYER_DTYPES = "x_bf16.router_bf16.bias_f32.weights_e4m3fn.scales_f32.out_bf16.v1"
LAYER_LAYOUTS = "w13_tile16x128_gate_up_interleaved.w2_tile16x128.x_row_major.out_row_major.v1"


def layer_semantics_request(numerical: str | None = None, **overrides: str) -> dict[str, str]:
    """The semantics this build's kernels implement; override a field to ask
    for something else (a row-major checkpoint layout, say)."""
    from .engine import QUANTIZATION
    sem = {"abi": LAYER_ABI, "dtypes": LAYER_DTYPES, "quantization": QUANTIZATION, "layouts": LAYER_LAYOUTS}
    if numerical is not None:
        sem["numerical"] = numerical
    sem.update(overrides)
    return sem


def catalog() -> tuple[HipCodeObjectTactic, ...]:
    """Every layer tactic in the gfx950 code object, best rank first."""
    from . import engine as E
    base = layer_semantics_request()
    sem = lambda front: tuple(sorted({**base, "numerical": E.NUMERICS[front]}.items()))  # noqa: E731
    limits = (("Ktot", 16), ("Etot", 512))
    fused_h = tuple(sorted({h for h, _ in E.FUSED_HI}))
    fused_i = tuple(sorted({i for _, i in E.FUSED_HI}))
    return (
        HipCodeObjectTactic(
            "gfx950.moe_fp8.fused_decode.exact", "fused", "exact", sem("exact"),
            sets=(("H", fused_h), ("I", fused_i)), ranges=(("T", 1, E.FUSED_MAX_T), ("E", 1, 4096), ("K", 1, 64), ("S", 0, 1)),
            limits=limits + (("cap_blocks", 1024),), pairs=tuple(E.FUSED_HI), rank=10,
            evidence_refs=("kernels/gfx950/templates/moe/decode/gate_up_mfma.inc:12-161",
                           "kernels/gfx950/templates/moe/decode/down_reduce_mfma_2wave.inc:14-291")),
        HipCodeObjectTactic(
            "gfx950.moe_fp8.stream.exact", "stream", "exact", sem("exact"),
            sets=(("H", E.STREAM_H), ("I", E.STREAM_I)), ranges=(("T", 1, 256), ("E", 1, 4096), ("K", 1, 64), ("S", 0, 1)),
            rank=20, evidence_refs=("kernels/gfx950/templates/moe/decode/gate_up_mfma.inc:12-161",)),
        # the same kernels past decode sizes: correct, but ranked behind the tile path
        HipCodeObjectTactic(
            "gfx950.moe_fp8.stream_wide_t.exact", "stream", "exact", sem("exact"),
            sets=(("H", E.STREAM_H), ("I", E.STREAM_I)), ranges=(("T", 257, 1 << 20), ("E", 1, 4096), ("K", 1, 64), ("S", 0, 1)),
            rank=50, evidence_refs=("kernels/gfx950/templates/moe/decode/gate_up_mfma.inc:12-161",)),
        HipCodeObjectTactic(
            "gfx950.moe_fp8.tile.screen", "tile", "screen", sem("screen"),
            sets=(("H", tuple(h for h in E.TILE_H if h in E.SCREEN_H)), ("I", E.TILE_I)),
            ranges=(("T", 1, 1 << 20), ("E", 1, E.SCREEN_EMAX[-1]), ("K", 1, 64), ("S", 0, 1)),
            limits=(("x_bytes", (1 << 31) - 1),),  # 32-bit buffer offsets into bf16 x
            rank=30, evidence_refs=("kernels/gfx950/templates/moe/prefill/fused_splitk2/entry_routing.inc:27-112",)),
        HipCodeObjectTactic(
            "gfx950.moe_fp8.tile.exact", "tile", "exact", sem("exact"),
            sets=(("H", E.TILE_H), ("I", E.TILE_I)), ranges=(("T", 1, 1 << 20), ("E", 1, 4096), ("K", 1, 64), ("S", 0, 1)),
            limits=(("x_bytes", (1 << 32) - 2),),  # 32-bit buffer offsets into FP8 x_q
            rank=40, evidence_refs=("kernels/gfx950/templates/moe/prefill/fused_splitk2/entry_routing.inc:27-112",)),
    )


def layer_request(cfg: MoEConfig, *, semantics: Mapping[str, str] | None = None, path: str = "auto",
                  front: str = "auto", graph_capture: bool = True, deterministic: bool = True) -> dict[str, Any]:
    return {
        "family": FAMILY, "operation": OPERATION, "target": TARGET, "wave_size": 64,
        "path": path, "front": front,
        "semantics": dict(semantics) if semantics is not None else layer_semantics_request(),
        "constants": {"T": cfg.T, "H": cfg.H, "I": cfg.I, "E": cfg.E, "K": cfg.K, "S": cfg.S},
        "derived": {"Ktot": cfg.Ktot, "Etot": cfg.Etot, "cap_blocks": cfg.cap_blocks, "x_bytes": 2 * cfg.T * cfg.H},
        "graph_capture": graph_capture, "deterministic": deterministic, "fallback": "framework",
    }


@dataclass(frozen=True)
class LayerPlan:
    selected: HipCodeObjectTactic | None
    execution: str                       # "kernel" or "fallback"
    fallback: str
    candidates: tuple[dict[str, Any], ...]

    def explain(self, name: str) -> dict[str, Any]:
        return {"name": name, "selected": self.selected.name if self.selected else None,
                "execution": self.execution, "fallback": self.fallback, "candidates": list(self.candidates)}


def plan_layer(request: Mapping[str, Any], *, allow_experimental: bool = False,
               tactics: tuple[HipCodeObjectTactic, ...] | None = None) -> LayerPlan:
    """Best-ranked tactic that rejects nothing, else the request's fallback.
    Candidates are listed compatible first (by rank), then rejected (by name)."""
    tactics = catalog() if tactics is None else tactics
    ok, bad = [], []
    for t in tactics:
        why = t.rejection_reasons(request, allow_experimental=allow_experimental)
        (bad if why else ok).append((t, why))
    ok.sort(key=lambda p: (p[0].rank, p[0].name))
    bad.sort(key=lambda p: p[0].name)
    if len(ok) > 1 and ok[0][0].rank == ok[1][0].rank:
        tied = ", ".join(t.name for t, _ in ok if t.rank == ok[0][0].rank)
        raise ValueError(f"ambiguous tactics at rank {ok[0][0].rank}: {tied}")
    cands = tuple([{"tactic": t.name, "selected": i == 0, "reasons": []} for i, (t, _) in enumerate(ok)]
                  + [{"tactic": t.name, "selected": False, "reasons": list(why)} for t, why in bad])
    fallback = str(request.get("fallback", "framework"))
    if not ok:
        return LayerPlan(None, "fallback", fallback, cands)
    return LayerPlan(ok[0][0], "kernel", fallback, cands)


# ---------------------------------------------------------------------------
# Workspace packing

@dataclass(frozen=True)
class BufferSlot:
    name: str
    offset: int
    size: int
    first_use: int
    last_use: int
    persistent: bool

    def to_dict(self) -> dict[str, Any]:
        return {"name": self.name, "offset": self.offset, "size": self.size, "alignment": 256,
                "first_use": self.first_use, "last_use": self.last_use, "persistent": self.persistent}


def _lifetimes(ops: list[dict], names: set[str]) -> dict[str, tuple[int, int, bool]]:
    """(first op, last op, read before written) of each named tensor in one layer call."""
    out: dict[str, tuple[int, int, bool]] = {}
    for i, op in enumerate(ops):
        used = {a for a in op["args"] if isinstance(a, str)}
        for n in used & names:
            if n in out:
                first, _, rbw = out[n]
                out[n] = (first, i, rbw)
            else:
                out[n] = (i, i, n in op["reads"] and n not in op["writes"])
    return out


def pack_workspace(sizes: Mapping[str, int], ops: list[dict], persistent: set[str],
                   align: int = 256) -> tuple[int, list[BufferSlot]]:
    """Offsets for the engine's temporaries. Persistent tensors (state carried
    from one launch to the next, like the hand-off counters that start at zero
    and are put back to zero) get bytes of their own; every other tensor lives
    from the first to the last operation that names it and shares bytes with
    tensors whose lifetimes do not overlap. Placement: largest first, each at
    the lowest aligned offset clear of every placed tensor it overlaps in time."""
    names = set(sizes)
    life = _lifetimes(ops, names)
    last_op = max(len(ops) - 1, 0)
    for n in names:
        if n not in life:  # named by no operation: keep it for the whole call
            life[n] = (0, last_op, False)
    for n, (_, _, rbw) in life.items():
        if rbw and n not in persistent:
            raise ValueError(f"{n} is read before any operation writes it; it must be persistent")
    rounded = {n: (s + align - 1) // align * align for n, s in sizes.items()}
    slots: list[BufferSlot] = []
    cursor = 0
    for n in sorted(persistent & names):
        slots.append(BufferSlot(n, cursor, rounded[n], 0, last_op, True))
        cursor += rounded[n]
    base = cursor
    placed: list[BufferSlot] = []
    for n in sorted(names - persistent, key=lambda k: (-rounded[k], life[k][0], k)):
        first, last, _ = life[n]
        busy = sorted((s.offset, s.offset + s.size) for s in placed
                      if not (last < s.first_use or first > s.last_use))
        off = base
        for lo, hi in busy:
            if off + rounded[n] <= lo:
                break
            off = max(off, hi)
        slot = BufferSlot(n, off, rounded[n], first, last, False)
        placed.append(slot)
    slots += placed
    top = max((s.offset + s.size for s in slots), default=0)
    return top, sorted(slots, key=lambda s: s.name)
