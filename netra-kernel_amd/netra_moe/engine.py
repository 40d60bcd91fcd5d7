"""Emit a netra-engine-1 directory for one fixed-shape MoE layer.

The directory layout and engine.json fields are the ones the reference
runtime reads (runtime/gfx950/engine/netra_engine.hip:273-383; emitted by
compiler/netra_compiler/engine.py:373-504):

  engine.json        format_version, target, wave_size, required_rocm,
                     workspace_bytes, profiles[].guards, operations[] with
                     launch/hsaco/kernel_symbol/typed arguments
  contracts.json     one HIP kernel contract (stable nk_ id) per operation
  graph_recipe.json  tensors, binding slots (profile, op, arg) per tensor and the
                     RAW/WAR/WAW operation dependencies
  memory_plan.json   workspace offsets of the engine-owned tensors
  hsaco/             the code object

Caller-owned tensors (inputs, weights, output and any intermediate the caller
asks to see) are bound pointer slots; every other intermediate lives in the
engine workspace.
"""
from __future__ import annotations

import hashlib
import json
import shutil
from dataclasses import dataclass
from pathlib import Path

from .config import BLOCK_M, MoEConfig
from .contracts import FallbackContract, HipKernelContract, Launch, _pairs, canonical_json, stable_hash
from .profiles import profile_for
from . import paths

DTYPE_BYTES = {"bf16": 2, "f32": 4, "e4m3": 1, "i32": 4, "u32": 4, "u64": 8}
ALIGN = 256
OPERATION_NAME = "moe.routed_layer"


@dataclass(frozen=True)
class TensorSpec:
    name: str
    dtype: str
    shape: tuple[int, ...]
    role: str  # input | weight | output | temporary

    @property
    def nbytes(self) -> int:
        n = DTYPE_BYTES[self.dtype]
        for d in self.shape:
            n *= d
        return n


GEMM_PATHS = ("fused", "stream", "tile")
FUSED_HI = ((512, 256), (1024, 1024), (2048, 512), (4096, 256))  # netra_moe_ffn_{gate_up,down}_h<H>_i<I>_<v>_gfx950
FUSED_MAX_T = 64                     # one bitmask word per expert in the gate/up prologue
FFN_NARROW_T = 16                    # T at or below which the decode FFN splits K (the "narrow" variant)
NARROW_ROWS_DOWN_T = 5               # narrow T at or above which down takes the wide item shape + combine kernel
FFN_COUNTERS = 64 * 64               # combine hand-off counters [token][column group] (kCounters)
FFN_WIDE_P = {(512, 256): 2, (1024, 1024): 4, (2048, 512): 4, (4096, 256): 2}  # wide gate/up items per wave (PG)
STREAM_H = (512, 1024, 2048, 4096)   # netra_moe_gate_up_stream_h<H>_c<CH>_gfx950
STREAM_I = (256, 512, 1024, 2048)    # netra_moe_down_stream_i<I>_c<DC>_gfx950
TILE_H = (512, 1024, 2048, 4096)     # netra_moe_gate_up_tile_h<H>_gfx950
TILE_I = (256, 512, 1024)            # netra_moe_down_tile_i<I>_gfx950
ROWS_I = (256, 512)                  # netra_moe_down_rows_i<I>_gfx950 (block rows x runs of column groups)
DOWN_ROWS_ITEMS = 1024               # down_rows: fewer column groups per item until about this many items
TILE_GU_WAVES = 4                    # waves of netra_moe_gate_up_tile_h<H>_gfx950 (its launch bound)
LDS_GU_H = (512, 1024, 2048)         # netra_moe_gate_up_lds_h<H>_gfx950: 128-row pairs, LDS operand ring
# Stream kernel grids (measured at T=64 on one MI355X): gate/up fills the chip
# once, 256 CUs x 4 SIMDs x 2 resident waves (NK_GATE_UP_WAVES_PER_EU) / 8
# waves per workgroup; down runs 4096 four-wave workgroups, about four times
# what is resident at once, with 2 K blocks per step, so each wave streams few
# steps (46.2 us against 47.3 us for 2048 workgroups of 1-block steps, 49 us
# for 1024).
STREAM_GRID_GATE_UP = 256
STREAM_GU_THREADS = 512
STREAM_GRID_DOWN = 4096
# K blocks per prefetch step of the stream kernels (symbol suffix _c<n>): the
# bytes each wave keeps in flight, which bounds the weight stream.
STREAM_GU_CHUNK = 2
STREAM_DN_CHUNK = 2


def stream_chunks(cfg: MoEConfig) -> tuple[int, int]:
    """(gate/up, down) K blocks per step, limited so every item has an even step count."""
    kb_h, kb_i = cfg.H // 128, cfg.I // 128
    cu = STREAM_GU_CHUNK if kb_h % (2 * STREAM_GU_CHUNK) == 0 else 2
    cd = STREAM_DN_CHUNK if kb_i % (2 * STREAM_DN_CHUNK) == 0 else 1
    return cu, cd


def fused_supported(cfg: MoEConfig) -> bool:
    """The decode FFN kernels (netra_moe_ffn_gate_up / netra_moe_ffn_down) cover T <= 64 for the
    instantiated (H, I), up to 512 experts, 16 routes per token and 1024
    capacity blocks."""
    return (cfg.T <= FUSED_MAX_T and (cfg.H, cfg.I) in FUSED_HI and cfg.Etot <= 512 and cfg.Ktot <= 16
            and cfg.cap_blocks <= 1024)


def _planned(cfg: MoEConfig, path: str = "auto"):
    from .planner import layer_request, plan_layer
    plan = plan_layer(layer_request(cfg, path=path))
    if plan.selected is None:
        why = "; ".join(f"{c['tactic']}: {', '.join(c['reasons'])}" for c in plan.candidates)
        raise ValueError(f"no gfx950 kernel path serves this configuration ({why})")
    return plan.selected


def resolve_path(cfg: MoEConfig, path: str = "auto") -> str:
    """fused: route, gate/up with the sort, down (+ combine) for T <= 64;
    stream: split-K weight streaming (decode-sized T); tile: 64-row block
    tiles. auto takes the planner's best-ranked tactic (netra_moe.planner)."""
    if path == "auto":
        path = _planned(cfg).path
    if path not in GEMM_PATHS:
        raise ValueError(f"unknown GEMM path {path!r}")
    if path == "fused" and not fused_supported(cfg):
        raise ValueError("the fused decode FFN needs T <= 64, (H, I) in "
                         f"{FUSED_HI}, at most 512 experts and 16 routes per token")
    if path == "stream" and (cfg.H not in STREAM_H or cfg.I not in STREAM_I):
        raise ValueError(f"stream path kernels exist for H in {STREAM_H} and I in {STREAM_I}")
    if path == "tile" and (cfg.H not in TILE_H or cfg.I not in TILE_I):
        raise ValueError(f"tile path kernels exist for H in {TILE_H} and I in {TILE_I}")
    return path


def gate_up_lds_bytes(H: int) -> int:
    """Static LDS of netra_moe_gate_up_lds_h<H>: three stages of (9 row tiles +
    16 weight tiles) x 2 KiB, the activation scales of 144 rows in 1 KiB
    copies of 256 / (H / 128) rows each, the weight block scales, the row tokens."""
    kb = H // 128
    rows_per_copy = 256 // kb
    return 3 * 25 * 2048 + (144 + rows_per_copy - 1) // rows_per_copy * 1024 + 64 * 4 + 145 * 4


def xcd_grid(items: int) -> int:
    """Workgroups for an XCD-major item assignment (nktile::xcd_item): a
    multiple of 8 covering every item."""
    return (items + 7) // 8 * 8


FRONTS = ("exact", "screen")
SCREEN_H = (512, 1024, 2048)          # netra_moe_route_screen_h<H>_gfx950 / route_select_h<H>_e<EMAX>
SCREEN_EMAX = (256, 512)              # expert capacities of the route_select kernels
SCREEN_SELECT_SHAPES = ((4, 1), (8, 1), (8, 2), (8, 4))  # route_select_h<H>_e<EMAX>_w<W>x<WPT>: W waves, WPT per token


def resolve_front(cfg: MoEConfig, path: str = "auto", front: str = "auto") -> str:
    """exact: VALU router (every logit in the contract order) + top-k + one-
    workgroup sort; screen: bf16-MFMA screen with exact recomputation of the
    certified candidates + two-kernel sort (the tile path's default)."""
    path = resolve_path(cfg, path)
    ok = cfg.H in SCREEN_H and cfg.E <= SCREEN_EMAX[-1]
    if front == "auto":
        front = _planned(cfg, path).front
    if path == "fused" and front != "exact":
        raise ValueError("the fused decode path computes every logit (exact front end)")
    if front not in FRONTS:
        raise ValueError(f"unknown front end {front!r}")
    if front == "screen" and not ok:
        raise ValueError(f"screen front end needs H in {SCREEN_H} and E <= {SCREEN_EMAX[-1]}")
    return front


ROUTE_SLICES = 8                     # expert-total counters per expert (route_select's atomic adds, nkroute::kSlices)
SCREEN_WG_TARGET = 256               # route_screen: split K until the grid has this many workgroups
                                     # (measured: T=512 screen 14.3 -> 6.1 us at 4 splits; 8 splits cost the select more)


def screen_splits(cfg: MoEConfig) -> int:
    """K splits of the screen GEMM (netra_moe_route_screen_h<H>_k<H/128/Z>): the
    smallest power of two giving SCREEN_WG_TARGET workgroups (one per CU: a
    workgroup holds 128 KiB of LDS), at least two 128-K blocks per split."""
    tiles = (cfg.T + 127) // 128 * ((screen_row_pad(cfg) + 127) // 128)
    nj = cfg.H // 128
    z = 1
    while tiles * z < SCREEN_WG_TARGET and nj // (2 * z) >= 2:
        z *= 2
    return z


def screen_row_pad(cfg: MoEConfig) -> int:
    """Expert rows rounded up to the screen GEMM's 64-row tiles (row stride of
    the screen buffer). The shared-gate row E is not screened: route_select
    computes its logit exactly for every token."""
    return (cfg.E + 63) // 64 * 64


def screen_emax(cfg: MoEConfig) -> int:
    return next(e for e in SCREEN_EMAX if cfg.E <= e)


SCREEN_WAVE_TARGET = 2048            # route_select: waves per token until T * WPT reaches this many


def screen_waves_per_token(cfg: MoEConfig) -> int:
    """Waves per token of route_select (WPT of netra_moe_route_select_h<H>_e<EMAX>_w<W>x<WPT>):
    1, 2 or 4 (at most H / 512, the row's 512-element chunks), the most that
    keeps T * WPT within SCREEN_WAVE_TARGET, so small T still spreads a few
    thousand waves over the chip (each token's exact dot products, row staging
    and quant split over its waves)."""
    wpt = 1
    while wpt < 4 and 2 * wpt <= cfg.H // 512 and cfg.T * 2 * wpt <= SCREEN_WAVE_TARGET:
        wpt *= 2
    return wpt


def screen_waves(cfg: MoEConfig) -> int:
    """Waves per route_select workgroup: 8 when tokens share waves, else 4 for
    T <= 1024 (small workgroups spread T tokens over the chip's 256 CUs), else 8."""
    if screen_waves_per_token(cfg) > 1:
        return 8
    return 4 if cfg.T <= 1024 else 8


def screen_tokens(cfg: MoEConfig) -> int:
    """Tokens per route_select workgroup."""
    return screen_waves(cfg) // screen_waves_per_token(cfg)


def screen_groups(cfg: MoEConfig) -> int:
    return (cfg.T + screen_tokens(cfg) - 1) // screen_tokens(cfg)


def tensor_table(cfg: MoEConfig, path: str = "auto", front: str = "auto") -> dict[str, TensorSpec]:
    path = resolve_path(cfg, path)
    front = resolve_front(cfg, path, front)
    T, H, I = cfg.T, cfg.H, cfg.I
    specs = [
        TensorSpec("x", "bf16", (T, H), "input"),
        TensorSpec("router_w", "bf16", (cfg.router_rows, H), "weight"),
        TensorSpec("router_bias", "f32", (cfg.E,), "weight"),
        TensorSpec("w13", "e4m3", (cfg.Etot, 2 * I, H), "weight"),
        TensorSpec("w13_scale", "f32", (cfg.Etot, 2 * I // 128, H // 128), "weight"),
        TensorSpec("w2", "e4m3", (cfg.Etot, H, I), "weight"),
        TensorSpec("w2_scale", "f32", (cfg.Etot, H // 128, I // 128), "weight"),
        TensorSpec("out", "bf16", (T, H), "output"),
        TensorSpec("logits", "bf16", (T, cfg.router_rows), "temporary"),
        TensorSpec("topk_ids", "i32", (T, cfg.Ktot), "temporary"),
        TensorSpec("topk_weights", "f32", (T, cfg.Ktot), "temporary"),
        TensorSpec("x_q", "e4m3", (T, H), "temporary"),
        TensorSpec("x_scale", "f32", (T, H // 128), "temporary"),
        TensorSpec("sorted_ids", "i32", (cfg.cap_rows,), "temporary"),
        TensorSpec("sorted_expert", "i32", (cfg.cap_blocks,), "temporary"),
        TensorSpec("tile_map", "i32", (cfg.cap_tiles,), "temporary"),
        TensorSpec("pair_map", "i32", (cfg.cap_blocks,), "temporary"),
        TensorSpec("num_valid", "i32", (4,), "temporary"),
        TensorSpec("expert_counts", "i32", (cfg.Etot,), "temporary"),
    ]
    if path == "fused":
        # hand-off counters (route: one per token group, padded to a line; decode
        # FFN combine: one per (token, column range)); zero at engine creation
        # and put back to zero by every launch
        specs += [TensorSpec("route_counters", "u32", (route_groups(cfg), COUNTER_STRIDE), "temporary"),
                  TensorSpec("ffn_counters", "u32", (FFN_COUNTERS,), "temporary"),
                  # bf16 h rows of every tile (the narrow gate/up hands them to down)
                  TensorSpec("h_rows", "bf16", (cfg.cap_tiles * 16, I), "temporary")]
    elif front == "exact":
        specs += [TensorSpec("mask", "u64", (cfg.Etot, cfg.mask_words_per_expert), "temporary"),
                  # top-k hand-off counters of the route kernel, one per token group;
                  # zero at engine creation and put back to zero by every launch
                  TensorSpec("route_counters", "u32", (route_groups(cfg), COUNTER_STRIDE), "temporary")]
    else:
        specs += [TensorSpec("screen", "f32", (screen_splits(cfg), T, screen_row_pad(cfg)), "temporary"),
                  TensorSpec("route_wsq", "f32", (screen_splits(cfg), screen_row_pad(cfg)), "temporary"),
                  # per route_select workgroup: its routes' sorted-id entries grouped
                  # by expert, and the groups' offsets (last entry the route count)
                  TensorSpec("route_hist", "i32", (screen_groups(cfg), cfg.Etot + 1), "temporary"),
                  TensorSpec("route_bucket", "i32", (screen_groups(cfg), screen_tokens(cfg) * cfg.Ktot), "temporary"),
                  # expert totals in ROUTE_SLICES atomic counters each (cleared by route_screen)
                  TensorSpec("route_slices", "i32", (cfg.Etot, ROUTE_SLICES), "temporary")]
    if path in ("stream", "fused"):
        specs += [TensorSpec("h_q", "e4m3", (cfg.cap_rows, I), "temporary"),
                  TensorSpec("h_scale", "f32", (cfg.cap_rows // 16, I // 128, 16), "temporary")]
    else:
        specs += [TensorSpec("h_q", "e4m3", (cfg.cap_rows, I), "temporary"),
                  TensorSpec("h_scale", "f32", (cfg.cap_rows, I // 128), "temporary")]
    specs.append(TensorSpec("partial", "bf16" if path == "tile" else "f32", (cfg.routes, H), "temporary"))
    return {s.name: s for s in specs}


EXACT_FRONT_OPS = ("route", "sort")
SCREEN_FRONT_OPS = ("route_screen", "route_select", "sort_route")
PATH_OPS = {"stream": ("gate_up", "down", "combine"), "tile": ("gate_up", "down", "combine")}


def op_names(cfg: MoEConfig, path: str = "auto", front: str = "auto") -> tuple[str, ...]:
    """Engine operation names of one layer call, in launch order."""
    path = resolve_path(cfg, path)
    if path == "fused":
        dv = down_variant(cfg)
        return (("route", "gate_up") + (() if dv == "merged" else ("down",))
                + (("combine",) if dv in ("wide", "rows", "merged") else ()))
    front_ops = EXACT_FRONT_OPS if resolve_front(cfg, path, front) == "exact" else SCREEN_FRONT_OPS
    return front_ops + PATH_OPS[path]
ROUTER_H = (512, 1024, 2048, 4096)   # netra_moe_router_h<H>_t<NT>_gfx950


ROUTER_SMALL_T = 128                 # up to this T the router runs one token per workgroup


def router_tokens(H: int, T: int) -> int:
    """Tokens per router workgroup (template NT of netra_moe_router_h<H>_t<NT>):
    for small T the fewest the staging allows (NT * H a multiple of 2048:
    shorter fmaf chains per wave, more workgroups; measured 7.9 -> 6.0 us at
    T = 64, H = 2048), else four, so large T does not re-read the router rows
    from L2 for every token; two at H = 4096."""
    if H >= 4096:
        return 2
    return max(1, 2048 // H) if T <= ROUTER_SMALL_T else 4


COUNTER_STRIDE = 64  # u32 words per hand-off counter (one 256-byte line each; kCounterStride)


def route_groups(cfg: MoEConfig) -> int:
    """Token groups of the route kernel (its grid's y extent, one hand-off counter each)."""
    nt = router_tokens(cfg.H, cfg.T)
    return (cfg.T + nt - 1) // nt


def _screen_front(cfg: MoEConfig) -> list[dict]:
    T, H = cfg.T, cfg.H
    u = lambda v: ("u32", int(v))  # noqa: E731
    G = screen_groups(cfg)
    Wt = screen_tokens(cfg)
    Wv, WPT = screen_waves(cfg), screen_waves_per_token(cfg)
    RP = screen_row_pad(cfg)
    Z = screen_splits(cfg)
    return [
        dict(name="moe.route_screen", symbol=f"netra_moe_route_screen_h{H}_k{H // 128 // Z}_gfx950",
             grid=((T + 127) // 128, (RP + 127) // 128, Z), block=(256, 1, 1), lds=4 * 2 * 128 * 128, dyn=0,
             args=["x", "router_w", "screen", "route_wsq", "route_slices", u(cfg.Etot * ROUTE_SLICES),
                   u(T), u(H), u(cfg.E), u(RP)],
             reads=["x", "router_w"], writes=["screen", "route_wsq", "route_slices"],
             refs=["kernels/gfx950/templates/routing/bf16_gemv.inc:16-150"]),
        dict(name="moe.route_select",
             symbol=f"netra_moe_route_select_h{H}_e{screen_emax(cfg)}_w{Wv}x{WPT}_gfx950",
             grid=(G, 1, 1), block=(64 * Wv, 1, 1),
             lds=Wt * (H * 4 + 2 * (2 * screen_emax(cfg) + 1) + 64 * 4 + 4 * WPT
                       + (8 * screen_emax(cfg) if WPT > 1 else 0)) + 8 * screen_emax(cfg) + 4, dyn=0,
             args=["x", "router_w", "router_bias", "screen", "route_wsq", "logits", "topk_ids", "topk_weights", "x_q",
                   "x_scale", "route_hist", "route_bucket", "route_slices",
                   u(T), u(H), u(cfg.E), u(cfg.K), u(cfg.S), u(RP), u(Z), u(G)],
             reads=["x", "router_w", "router_bias", "screen", "route_wsq", "route_slices"],
             writes=["logits", "topk_ids", "topk_weights", "x_q", "x_scale", "route_hist", "route_bucket",
                     "route_slices"],
             refs=["kernels/gfx950/templates/routing/bf16_gemv.inc:16-150",
                   "runtime/gfx950/routing/decode/qwen36_shared_gate_append_bridge.hip:76-112"]),
        dict(name="moe.sort_route", symbol="netra_moe_sort_route_gfx950",
             grid=(cfg.Etot, 1, 1), block=(256, 1, 1), lds=4 * 20, dyn=4 * (4 * cfg.Etot + 3),
             args=["route_hist", "route_bucket", "route_slices", "expert_counts", "sorted_ids", "sorted_expert",
                   "tile_map", "pair_map", "num_valid",
                   u(T), u(cfg.Ktot), u(cfg.Etot), u(cfg.S), u(G), u(Wt), u(cfg.cap_blocks)],
             reads=["route_hist", "route_bucket", "route_slices"],
             writes=["expert_counts", "sorted_ids", "sorted_expert", "tile_map", "pair_map", "num_valid"],
             refs=["kernels/gfx950/templates/moe/prefill/fused_splitk2/entry_routing.inc:27-112",
                   "manifests/gfx950/models/qwen36-35b-c64-fp8.json:43-49"]),
    ]

def down_rows_groups(cfg: MoEConfig) -> int:
    """128-column groups per netra_moe_down_rows item: all H / 128 when the
    expected block count fills the chip, else fewer (a power of two) so that
    about DOWN_ROWS_ITEMS items exist."""
    nb = cfg.H // 128
    blocks = (cfg.routes + 63) // 64 + min(cfg.Etot, cfg.routes) // 2  # expected non-empty blocks
    nbc = nb
    while nbc > 1 and nbc % 2 == 0 and blocks * (nb // nbc) < DOWN_ROWS_ITEMS:
        nbc //= 2
    return nbc


def _route_op(cfg: MoEConfig) -> dict:
    """Router logits + input quant + top-k (hand-off to the last row-group workgroup of each token group)."""
    T, H = cfg.T, cfg.H
    u = lambda v: ("u32", int(v))  # noqa: E731
    NT = router_tokens(H, T)
    return dict(name="moe.route", symbol=f"netra_moe_route_h{H}_t{NT}_gfx950",
                grid=((cfg.router_rows + 15) // 16, route_groups(cfg), 1),
                block=(256, 1, 1), lds=4 * NT * H + 4, dyn=0,
                args=["x", "router_w", "router_bias", "logits", "x_q", "x_scale", "topk_ids", "topk_weights",
                      "route_counters", u(T), u(H), u(cfg.router_rows), u(cfg.E), u(cfg.K), u(cfg.S)],
                reads=["x", "router_w", "router_bias", "route_counters"],
                writes=["logits", "x_q", "x_scale", "topk_ids", "topk_weights", "route_counters"],
                refs=["kernels/gfx950/templates/routing/bf16_gemv.inc:16-150",
                      "tools/benchmark/export_qwen36_router_bf16_capture.py:78",
                      "runtime/gfx950/routing/decode/qwen36_shared_gate_append_bridge.hip:76-112",
                      "tools/benchmark/export_qwen36_shared_gate_append_capture.py:97-107,134-139"])


def _router_logits_op(cfg: MoEConfig) -> dict:
    """Router logits + input quant only (the narrow decode FFN runs the top-k)."""
    T, H = cfg.T, cfg.H
    u = lambda v: ("u32", int(v))  # noqa: E731
    NT = router_tokens(H, T)
    return dict(name="moe.route", symbol=f"netra_moe_router_logits_h{H}_t{NT}_gfx950",
                grid=((cfg.router_rows + 15) // 16, (T + NT - 1) // NT, 1),
                block=(256, 1, 1), lds=4 * NT * H, dyn=0,
                args=["x", "router_w", "logits", "x_q", "x_scale", u(T), u(H), u(cfg.router_rows)],
                reads=["x", "router_w"], writes=["logits", "x_q", "x_scale"],
                refs=["kernels/gfx950/templates/routing/bf16_gemv.inc:16-150",
                      "tools/benchmark/export_qwen36_router_bf16_capture.py:78"])


def ffn_variant(cfg: MoEConfig) -> str:
    """narrow (K split over waves) for a handful of tokens, else wide."""
    return "narrow" if cfg.T <= FFN_NARROW_T else "wide"


# (H, I) with a single-token down kernel (netra_moe_ffn_down_h<H>_i<I>_single)
SINGLE_DOWN = {(2048, 512)}
# (H, I) with a gate/up + down per tile kernel (netra_moe_ffn_gate_up_down_h<H>_i<I>;
# one wide gate/up item per tile) -> the expected tile count (expected_tiles)
# from which it replaces the wide down. The merged kernel streams each tile's
# W13 and W2 from one workgroup, so it wants enough tiles to keep the chip
# streaming; the separate down spreads each tile over many workgroups. Layer
# times measured on one MI355X against gate/up + down (µs, merged / separate):
# H 2048, I 512, E 256, K 8: T=21 (126.6 tiles) 85.2 / 84.6, 22 (130.7) 86.2 /
# 87.0, 23 86.8 / 88.3, 32 95.3 / 97.6, 64 130.6 / 131.1; E 64: T=64 K=4 (67.0)
# 82.4 / 72.1, T=48 K=6 (66.4) 80.9 / 71.7. H 512, I 256, from 19 tiles on:
# E 16 K 2 T=40 (18.9) 23.5 / 25.2, E 64 K 4 T=32 (57.9) 24.1 / 25.7, E 128
# K 8 T=24 25.6 / 28.0, E 256 T=17 25.7 / 28.7, T=64 32.0 / 35.0. (H 4096, I
# 256: 138.0 / 138.6 at T=64, 97.6 / 96.8 at T=24, 85.2 / 70.2 with E 32 at
# T=48: left out.)
MERGED_MIN_TILES = {(512, 256): 0, (2048, 512): 128}
# (H, I) -> the expected tile count from which the merged kernel splits
# gate/up's K over its waves (netra_moe_ffn_gate_up_down_h<H>_i<I>_ksplit: the
# workgroup reads one 16-column item's 64 KiB of W13 per step, split sums
# added in LDS), layer µs against the unsplit merged kernel at E 256, K 8:
# T=24 (137 tiles) 88.9 / 88.4, 32 (166) 94.5 / 95.1, 64 (226) 128.5 / 129.5
MERGED_KSPLIT_MIN_TILES = {(2048, 512): 150}


def expected_tiles(cfg: MoEConfig) -> float:
    """16-row tiles of a decode call under uniform routing: the routed experts
    a call is expected to touch, plus the shared experts' tiles."""
    touched = cfg.E * (1.0 - (1.0 - cfg.K / cfg.E) ** cfg.T) if cfg.E else 0.0
    return touched + cfg.S * ((cfg.T + 15) // 16)


def down_variant(cfg: MoEConfig) -> str:
    """single (one workgroup per 16 output columns across all routes, the
    combine in the workgroup) for one token; rows (the narrow gate/up's bf16
    rows, the wide down's items, the combine kernel after it) from
    NARROW_ROWS_DOWN_T narrow tokens (measured at H 2048, I 512 with HBM-cold
    weights: 38.4 / 41.4 / 44.8 / 49.0 against 39.7 / 43.8 / 49.1 / 53.1 µs
    at T = 5 .. 8, 35.2 against 34.0 at T = 4); merged (the down of each tile
    run by its wide gate/up workgroup, the combine kernel after it) from
    MERGED_MIN_TILES expected tiles; else the FFN variant."""
    if cfg.T == 1 and (cfg.H, cfg.I) in SINGLE_DOWN and cfg.Ktot <= 16:
        return "single"
    v = ffn_variant(cfg)
    if v == "wide" and expected_tiles(cfg) >= MERGED_MIN_TILES.get((cfg.H, cfg.I), float("inf")):
        return "merged"
    return "rows" if v == "narrow" and cfg.T >= NARROW_ROWS_DOWN_T else v


def ffn_lds_bytes(cfg: MoEConfig) -> tuple[int, int]:
    """Static LDS of netra_moe_ffn_{gate_up,down}_h<H>_i<I>_<v> (their
    __shared__ arrays, rounded up)."""
    kb, kbi = cfg.H // 128, cfg.I // 128
    narrow = ffn_variant(cfg) == "narrow"
    red = 8 * 8 * 64 * 4 if narrow else 0
    gu = max(kb * 2048, red, 1024 * 4 + 513 * 4) + 64 * kb + (8 if narrow else 16 * (128 * FFN_WIDE_P[(cfg.H, cfg.I)] + 8)) * 2
    gu += 64 * 16 * 4 + 512 * 8 + 2 * 513 * 4 + 48 * 4
    if down_variant(cfg) == "merged" and expected_tiles(cfg) >= MERGED_KSPLIT_MIN_TILES.get((cfg.H, cfg.I), float("inf")):
        gu += 2 * 8 * 8 * 64 * 4  # the K split's sums, two steps
    dn = max(kbi * 2048, 0 if down_variant(cfg) == "rows" else red) + 64 * kbi + 4
    if down_variant(cfg) == "single":
        dn = 8 * 2 * cfg.I + 16 * 16 * 4
    return (gu + 255) // 256 * 256, (dn + 255) // 256 * 256


# Workgroups of the decode FFN kernels per (operation, variant), measured at
# T = 64 / T = 1 on one MI355X: wide gate/up streams a whole tile per
# workgroup and fills the chip once at 2 waves per SIMD (its register budget);
# narrow gate/up runs two 8-wave workgroups per CU; down deals its items over
# more workgroups than are resident (two per CU at a time). H = 4096 gate/up
# runs one per CU: the LDS of two does not fit.
FFN_GRID = {("gate_up", "wide"): 256, ("gate_up", "narrow"): 512, ("down", "wide"): 2048, ("down", "narrow"): 1024}


def ffn_grid(cfg: MoEConfig, op: str) -> int:
    g = FFN_GRID[(op, ffn_variant(cfg))]
    return 256 if op == "gate_up" and cfg.H > 2048 else g


def _fused_decode(cfg: MoEConfig) -> list[dict]:
    """Route (router + top-k; narrow: router logits only), gate/up with the sort
    (narrow: top-k and sort) as its prologue, down with the combine folded in
    (one token, and narrow below NARROW_ROWS_DOWN_T tokens) or followed by the
    combine kernel (wide, and narrow's rows down)."""
    T, H, I = cfg.T, cfg.H, cfg.I
    u = lambda v: ("u32", int(v))  # noqa: E731
    v = ffn_variant(cfg)
    lds_gu, lds_dn = ffn_lds_bytes(cfg)
    sort_out = ["sorted_ids", "sorted_expert", "tile_map", "pair_map", "num_valid", "expert_counts"]
    # narrow: the router writes the logits only and the gate/up prologue runs
    # the top-k (one wave per token), which takes the route kernel's hand-off
    # off the chain; wide: the route kernel's top-k feeds gate/up
    narrow = v == "narrow"
    route = _router_logits_op(cfg) if narrow else _route_op(cfg)
    topk = ["topk_ids", "topk_weights"]
    ops = [
        route,
        dict(name="moe.gate_up", symbol=f"netra_moe_ffn_gate_up_h{H}_i{I}_{v}_gfx950",
             grid=(ffn_grid(cfg, "gate_up"), 1, 1), block=(512, 1, 1), lds=lds_gu, dyn=0,
             args=["logits", "router_bias", *topk, "x_q", "x_scale", "w13", "w13_scale", *sort_out,
                   "h_rows", "h_q", "h_scale", u(T), u(cfg.E), u(cfg.K), u(cfg.S), u(cfg.cap_blocks)],
             reads=(["logits", "router_bias"] if narrow else ["topk_ids"]) + ["x_q", "x_scale", "w13", "w13_scale"],
             writes=(topk if narrow else []) + [*sort_out, "h_rows", "h_q", "h_scale"],
             refs=["kernels/gfx950/templates/moe/decode/gate_up_mfma.inc:12-161",
                   "kernels/gfx950/templates/moe/decode/silu_quant.inc:16-236",
                   "kernels/gfx950/templates/moe/prefill/fused_splitk2/entry_routing.inc:27-112"]
             + (["runtime/gfx950/routing/decode/qwen36_shared_gate_append_bridge.hip:76-112"] if narrow else [])),
        dict(name="moe.down", symbol=f"netra_moe_ffn_down_h{H}_i{I}_{down_variant(cfg)}_gfx950",
             grid=(H // 16 if down_variant(cfg) == "single" else
                   FFN_GRID[("down", "wide")] if down_variant(cfg) == "rows" else ffn_grid(cfg, "down"), 1, 1),
             block=(512, 1, 1),
             lds=lds_dn, dyn=0,
             args=["topk_weights", "w2", "w2_scale", "sorted_ids", "sorted_expert", "tile_map", "num_valid",
                   "h_rows", "h_q", "h_scale", "partial", "ffn_counters", "out",
                   u(T), u(cfg.E), u(cfg.K), u(cfg.S)],
             reads=["topk_weights", "w2", "w2_scale", "sorted_ids", "sorted_expert", "tile_map", "num_valid",
                    "h_rows", "h_q", "h_scale", "ffn_counters"],
             writes=["h_q", "h_scale", "partial", "ffn_counters", "out"],
             refs=["kernels/gfx950/templates/moe/decode/down_reduce_mfma_2wave.inc:14-291"]),
    ]
    if down_variant(cfg) in ("single", "rows"):  # no hand-off: the combine counters stay untouched
        ops[-1]["reads"].remove("ffn_counters")
        ops[-1]["writes"].remove("ffn_counters")
    if down_variant(cfg) == "rows":  # h requantised from the rows (copies for inspection), partials out
        ops[-1]["writes"] = ["h_q", "h_scale", "partial"]
    if down_variant(cfg) == "merged":  # gate/up runs each tile's down: its partials out, no down launch
        gu = ops[1]
        ks = "_ksplit" if expected_tiles(cfg) >= MERGED_KSPLIT_MIN_TILES.get((H, I), float("inf")) else ""
        gu["symbol"] = f"netra_moe_ffn_gate_up_down_h{H}_i{I}{ks}_gfx950"
        i = gu["args"].index("h_scale") + 1
        gu["args"][i:i] = ["w2", "w2_scale", "partial"]
        gu["reads"] += ["w2", "w2_scale"]
        gu["writes"] = [*sort_out, "h_q", "h_scale", "partial"]
        gu["refs"] += ops[2]["refs"]
        del ops[2]
    if down_variant(cfg) in ("wide", "rows", "merged"):  # fp32 partials for the combine kernel
        if v == "wide" and down_variant(cfg) == "wide":
            ops[-1]["writes"] = ["partial"]
        ops.append(dict(name="moe.combine", symbol="netra_moe_combine_gfx950",
                        grid=((H + 1023) // 1024, T, 1), block=(256, 1, 1), lds=0, dyn=0,
                        args=["partial", "topk_weights", "out", u(T), u(H), u(cfg.Ktot)],
                        reads=["partial", "topk_weights"], writes=["out"],
                        refs=["kernels/gfx950/templates/moe/prefill/route_reduce_splitk2_f16.inc:6-117"]))
    return ops


def _tile_down(cfg: MoEConfig) -> dict:
    T, H, I = cfg.T, cfg.H, cfg.I
    u = lambda v: ("u32", int(v))  # noqa: E731
    common = ["sorted_ids", "sorted_expert", "num_valid"]
    refs = ["kernels/gfx950/templates/moe/prefill/fused_splitk2/down_partial.inc",
            "kernels/gfx950/templates/moe/prefill/route_reduce_splitk2_f16.inc:6-117"]
    if I in ROWS_I and cfg.routes * H * 2 < 1 << 31:
        nbc = down_rows_groups(cfg)
        return dict(name="moe.down", symbol=f"netra_moe_down_rows_i{I}_gfx950",
                    grid=(xcd_grid(cfg.cap_blocks * (H // 128 // nbc)), 1, 1), block=(512, 1, 1),
                    lds=64 * I + 2 * 64 * 272 + 64 * (I // 128) * 4 + 64 * 4, dyn=0,
                    args=["h_q", "h_scale", "w2", "w2_scale", *common, "partial",
                          u(T), u(H), u(I), u(cfg.Ktot), u(cfg.Etot), u(nbc)],
                    reads=["h_q", "h_scale", "w2", "w2_scale", *common], writes=["partial"], refs=refs)
    return dict(name="moe.down", symbol=f"netra_moe_down_tile_i{I}_gfx950",
                grid=(xcd_grid(cfg.cap_blocks * (H // 128)), 1, 1), block=(256, 1, 1),
                lds=max(64 * (I + 16), 64 * 272) + 64 * (I // 128) * 4 + 64 * 4, dyn=0,
                args=["h_q", "h_scale", "w2", "w2_scale", *common, "partial",
                      u(T), u(H), u(I), u(cfg.Ktot), u(cfg.Etot)],
                reads=["h_q", "h_scale", "w2", "w2_scale", *common], writes=["partial"], refs=refs)


def operations(cfg: MoEConfig, path: str = "auto", front: str = "auto") -> list[dict]:
    """The six launches of one layer call, in stream order."""
    path = resolve_path(cfg, path)
    front = resolve_front(cfg, path, front)
    T, H, I = cfg.T, cfg.H, cfg.I
    W = cfg.mask_words_per_expert
    if H not in ROUTER_H:
        raise ValueError(f"router kernels exist for H in {ROUTER_H}")
    u = lambda v: ("u32", int(v))  # noqa: E731
    ops = [
        _route_op(cfg),
        dict(name="moe.sort", symbol="netra_moe_sort_gfx950",
             grid=(1, 1, 1), block=(1024, 1, 1), lds=0, dyn=cfg.sort_lds_bytes,
             args=["topk_ids", "mask", "sorted_ids", "sorted_expert", "tile_map", "pair_map", "num_valid",
                   "expert_counts",
                   u(T), u(cfg.Ktot), u(cfg.Etot), u(W), u(cfg.cap_blocks)],
             reads=["topk_ids"],
             writes=["mask", "sorted_ids", "sorted_expert", "tile_map", "pair_map", "num_valid", "expert_counts"],
             refs=["kernels/gfx950/templates/moe/prefill/fused_splitk2/entry_routing.inc:27-112"]),
    ]
    if front == "screen":
        ops = _screen_front(cfg)
    if path == "fused":
        return _fused_decode(cfg)
    common = ["sorted_ids", "sorted_expert", "num_valid"]
    if path == "stream":
        ops += [
            dict(name="moe.gate_up", symbol=f"netra_moe_gate_up_stream_h{H}_c{stream_chunks(cfg)[0]}_gfx950",
                 grid=(STREAM_GRID_GATE_UP, 1, 1), block=(STREAM_GU_THREADS, 1, 1), lds=0, dyn=0,
                 args=["x_q", "x_scale", "w13", "w13_scale", "sorted_ids", "sorted_expert",
                       "tile_map", "num_valid", "h_q", "h_scale",
                       u(T), u(H), u(I), u(cfg.Ktot), u(cfg.Etot)],
                 reads=["x_q", "x_scale", "w13", "w13_scale", *common, "tile_map"], writes=["h_q", "h_scale"],
                 refs=["kernels/gfx950/templates/moe/decode/gate_up_mfma.inc:12-161",
                       "kernels/gfx950/templates/moe/decode/silu_quant.inc:16-236"]),
            dict(name="moe.down", symbol=f"netra_moe_down_stream_i{I}_c{stream_chunks(cfg)[1]}_gfx950",
                 grid=(STREAM_GRID_DOWN, 1, 1), block=(256, 1, 1), lds=0, dyn=0,
                 args=["h_q", "h_scale", "w2", "w2_scale", "sorted_ids", "sorted_expert", "tile_map",
                       "num_valid", "partial",
                       u(T), u(H), u(I), u(cfg.Ktot), u(cfg.Etot)],
                 reads=["h_q", "h_scale", "w2", "w2_scale", *common, "tile_map"], writes=["partial"],
                 refs=["kernels/gfx950/templates/moe/decode/down_reduce_mfma_2wave.inc:14-291"]),
        ]
    else:
        if H in LDS_GU_H:
            if T * H >= 1 << 31:
                raise ValueError("netra_moe_gate_up_lds needs T * H < 2^31 (32-bit activation offsets)")
            gate_up = dict(
                name="moe.gate_up", symbol=f"netra_moe_gate_up_lds_h{H}_gfx950",
                grid=(xcd_grid(cfg.cap_blocks * (I // 128)), 1, 1), block=(512, 1, 1),
                lds=gate_up_lds_bytes(H), dyn=0,
                args=["x_q", "x_scale", "w13", "w13_scale", *common, "pair_map", "h_q", "h_scale",
                      u(T), u(H), u(I), u(cfg.Ktot), u(cfg.Etot)],
                reads=["x_q", "x_scale", "w13", "w13_scale", *common, "pair_map"], writes=["h_q", "h_scale"],
                refs=["kernels/gfx950/templates/moe/prefill/fused_splitk2/gate_up.inc",
                      "kernels/gfx950/templates/moe/prefill/fused_splitk2/silu_quant.inc"])
        else:
            gate_up = dict(
                name="moe.gate_up", symbol=f"netra_moe_gate_up_tile_h{H}_gfx950",
                grid=(xcd_grid(cfg.cap_blocks * (I // 128)), 1, 1), block=(64 * TILE_GU_WAVES, 1, 1),
                lds=2 * 64 * 144 + 2 * 64 * (H // 128) * 4 + 64 * 4 + TILE_GU_WAVES * 64 * 4 + 64 * 4, dyn=0,
                args=["x_q", "x_scale", "w13", "w13_scale", *common, "h_q", "h_scale",
                      u(T), u(H), u(I), u(cfg.Ktot), u(cfg.Etot)],
                reads=["x_q", "x_scale", "w13", "w13_scale", *common], writes=["h_q", "h_scale"],
                refs=["kernels/gfx950/templates/moe/prefill/fused_splitk2/gate_up.inc",
                      "kernels/gfx950/templates/moe/prefill/fused_splitk2/silu_quant.inc"])
        ops += [
            gate_up,
            _tile_down(cfg),
        ]
    combine_sym, combine_cols = ("netra_moe_combine_gfx950", 1024) if path == "stream" else \
        ("netra_moe_combine_bf16_gfx950", 2048)
    ops.append(
        dict(name="moe.combine", symbol=combine_sym,
             grid=((H + combine_cols - 1) // combine_cols, T, 1), block=(256, 1, 1), lds=0, dyn=0,
             args=["partial", "topk_weights", "out", u(T), u(H), u(cfg.Ktot)],
             reads=["partial", "topk_weights"], writes=["out"],
             refs=["kernels/gfx950/templates/moe/prefill/route_reduce_splitk2_f16.inc:6-117"]))
    return ops


# Contract semantics. The layouts semantic names what the kernels read: W13 in
# the gate/up-interleaved tile16x128 layout (netra_moe_pack_tiles_gate_up), W2
# in tile16x128, sorted ids in 64-row expert blocks with (slot << 24) | token,
# and h between the GEMMs in the path's own layout. A planner that matches on
# semantics (as the reference's does, compiler/netra_compiler/backends/gfx950/
# catalog.py:89-212) must not hand these kernels row-major or AITER-shuffled
# weights. The numerical semantic differs by front end: the screen front end
# leaves non-selected logits as bf16 MFMA screen values, not contract values.
WEIGHT_LAYOUTS = "w13_tile16x128_gate_up_interleaved.w2_tile16x128"
H_LAYOUTS = {"fused": "h_tile16x128_rowscale16", "stream": "h_tile16x128_rowscale16", "tile": "h_row_major_rowscale"}
NUMERICS = {
    "exact": "router_16slice_fma_tree.topk_lowidx.exp_cw7.v1",
    "screen": "router_bf16_mfma_screen_certified_exact_candidates.topk_lowidx.exp_cw7.v1",
}
QUANTIZATION = "fp8e4m3fn_block128x128_weights_1x128_activations.v1"


def layouts_semantic(path: str) -> str:
    return f"{WEIGHT_LAYOUTS}.sorted_m64_slot24.{H_LAYOUTS[path]}.v1"


def layer_semantics(symbol: str, path: str, front: str) -> tuple[tuple[str, str], ...]:
    return (("abi", f"{symbol}.ptr_then_u32.v1"), ("quantization", QUANTIZATION),
            ("layouts", layouts_semantic(path)), ("numerical", NUMERICS[front]))


def _dependencies(ops: list[dict]) -> list[list[int]]:
    deps = []
    for i, op in enumerate(ops):
        mine = set()
        for j in range(i):
            prev = ops[j]
            raw = set(op["reads"]) & set(prev["writes"])
            war = set(op["writes"]) & set(prev["reads"])
            waw = set(op["writes"]) & set(prev["writes"])
            if raw or war or waw:
                mine.add(j)
        deps.append(sorted(mine))
    return deps


# Tensors whose contents carry from one launch to the next: the hand-off
# counters start at zero (the workspace is zeroed at engine creation) and every
# launch puts them back to zero. They get bytes of their own in the workspace.
PERSISTENT_TENSORS = frozenset({"route_counters", "ffn_counters"})

COMPILER_NAME = "netra-moe-compiler"
COMPILER_VERSION = "0.3.0"
# The eight artefact files of a netra-engine-1 directory, in the reference
# compiler's order (compiler/netra_compiler/engine.py:478-479).
ARTIFACT_FILES = ("contracts.json", "graph.json", "graph_recipe.json", "memory_plan.json",
                  "layout_plan.json", "symbols.json", "validation_plan.json", "explain.json")
# Configuration fields an engine is guarded on, named as the reference's
# deployment guards name them (compiler/netra_compiler/engine.py:445-468).
ACTIVATION_QUANT, WEIGHT_QUANT = "e4m3_per_128", "e4m3_128x128"
IR_DTYPES = {"bf16": "bf16", "f32": "fp32", "e4m3": "fp8_e4m3", "i32": "int32", "u32": "uint32", "u64": "uint64"}


def _quantization() -> dict:
    return {"activation": ACTIVATION_QUANT, "weight": WEIGHT_QUANT,
            "activation_scale_block": 128, "weight_scale_block": [128, 128]}


def op_typing(cfg: MoEConfig, op: dict, path: str) -> dict:
    """The typed-contract fields of one operation: shape [m, n, k], dtypes
    [input, weight, accumulator, output], layouts [activation, weight,
    output], epilogue and numerical rules, in the reference's vocabulary
    (compiler/netra_compiler/contracts.py:176-285, types.py:11-32)."""
    kind = op["name"].split(".", 1)[1]
    T, H, I = cfg.T, cfg.H, cfg.I
    h_layout = H_LAYOUTS[path]
    partial_dtype = "bf16" if path == "tile" else "fp32"
    num = {"accumulation_dtype": "fp32", "nan_behavior": "ieee_preserve", "deterministic": True}
    router = {"output_rounding": "rne_bf16_logits",
              "reduction_order": "sixteen_slice_fmaf_chains_then_tree_8_4_2_1"}
    topk = {"selection": "topk_lowest_index_on_ties.softmax_of_selected_exp_cw7"}
    if kind in ("route", "route_select"):
        typ = dict(shape=[T, cfg.router_rows, H], dtypes=["bf16", "bf16", "fp32", "fp32"],
                   layouts=["row_major", "row_major", "topk_slots_row_major"], epilogue="identity",
                   numerical={**num, **router, **topk})
        if op["symbol"].startswith("netra_moe_router_logits"):
            typ.update(dtypes=["bf16", "bf16", "fp32", "bf16"], layouts=["row_major", "row_major", "row_major"],
                       numerical={**num, **router})
    elif kind == "route_screen":
        typ = dict(shape=[T, cfg.E, H], dtypes=["bf16", "bf16", "fp32", "fp32"],
                   layouts=["row_major", "row_major", "screen_partials_ksplit"], epilogue="identity",
                   numerical={**num, "output_rounding": "fp32_partial_per_k_split",
                              "reduction_order": "bf16_mfma_k_split_partials"})
    elif kind in ("sort", "sort_route"):
        typ = dict(shape=[cfg.routes, cfg.Etot, 1], dtypes=["int32", "int32", "int32", "int32"],
                   layouts=["topk_slots_row_major", "none", "sorted_m64_slot24"], epilogue="identity",
                   numerical={**num, "accumulation_dtype": "int32", "output_rounding": "exact_integer",
                              "reduction_order": "expert_then_token_ascending"})
    elif kind == "gate_up":
        typ = dict(shape=[cfg.routes, 2 * I, H], dtypes=["fp8_e4m3", "fp8_e4m3", "fp32", "fp8_e4m3"],
                   layouts=["row_major_scale_1x128", "tile16x128_gate_up_interleaved", h_layout],
                   epilogue="gated_silu",
                   numerical={**num, "output_rounding": "silu_mul_rne_bf16_then_e4m3_per_128",
                              "reduction_order": "k_block_ascending_fixed"})
    elif kind == "down":
        combined = path == "fused" and down_variant(cfg) in ("narrow", "single")
        typ = dict(shape=[cfg.routes, H, I],
                   dtypes=["fp8_e4m3", "fp8_e4m3", "fp32", "bf16" if combined else partial_dtype],
                   layouts=[h_layout, "tile16x128", "row_major" if combined else "route_partials_row_major"],
                   epilogue="identity",
                   numerical={**num, "reduction_order": "k_block_ascending_fixed",
                              "output_rounding": "topk_slots_ascending_fmaf_then_rne_bf16" if combined
                              else f"route_partial_{partial_dtype}"})
    elif kind == "combine":
        typ = dict(shape=[T, H, cfg.Ktot], dtypes=[partial_dtype, "fp32", "fp32", "bf16"],
                   layouts=["route_partials_row_major", "topk_slots_row_major", "row_major"], epilogue="identity",
                   numerical={**num, "output_rounding": "rne_bf16",
                              "reduction_order": "topk_slots_ascending_fmaf"})
    else:
        raise ValueError(f"no typed contract for operation {op['name']}")
    typ["quantization"] = _quantization()
    return typ


def _kernarg_layout(args: list) -> tuple[list[int], int]:
    """Byte offset of every kernel argument (pointers 8 bytes, u32 constants
    4, each at its natural alignment) and the 8-byte-aligned kernarg size."""
    offs, pos = [], 0
    for a in args:
        size = 4 if isinstance(a, tuple) else 8
        pos = (pos + size - 1) // size * size
        offs.append(pos)
        pos += size
    return offs, (pos + 7) // 8 * 8


def model_configuration(cfg: MoEConfig) -> dict:
    """The layer's configuration as an engine is guarded on it."""
    return {"architecture": "routed_moe_fp8_block128", "hidden_size": cfg.H,
            "moe_intermediate_size": cfg.I, "num_experts": cfg.E, "num_experts_per_tok": cfg.K,
            "shared_experts": cfg.S, "quantization_method": "fp8", "quantization_format": "e4m3fn",
            "activation_quantization": ACTIVATION_QUANT, "weight_scale_block": [128, 128],
            "kernel_scale_dtype": "fp32", "tensor_parallel": 1, "tokens": cfg.T}


DEPLOYMENT_GUARD_FIELDS = ("architecture", "hidden_size", "quantization_method", "quantization_format",
                           "activation_quantization", "weight_scale_block", "kernel_scale_dtype",
                           "tensor_parallel")


def _compiler_record(code_sha: str) -> dict:
    """Compiler identity: the package's Python sources, the tactic catalog and
    the code object (what the engine's contents follow from)."""
    from .planner import catalog
    pkg = Path(__file__).resolve().parent
    sources = {f.name: hashlib.sha256(f.read_bytes()).hexdigest() for f in sorted(pkg.glob("*.py"))}
    tactics = [{"name": t.name, "path": t.path, "front": t.front, "rank": t.rank, "maturity": t.maturity}
               for t in catalog()]
    return {"name": COMPILER_NAME, "version": COMPILER_VERSION,
            "source_hash": stable_hash({"version": COMPILER_VERSION, "python_sources": sources,
                                        "tactics": tactics, "code_object_sha256": code_sha})}


def _layout_plan() -> dict:
    """How checkpoint weights become the bound tensors (netra_moe.prep: the
    steps of compiler/netra_compiler/layouts.py:109-206 for this layout)."""
    def step(src, dst, transform, params=(), scope="synthetic_checkpoint_bit_exact"):
        return {"source_layout": src, "target_layout": dst, "transform": transform,
                "parameters": dict(params), "validated_scope": scope}

    def scale(name, tensors):
        return {"tensor": name, "checkpoint_tensors": tensors, "checkpoint_dtype": "bf16",
                "kernel_dtype": "fp32", "block": [128, 128], "checkpoint_layout": "row_major_block_grid",
                "kernel_layout": "row_major_block_grid",
                "steps": ["concatenate_output_scale_shards_axis0", "widen_bf16_to_fp32_exact", "stack_experts"]}
    rm = "checkpoint_row_major_fp8_block128"
    w13_src = ["mlp.experts.*.gate_proj.weight", "mlp.experts.*.up_proj.weight",
               "mlp.shared_expert.gate_proj.weight", "mlp.shared_expert.up_proj.weight"]
    w2_src = ["mlp.experts.*.down_proj.weight", "mlp.shared_expert.down_proj.weight"]
    return {"format": "netra-layout-plan-1", "bindings": [
        {"tensor": "w13", "checkpoint_layout": rm, "kernel_layout": "tile16x128_gate_up_interleaved",
         "output_layout": None, "checkpoint_tensors": w13_src,
         "steps": [step(rm, rm, "concatenate_output_shards", (("axis", 0),)),
                   step(rm, "stacked_row_major_fp8_block128", "stack_experts",
                        (("rows_gate_then_up", 1), ("shared_expert_last", 1))),
                   step("stacked_row_major_fp8_block128", "tile16x128_gate_up_interleaved",
                        "tile16x128_gate_up_interleaved", (("tile_m", 16), ("tile_k", 128)))],
         "scale": scale("w13_scale", [n + "_scale_inv" for n in w13_src])},
        {"tensor": "w2", "checkpoint_layout": rm, "kernel_layout": "tile16x128",
         "output_layout": None, "checkpoint_tensors": w2_src,
         "steps": [step(rm, rm, "concatenate_output_shards", (("axis", 0),)),
                   step(rm, "stacked_row_major_fp8_block128", "stack_experts", (("shared_expert_last", 1),)),
                   step("stacked_row_major_fp8_block128", "tile16x128", "tile16x128",
                        (("tile_m", 16), ("tile_k", 128)))],
         "scale": scale("w2_scale", [n + "_scale_inv" for n in w2_src])},
    ]}


def _graph(cfg: MoEConfig, tensors: dict, ops: list[dict]) -> dict:
    """The layer as a netra-ir-1 graph (compiler/netra_compiler/ir.py:126-249):
    typed tensors with roles, operations with their inputs and outputs."""
    role = lambda n, s: "state" if n in PERSISTENT_TENSORS else s.role  # noqa: E731
    return {
        "format": "netra-ir-1", "name": f"netra-moe-{cfg.name}",
        "tensors": [{"name": n, "shape": list(s.shape), "dtype": IR_DTYPES[s.dtype],
                     "layout": "engine_internal" if s.role == "temporary" else "row_major",
                     "role": role(n, s), "alias_of": None, "persistent": n in PERSISTENT_TENSORS}
                    for n, s in tensors.items()],
        "operations": [{"name": op["name"], "kind": "moe_fp8_block128", "inputs": list(op["reads"]),
                        "outputs": list(op["writes"]), "attributes": {"kernel_symbol": op["symbol"]},
                        "numerical": {}} for op in ops],
        "inputs": [n for n, s in tensors.items() if s.role in ("input", "weight")],
        "outputs": [n for n, s in tensors.items() if s.role == "output"],
        "state": sorted(n for n in tensors if n in PERSISTENT_TENSORS),
    }


def _symbol_listing(hsaco: Path, code: bytes, symbols: list[str]) -> str:
    """Text listing of the kernel symbols an engine names in its code object,
    the source its validation plan points at for each symbol."""
    sha = hashlib.sha256(code).hexdigest()
    return "".join([f"# kernel symbols of {hsaco.name} (sha256 {sha}) used by this engine\n"]
                   + [s + "\n" for s in symbols])


def _write(directory: Path, docs: dict) -> None:
    for fname, doc in docs.items():
        (directory / fname).write_text(canonical_json(doc))


def _finish_engine(engine: dict) -> dict:
    engine["engine_id"] = "ne_" + stable_hash(engine)[:24]
    return engine


def compile_moe_engine(cfg: MoEConfig, directory: Path, *, expose: tuple[str, ...] = (),
                       hsaco: Path | None = None, path: str = "auto", front: str = "auto",
                       semantics: dict | None = None, allow_experimental: bool = False) -> dict:
    """Plan the layer (netra_moe.planner), then write the netra-engine-1
    directory the reference compiler writes (compiler/netra_compiler/engine.py:
    373-504): engine.json, contracts.json (netra-contract-set-1), graph.json,
    graph_recipe.json, memory_plan.json, layout_plan.json, symbols.json,
    validation_plan.json and explain.json (every tactic considered, with its
    rejection reasons), plus hsaco/. When no tactic serves the request the
    engine holds one framework-fallback operation and no kernels. Returns the
    graph recipe (also on disk)."""
    from .planner import catalog, layer_request, pack_workspace, plan_layer
    directory = Path(directory)
    hsaco = Path(hsaco) if hsaco else paths.hsaco_path()
    if not hsaco.is_file():
        raise FileNotFoundError(f"code object {hsaco} is missing; run the build first")
    plan = plan_layer(layer_request(cfg, semantics=semantics, path=path, front=front),
                      allow_experimental=allow_experimental)
    profile = profile_for(cfg)
    code = hsaco.read_bytes()
    sha = hashlib.sha256(code).hexdigest()
    explain = {"format": "netra-explain-1", "profile": profile.to_dict(),
               "operations": [plan.explain("moe.layer")]}
    model_cfg = model_configuration(cfg)
    engine = {
        "format_version": "netra-engine-1",
        "target": "gfx950",
        "wave_size": 64,
        "required_rocm": {"minimum": "7.0", "code_object_version": 6},
        "name": f"netra-moe-{cfg.name}",
        "configuration": cfg.to_dict(),
        "model_configuration_hash": stable_hash(model_cfg),
        "checkpoint_hash": None,
        "deployment_guards": {k: model_cfg[k] for k in DEPLOYMENT_GUARD_FIELDS},
        "tensor_parallel": 1,
        "profiles": [profile.to_dict()],
        "layout_plan": "layout_plan.json", "graph_recipe": "graph_recipe.json", "memory_plan": "memory_plan.json",
        "validation_status": "static_only_not_promoted",
        "compiler": _compiler_record(sha),
        "golden_artifacts": [],
        "artifact_files": list(ARTIFACT_FILES),
    }
    validation = {"format": "netra-validation-plan-1", "static": "pending", "cross_assembly": "not_applicable",
                  "hardware": "not_run", "real_checkpoint_correctness": "not_run", "graph_replay": "not_run",
                  "matched_server_ab": "not_run", "promotion_eligible": False, "candidates": [],
                  "golden_artifacts": [],
                  "commands": ["netra_engine_manifest_check ENGINE_DIR",
                               "python -m pytest tests -m gpu (gfx950 device; parity against the CPU oracle)"]}
    directory.mkdir(parents=True, exist_ok=True)
    if plan.selected is None:
        # the requested computation, with no tactic to run it (contracts.py:288-375)
        fb = FallbackContract(
            operation=OPERATION_NAME, shape=(cfg.routes, 2 * cfg.I, cfg.H),
            dtypes=("bf16", "fp8_e4m3", "fp32", "bf16"), quantization=_pairs(_quantization()),
            layouts=("row_major", str((semantics or {}).get("layouts", "unspecified")), "row_major"),
            epilogue="gated_silu", numerical=_pairs({"accumulation_dtype": "fp32", "deterministic": True}),
            fallback=plan.fallback)
        engine.update(gemm_path=None, front_end=None, workspace_bytes=0, selected_tactics=[], kernel_symbols=[],
                      operations=[{"index": 0, "name": "moe.layer", "kind": OPERATION_NAME,
                                   "contract_id": fb.stable_id, "tactic": None, "maturity": None,
                                   "execution": "fallback", "kernel_symbol": None, "launch": None,
                                   "workspace_offset": None, "fallback": plan.fallback,
                                   "bindings": {"inputs": ["x", "router_w", "router_bias", "w13", "w13_scale",
                                                           "w2", "w2_scale"], "outputs": ["out"]},
                                   "artifact_kind": None}],
                      fallbacks={"moe.layer": plan.fallback})
        recipe = {"format": "netra-graph-recipe-1", "profile": profile.name, "capture_at_initialization": False,
                  "portable_serialized_hip_graph": False, "execution": "fallback", "gemm_path": None,
                  "front_end": None, "operations": [], "tensors": {}, "bindings": {}, "dependencies": []}
        graph = {"format": "netra-ir-1", "name": f"netra-moe-{cfg.name}", "tensors": [], "operations": [],
                 "inputs": [], "outputs": [], "state": []}
        _write(directory, {
            "contracts.json": {"format": "netra-contract-set-1", "contracts": [fb.to_dict()]},
            "graph.json": graph, "graph_recipe.json": recipe,
            "memory_plan.json": {"format": "netra-memory-plan-1", "workspace_bytes": 0, "alignment": ALIGN,
                                 "buffers": [], "offsets": {}},
            "layout_plan.json": _layout_plan(), "symbols.json": {"selected": [], "candidates": []},
            "validation_plan.json": validation, "explain.json": explain,
            "engine.json": _finish_engine(engine)})
        return recipe

    path, front = plan.selected.path, plan.selected.front
    tensors = tensor_table(cfg, path, front)
    unknown = set(expose) - set(tensors)
    if unknown:
        raise ValueError(f"cannot expose unknown tensors {sorted(unknown)}")
    ops = operations(cfg, path, front)

    # Workspace: engine-owned temporaries, interval-packed, 256-byte aligned.
    owned = {n: s.nbytes for n, s in tensors.items() if s.role == "temporary" and n not in expose}
    workspace_bytes, slots = pack_workspace(owned, ops, set(PERSISTENT_TENSORS), ALIGN)
    offsets = {sl.name: sl.offset for sl in slots}
    deps = _dependencies(ops)

    bindings: dict[str, list[list[int]]] = {}
    op_records, contracts = [], []
    for oi, op in enumerate(ops):
        arguments = []
        arg_offsets, kernarg = _kernarg_layout(op["args"])
        for ai, a in enumerate(op["args"]):
            if isinstance(a, tuple):
                arguments.append({"kind": "u32_constant", "value": a[1], "offset": arg_offsets[ai]})
            elif a in offsets:
                arguments.append({"kind": "pointer", "source": "workspace", "tensor": a,
                                  "workspace_offset": offsets[a], "offset": arg_offsets[ai]})
            else:
                arguments.append({"kind": "pointer", "source": "binding", "tensor": a, "offset": arg_offsets[ai]})
                bindings.setdefault(a, []).append([0, oi, ai])
        launch = Launch(tuple(op["grid"]), tuple(op["block"]), op["lds"], op["dyn"])
        typ = op_typing(cfg, op, path)
        contract = HipKernelContract(
            operation=op["name"], family="moe.fp8_block128.gfx950_hip", symbol=op["symbol"],
            constants=(("T", cfg.T), ("H", cfg.H), ("I", cfg.I), ("E", cfg.E), ("K", cfg.K),
                       ("S", cfg.S), ("BLOCK_M", BLOCK_M), ("SCALE_BLOCK", 128)),
            semantics=layer_semantics(op["symbol"], path, front),
            launch=launch, kernarg_size=kernarg, code_object_sha256=sha,
            shape=tuple(typ["shape"]), dtypes=tuple(typ["dtypes"]), quantization=_pairs(typ["quantization"]),
            layouts=tuple(typ["layouts"]), epilogue=typ["epilogue"], tactic=plan.selected.name,
            numerical=_pairs(typ["numerical"]), maturity=plan.selected.maturity, fallback=plan.fallback,
            source_refs=tuple(op["refs"]), evidence_refs=tuple(plan.selected.evidence_refs))
        contracts.append(contract.to_dict())
        op_records.append({
            "index": oi, "name": op["name"], "kind": OPERATION_NAME, "contract_id": contract.stable_id,
            "tactic": plan.selected.name, "maturity": plan.selected.maturity, "execution": "kernel",
            "kernel_symbol": op["symbol"], "launch": launch.to_dict(), "workspace_offset": None,
            "fallback": plan.fallback, "bindings": {"inputs": list(op["reads"]), "outputs": list(op["writes"])},
            "artifact_kind": "hip_code_object", "hsaco": "hsaco/" + hsaco.name, "hsaco_sha256": sha,
            "kernarg_size": kernarg, "arguments": arguments,
        })

    selected_symbols = sorted({op["symbol"] for op in ops})
    # kernels of the other tactics that also serve this request (explain.json's compatible candidates)
    other: set[str] = set()
    by_name = {t.name: t for t in catalog()}
    for cand in plan.candidates:
        t = by_name.get(cand["tactic"])
        if t is None or cand["reasons"] or t is plan.selected:
            continue
        other.update(o["symbol"] for o in operations(cfg, t.path, t.front))
    candidate_symbols = sorted(other - set(selected_symbols))
    listing = f"hsaco/{hsaco.stem}.symbols.txt"
    validation["candidates"] = [
        {"symbol": sym, "source": listing, "artifact_kind": "hip_code_object", "hsaco": "hsaco/" + hsaco.name,
         "hsaco_sha256": sha, "selected": sym in selected_symbols}
        for sym in selected_symbols + candidate_symbols]

    engine.update(gemm_path=path, front_end=front, workspace_bytes=workspace_bytes,
                  selected_tactics=[plan.selected.name], kernel_symbols=selected_symbols,
                  operations=op_records, fallbacks={})
    recipe = {
        "format": "netra-graph-recipe-1",
        "profile": profile.name,
        "capture_at_initialization": True,
        "portable_serialized_hip_graph": False,
        "execution": "kernel",
        "gemm_path": path,
        "front_end": front,
        "operations": [{"index": r["index"], "name": r["name"], "depends_on": deps[r["index"]],
                        "execution": "kernel", "kernel_symbol": r["kernel_symbol"], "launch": r["launch"],
                        "bindings": r["bindings"], "workspace_offset": None} for r in op_records],
        "tensors": {n: {"dtype": s.dtype, "shape": list(s.shape), "role": s.role,
                        "bytes": s.nbytes, "storage": "workspace" if n in offsets else "binding"}
                    for n, s in tensors.items()},
        "bindings": bindings,
        "dependencies": deps,
    }
    memory_plan = {"format": "netra-memory-plan-1", "workspace_bytes": workspace_bytes, "alignment": ALIGN,
                   "unpacked_bytes": sum((b + ALIGN - 1) // ALIGN * ALIGN for b in owned.values()),
                   "buffers": [sl.to_dict() for sl in slots], "offsets": offsets}

    (directory / "hsaco").mkdir(exist_ok=True)
    target = directory / "hsaco" / hsaco.name
    if not target.exists() or target.read_bytes() != code:
        shutil.copyfile(hsaco, target)
    (directory / listing).write_text(_symbol_listing(hsaco, code, selected_symbols + candidate_symbols))
    _write(directory, {
        "contracts.json": {"format": "netra-contract-set-1", "contracts": contracts},
        "graph.json": _graph(cfg, tensors, ops), "graph_recipe.json": recipe, "memory_plan.json": memory_plan,
        "layout_plan.json": _layout_plan(), "symbols.json": {"selected": selected_symbols,
                                                             "candidates": candidate_symbols},
        "validation_plan.json": validation, "explain.json": explain, "engine.json": _finish_engine(engine)})
    return recipe
