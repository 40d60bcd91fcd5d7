"""numpy front end of the CPU oracle (libmoe_oracle.so, built from moe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package. Each wrapper names
the reference file the C function restates (see moe_oracle.c).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libmoe_oracle.so"
BLOCK_M = 64

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.orc_bf16_from_f32.argtypes = [ctypes.c_float]; L.orc_bf16_from_f32.restype = ctypes.c_uint16
        L.orc_f32_from_bf16.argtypes = [ctypes.c_uint16]; L.orc_f32_from_bf16.restype = ctypes.c_float
        L.orc_e4m3_from_f32.argtypes = [ctypes.c_float]; L.orc_e4m3_from_f32.restype = ctypes.c_uint8
        L.orc_f32_from_e4m3.argtypes = [ctypes.c_uint8]; L.orc_f32_from_e4m3.restype = ctypes.c_float
        for name in ("orc_exp", "orc_silu", "orc_sigmoid"):
            getattr(L, name).argtypes = [ctypes.c_float]
            getattr(L, name).restype = ctypes.c_float
        L.orc_quant_rows_bf16.argtypes = [P, I64, I64, P, P]
        L.orc_quant_blocks_f32.argtypes = [P, I64, I64, I64, P, P, I]
        L.orc_router_logits.argtypes = [P, P, I64, I64, I64, P, I]
        L.orc_topk.argtypes = [P, P, I64, I64, I64, I64, P, P]
        L.orc_capacity_blocks.argtypes = [I64, I64, I64, I64]; L.orc_capacity_blocks.restype = I64
        L.orc_sort.argtypes = [P, I64, I64, I64, I64, I64, P, P, P, P, P, P]; L.orc_sort.restype = I64
        L.orc_gate_up.argtypes = [P, P, P, P, P, P, I64, I64, I64, I64, I64, P, P, P, I]
        L.orc_down_combine.argtypes = [P, P, P, P, P, P, I64, P, I64, I64, I64, I64, I64, P, P, P, I]
        L.orc_moe_tokens.argtypes = [P, P, P, P, P, P, P, P, P, I64, I64, I64, I64, P, P, I]
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def default_threads() -> int:
    return int(os.environ.get("NETRA_ORACLE_THREADS", os.cpu_count() or 1))


# ---- scalar numerics --------------------------------------------------------
def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    """Vectorised RNE to bf16 bits (same rule as orc_bf16_from_f32)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def f32_from_bf16(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_table() -> np.ndarray:
    L = lib()
    return np.array([L.orc_f32_from_e4m3(i) for i in range(256)], dtype=np.float32)


# ---- stages -------------------------------------------------------------------
def quant_rows_bf16(x_bf16: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """1x128 activation quant (a5/a7 rule)."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty((rows, cols // 128), np.float32)
    lib().orc_quant_rows_bf16(_p(x), rows, cols, _p(q), _p(s))
    return q, s


def quant_blocks_f32(w: np.ndarray, threads: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    w = np.ascontiguousarray(w, dtype=np.float32)
    g, n, k = w.shape
    q = np.empty((g, n, k), np.uint8)
    s = np.empty((g, n // 128, k // 128), np.float32)
    lib().orc_quant_blocks_f32(_p(w), g, n, k, _p(q), _p(s), threads or default_threads())
    return q, s


def router_logits(x_bf16: np.ndarray, w_bf16: np.ndarray, threads: int | None = None) -> np.ndarray:
    """a1: bf16 logits in the contract's fp32 order."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    T, H = x.shape
    rows = w.shape[0]
    out = np.empty((T, rows), np.uint16)
    lib().orc_router_logits(_p(x), _p(w), T, H, rows, _p(out), threads or default_threads())
    return out


def topk(logits_bf16: np.ndarray, bias: np.ndarray | None, E: int, K: int, S: int):
    """a2 + a3: ids int32 [T, K+S], weights f32 [T, K+S]."""
    l = np.ascontiguousarray(logits_bf16, dtype=np.uint16)
    T = l.shape[0]
    assert l.shape[1] == E + S
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    ids = np.empty((T, K + S), np.int32)
    w = np.empty((T, K + S), np.float32)
    lib().orc_topk(_p(l), _p(b), T, E, K, S, _p(ids), _p(w))
    return ids, w


def capacity_blocks(T: int, Ktot: int, Etot: int, bm: int = BLOCK_M) -> int:
    return int(lib().orc_capacity_blocks(T, Ktot, Etot, bm))


def sort(ids: np.ndarray, Etot: int, cap_blocks: int | None = None, bm: int = BLOCK_M,
         with_tiles: bool = False):
    """a4: (sorted_ids, sorted_expert, num_valid, counts[, tile_map, pair_map])."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, Ktot = ids.shape
    cap = cap_blocks if cap_blocks is not None else capacity_blocks(T, Ktot, Etot, bm)
    sid = np.empty(cap * bm, np.int32)
    sexp = np.empty(cap, np.int32)
    tmap = np.full((T * Ktot + 15) // 16 + Etot, -1, np.int32)
    pmap = np.full(cap, -1, np.int32)
    nv = np.empty(4, np.int32)
    counts = np.empty(Etot, np.int32)
    rows = lib().orc_sort(_p(ids), T, Ktot, Etot, bm, cap, _p(sid), _p(sexp), _p(tmap), _p(pmap),
                          _p(nv), _p(counts))
    if rows < 0:
        raise ValueError("invalid routing ids or capacity too small")
    if with_tiles:
        return sid, sexp, nv, counts, tmap, pmap
    return sid, sexp, nv, counts


def gate_up(x_q, x_s, w13, w13_s, sorted_ids, sorted_expert, num_valid_rows, T, H, I,
            threads: int | None = None, bm: int = BLOCK_M):
    """a6 + a7 over the sorted rows: (h_q, h_s, h_bf16) in sorted layout.
    Row r uses expert sorted_expert[r // bm]; bm = 1 with per-row experts
    evaluates an arbitrary selection of sorted rows."""
    rows = sorted_ids.shape[0]
    h_q = np.zeros((rows, I), np.uint8)
    h_s = np.zeros((rows, I // 128), np.float32)
    h_b = np.zeros((rows, I), np.uint16)
    arrs = [np.ascontiguousarray(a) for a in (x_q, x_s, w13, w13_s, sorted_ids, sorted_expert)]
    lib().orc_gate_up(*[_p(a) for a in arrs], int(num_valid_rows), T, H, I, bm,
                      _p(h_q), _p(h_s), _p(h_b), threads or default_threads())
    return h_q, h_s, h_b


def gate_up_rows(x_q, x_s, w13, w13_s, sorted_ids, sorted_expert, rows, T, H, I,
                 threads: int | None = None):
    """gate_up() on the sorted rows listed in `rows` only (any order):
    (h_q, h_s) with one row per entry of `rows`."""
    rows = np.asarray(rows, dtype=np.int64)
    sid = np.ascontiguousarray(sorted_ids[rows], dtype=np.int32)
    sexp = np.ascontiguousarray(sorted_expert[rows // BLOCK_M], dtype=np.int32)
    h_q, h_s, _ = gate_up(x_q, x_s, w13, w13_s, sid, sexp, rows.size, T, H, I, threads, bm=1)
    return h_q, h_s


def down_combine(h_q, h_s, w2, w2_s, sorted_ids, sorted_expert, num_valid_rows, weights, T, H, I,
                 threads: int | None = None):
    """a8: (partial f32 [T*Ktot, H], out_f32 [T, H], out bf16 bits [T, H])."""
    Ktot = weights.shape[1]
    partial = np.zeros((T * Ktot, H), np.float32)
    out_f = np.empty((T, H), np.float32)
    out = np.empty((T, H), np.uint16)
    arrs = [np.ascontiguousarray(a) for a in (h_q, h_s, w2, w2_s, sorted_ids, sorted_expert)]
    wts = np.ascontiguousarray(weights, dtype=np.float32)
    lib().orc_down_combine(*[_p(a) for a in arrs], int(num_valid_rows), _p(wts), T, H, I, Ktot,
                           BLOCK_M, _p(partial), _p(out_f), _p(out), threads or default_threads())
    return partial, out_f, out


def moe_tokens(x_q, x_s, w13, w13_s, w2, w2_s, ids, weights, tokens, H, I, threads: int | None = None):
    """Token-major whole expert path for the listed tokens: (out_f32, out bf16 bits)."""
    tokens = np.ascontiguousarray(tokens, dtype=np.int64)
    Ktot = ids.shape[1]
    n = tokens.shape[0]
    out_f = np.empty((n, H), np.float32)
    out = np.empty((n, H), np.uint16)
    arrs = [np.ascontiguousarray(a) for a in (x_q, x_s, w13, w13_s, w2, w2_s)]
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    wts = np.ascontiguousarray(weights, dtype=np.float32)
    lib().orc_moe_tokens(*[_p(a) for a in arrs], _p(ids), _p(wts), _p(tokens), n, H, I, Ktot,
                         _p(out_f), _p(out), threads or default_threads())
    return out_f, out


def moe_layer(x_bf16, router_w, bias, w13, w13_s, w2, w2_s, E, K, S, I, threads: int | None = None):
    """Whole layer through the sorted path. Returns a dict of every stage."""
    T, H = x_bf16.shape
    logits = router_logits(x_bf16, router_w, threads)
    ids, wts = topk(logits, bias, E, K, S)
    x_q, x_s = quant_rows_bf16(x_bf16)
    sid, sexp, nv, counts = sort(ids, E + S)
    h_q, h_s, h_b = gate_up(x_q, x_s, w13, w13_s, sid, sexp, nv[0], T, H, I, threads)
    partial, out_f, out = down_combine(h_q, h_s, w2, w2_s, sid, sexp, nv[0], wts, T, H, I, threads)
    return dict(logits=logits, topk_ids=ids, topk_weights=wts, x_q=x_q, x_scale=x_s,
                sorted_ids=sid, sorted_expert=sexp, num_valid=nv, expert_counts=counts,
                h_q=h_q, h_scale=h_s, h_bf16=h_b, partial=partial, out_f32=out_f, out=out)


def max_abs_rel(y: np.ndarray, ref: np.ndarray) -> float:
    """max |y - ref| / max |ref| (the layer's tolerance metric)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = float(np.max(np.abs(ref)))
    return float(np.max(np.abs(y - ref))) / denom if denom > 0 else float(np.max(np.abs(y - ref)))
