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
        L.orc_stage1_routes.argtypes = [P, P, P, P, P, I64, I64, I64, I64, I64, P, I]
        L.orc_silu_mul_quant.argtypes = [P, I64, I64, P, P]
        L.orc_down_reduce_routes.argtypes = [P, P, P, P, P, P, I64, I64, I64, I64, I64, P, P, I]
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


def stage1_routes(x_q, x_s, w13, w13_s, ids, Etot: int, I: int, threads: int | None = None) -> np.ndarray:
    """Per-route gate/up before SiLU: f32 [T*Ktot, 2I] (route r = t*Ktot + s)."""
    T, Ktot = ids.shape
    H = x_q.shape[1]
    out = np.empty((T * Ktot, 2 * I), np.float32)
    arrs = [np.ascontiguousarray(a) for a in (x_q, x_s, w13, w13_s)]
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    lib().orc_stage1_routes(*[_p(a) for a in arrs], _p(ids), T, Ktot, Etot, H, I, _p(out),
                            threads or default_threads())
    return out


def silu_mul_quant(gu: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """fp32 rows [g | u] [rows, 2I] -> (h e4m3 [rows, I], scales f32 [rows, I/128])."""
    gu = np.ascontiguousarray(gu, dtype=np.float32)
    rows, I = gu.shape[0], gu.shape[1] // 2
    q = np.empty((rows, I), np.uint8)
    s = np.empty((rows, I // 128), np.float32)
    lib().orc_silu_mul_quant(_p(gu), rows, I, _p(q), _p(s))
    return q, s


def down_reduce_routes(h_q, h_s, w2, w2_s, ids, weights, Etot: int, threads: int | None = None):
    """Per-route down + slot-ordered reduce per token: (out f32 [T, H], out bf16 bits [T, H])."""
    T, Ktot = ids.shape
    H, I = w2.shape[1], w2.shape[2]
    out_f = np.empty((T, H), np.float32)
    out = np.empty((T, H), np.uint16)
    arrs = [np.ascontiguousarray(a) for a in (h_q, h_s, w2, w2_s)]
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    wts = np.ascontiguousarray(weights, dtype=np.float32)
    lib().orc_down_reduce_routes(*[_p(a) for a in arrs], _p(ids), _p(wts), T, Ktot, Etot, H, I,
                                 _p(out_f), _p(out), threads or default_threads())
    return out_f, out


def shared_gate_append(x_bf16, wsg_bf16, ids, weights, E: int):
    """Shared-expert append (export_qwen36_shared_gate_append_capture.py:97-107,134-139):
    slots 0..K-1 copy the routed ids/weights, slot K = (E, f32(bf16(sigmoid(logit)))) with
    the logit in the router contract order."""
    T, K = ids.shape
    logit = router_logits(x_bf16, np.ascontiguousarray(wsg_bf16).reshape(1, -1))[:, 0]
    gate = np.array([lib().orc_f32_from_bf16(lib().orc_bf16_from_f32(
        lib().orc_sigmoid(lib().orc_f32_from_bf16(int(b))))) for b in logit], dtype=np.float32)
    out_ids = np.concatenate([ids.astype(np.int32), np.full((T, 1), E, np.int32)], axis=1)
    out_w = np.concatenate([weights.astype(np.float32), gate[:, None]], axis=1)
    return out_ids, out_w


def stage2_split_halves(h_q, h_s, w2, w2_s, experts) -> tuple[np.ndarray, np.ndarray]:
    """Split-K2 down partials per route row (the format of the reference's
    prefill producer, moe_prefill_m768_bridge.hip:144-147): half j sums the
    K blocks [j I/256, (j+1) I/256) of sum_kb ((h8 . w8) * h_s) * w_s, in
    float64. h rows [R, I] with their experts [R]; returns two [R, H] arrays."""
    table = e4m3_table().astype(np.float64)
    R, I = h_q.shape
    KB = I // 128
    out = [np.zeros((R, w2.shape[1])), np.zeros((R, w2.shape[1]))]
    for r in range(R):
        e = int(experts[r])
        h = table[h_q[r]].reshape(KB, 128)
        w = table[w2[e]].reshape(-1, KB, 128)
        ws = np.repeat(w2_s[e].astype(np.float64), 128, axis=0)  # [H, KB]
        dots = np.einsum("nkc,kc->nk", w, h) * h_s[r].astype(np.float64)[None, :] * ws
        out[0][r] = dots[:, : KB // 2].sum(axis=1)
        out[1][r] = dots[:, KB // 2:].sum(axis=1)
    return out[0], out[1]


def max_abs_rel(y: np.ndarray, ref: np.ndarray) -> float:
    """max |y - ref| / max |ref| (the layer's tolerance metric)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = float(np.max(np.abs(ref)))
    return float(np.max(np.abs(y - ref))) / denom if denom > 0 else float(np.max(np.abs(y - ref)))


# ---- checkpoint stacking ----------------------------------------------------------------
# Restates the weight-prep plan of reference compiler/netra_compiler/layouts.py:109-206
# (output shards concatenated along axis 0, bf16 block scales widened exactly to
# fp32) for the layer's stacked tensors: routed experts 0..E-1, the shared expert
# as expert E, W13 rows gate then up. Pinned by tests/test_prep_oracle.py
# (element-wise tile placement against the documented permutation, shard and
# shared-expert positions, exact widening).

def tile16x128(q: np.ndarray, gate_up: bool = False) -> np.ndarray:
    """Place every byte of row-major [G, N, K] e4m3 codes at its tile16x128
    position, computed per element: row tile r = n // 16, K block b = k // 128,
    half = (k % 32) // 16, lane = (k % 128) // 32 * 16 + n % 16, byte k % 16;
    tile (r, b) is 2048 bytes at (r' * K/128 + b) * 2048 with the half at
    half * 1024 and the lane at lane * 16. r' = r, or for W13 (gate_up) the
    interleaved order: gate tile j (r = j < N/32) at 2j, up tile j (r = N/32 + j)
    at 2j + 1."""
    g, n, k = q.shape
    nn, kk = np.meshgrid(np.arange(n), np.arange(k), indexing="ij")
    r, b = nn // 16, kk // 128
    if gate_up:
        half_tiles = n // 32
        r = np.where(r < half_tiles, 2 * r, 2 * (r - half_tiles) + 1)
    lane = (kk % 128) // 32 * 16 + nn % 16
    dst = (r * (k // 128) + b) * 2048 + ((kk % 32) // 16) * 1024 + lane * 16 + kk % 16
    out = np.empty((g, n * k), dtype=np.uint8)
    out[:, dst.reshape(-1)] = q.reshape(g, n * k)
    return out.reshape(g, n, k)


def _scale_f32(a: np.ndarray) -> np.ndarray:
    """Scale block grid as fp32: uint16 arrays are bf16 bit patterns (exact widening)."""
    return f32_from_bf16(a) if a.dtype == np.uint16 else np.asarray(a, np.float32)


def stack_checkpoint(tensors: dict, E: int, S: int, H: int, I: int, prefix: str) -> dict:
    """{name: array or list of output shards} -> w13 / w13_scale / w2 / w2_scale
    as the layer binds them (weights in tile16x128, scales fp32)."""
    def name(e, proj, scale=False):
        owner = "shared_expert" if e is None else f"experts.{e}"
        return f"{prefix}.{owner}.{proj}.{'weight_scale_inv' if scale else 'weight'}"

    def cat(v):
        return np.concatenate(v, axis=0) if isinstance(v, (list, tuple)) else np.asarray(v)

    experts = list(range(E)) + [None] * S
    w13 = np.stack([np.concatenate([cat(tensors[name(e, "gate_proj")]), cat(tensors[name(e, "up_proj")])], axis=0)
                    for e in experts])
    w2 = np.stack([cat(tensors[name(e, "down_proj")]) for e in experts])
    s13 = np.stack([np.concatenate([_scale_f32(cat(tensors[name(e, "gate_proj", True)])),
                                    _scale_f32(cat(tensors[name(e, "up_proj", True)]))], axis=0) for e in experts])
    s2 = np.stack([_scale_f32(cat(tensors[name(e, "down_proj", True)])) for e in experts])
    assert w13.shape == (E + S, 2 * I, H) and w2.shape == (E + S, H, I)
    return {"w13": tile16x128(w13.astype(np.uint8), gate_up=True), "w13_scale": s13.astype(np.float32),
            "w2": tile16x128(w2.astype(np.uint8)), "w2_scale": s2.astype(np.float32)}
