"""Weight preparation and synthetic layer inputs.

quantize_blocks() runs the gfx950 weight-prep kernel (libnetra_moe.so,
include/netra_moe.h) that turns fp32 expert weights into E4M3 with 128x128
fp32 block scales. synthetic_* build the seeded inputs of the benchmark
configurations: activations bf16 ~ N(0, 1), router and shared-gate weights
bf16 ~ N(0, 0.02), expert weights ~ N(0, 0.02) quantised at setup, and for the
speculative-verification config an expert bias log(Zipf(1.1)) over a seeded
permutation of the routed experts.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from . import paths
from .config import MoEConfig

_bridge = None


def bridge_library() -> ctypes.CDLL:
    global _bridge
    if _bridge is None:
        path = paths.bridge_library()
        if not path.is_file():
            raise FileNotFoundError(f"{path} is missing: build the native library first")
        lib = ctypes.CDLL(str(path))
        lib.netra_moe_quant_blocks.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_uint32] * 3 + [ctypes.c_void_p]
        lib.netra_moe_quant_blocks.restype = ctypes.c_int
        lib.netra_moe_pack_tiles.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_uint32] * 3 + [ctypes.c_void_p]
        lib.netra_moe_pack_tiles.restype = ctypes.c_int
        lib.netra_moe_pack_tiles_gate_up.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_uint32] * 3 + [ctypes.c_void_p]
        lib.netra_moe_pack_tiles_gate_up.restype = ctypes.c_int
        for fn in (lib.netra_moe_pack_tiles_from_aiter, lib.netra_moe_pack_tiles_gate_up_from_aiter):
            fn.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_uint32] * 3 + [ctypes.c_void_p]
            fn.restype = ctypes.c_int
        lib.netra_moe_e4m3_check.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_uint32, ctypes.c_void_p]
        lib.netra_moe_e4m3_check.restype = ctypes.c_int
        lib.netra_moe_copy.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_uint64, ctypes.c_void_p]
        lib.netra_moe_copy.restype = ctypes.c_int
        lib.netra_moe_prefill_launch_noalloc.argtypes = [ctypes.c_void_p] * 14 + [ctypes.c_uint32, ctypes.c_void_p]
        lib.netra_moe_prefill_launch_noalloc.restype = ctypes.c_int
        lib.netra_moe_last_error.argtypes = []
        lib.netra_moe_last_error.restype = ctypes.c_char_p
        _bridge = lib
    return _bridge


def quantize_blocks(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 [G, N, K] on the GPU -> (e4m3 bytes [G, N, K], fp32 scales [G, N/128, K/128])."""
    if w.dim() != 3 or w.dtype != torch.float32 or not w.is_cuda or not w.is_contiguous():
        raise ValueError("quantize_blocks needs a contiguous fp32 [G, N, K] GPU tensor")
    g, n, k = w.shape
    if n % 128 or k % 128:
        raise ValueError("N and K must be multiples of 128")
    q = torch.empty((g, n, k), dtype=torch.uint8, device=w.device)
    s = torch.empty((g, n // 128, k // 128), dtype=torch.float32, device=w.device)
    stream = torch.cuda.current_stream(w.device).cuda_stream
    lib = bridge_library()
    rc = lib.netra_moe_quant_blocks(w.data_ptr(), q.data_ptr(), s.data_ptr(), g, n, k, stream)
    if rc != 0:
        raise RuntimeError(f"netra_moe_quant_blocks failed ({rc}): {lib.netra_moe_last_error().decode()}")
    return q, s


def pack_tiles(q: torch.Tensor, gate_up: bool = False) -> torch.Tensor:
    """Row-major e4m3 bytes [G, N, K] on the GPU -> the kernels' tile16x128 layout
    (gate_up: W13, row tiles gate/up-interleaved, netra_moe_pack_tiles_gate_up)."""
    if q.dim() != 3 or q.dtype != torch.uint8 or not q.is_cuda or not q.is_contiguous():
        raise ValueError("pack_tiles needs a contiguous uint8 [G, N, K] GPU tensor")
    g, n, k = q.shape
    if n % (32 if gate_up else 16) or k % 128:
        raise ValueError("N must be a multiple of 16 (32 for W13) and K of 128")
    out = torch.empty_like(q)
    lib = bridge_library()
    fn = lib.netra_moe_pack_tiles_gate_up if gate_up else lib.netra_moe_pack_tiles
    rc = fn(q.data_ptr(), out.data_ptr(), g, n, k, torch.cuda.current_stream(q.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(f"weight packing failed ({rc}): {lib.netra_moe_last_error().decode()}")
    return out


def pack_tiles_from_aiter(q: torch.Tensor, gate_up: bool = False) -> torch.Tensor:
    """AITER 16x16-shuffled e4m3 bytes [G, N, K] on the GPU (the layout the
    reference's kernels consume) -> the kernels' tile16x128 layout, as
    pack_tiles() would produce from the row-major bytes."""
    if q.dim() != 3 or q.dtype != torch.uint8 or not q.is_cuda or not q.is_contiguous():
        raise ValueError("pack_tiles_from_aiter needs a contiguous uint8 [G, N, K] GPU tensor")
    g, n, k = q.shape
    if n % (32 if gate_up else 16) or k % 128:
        raise ValueError("N must be a multiple of 16 (32 for W13) and K of 128")
    out = torch.empty_like(q)
    lib = bridge_library()
    fn = lib.netra_moe_pack_tiles_gate_up_from_aiter if gate_up else lib.netra_moe_pack_tiles_from_aiter
    rc = fn(q.data_ptr(), out.data_ptr(), g, n, k, torch.cuda.current_stream(q.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(f"weight packing failed ({rc}): {lib.netra_moe_last_error().decode()}")
    return out


def aiter_shuffle_host(q: np.ndarray) -> np.ndarray:
    """AITER 16x16 shuffle of row-major bytes [..., N, K]: element (n, k) goes to
    [n/16][k/32][(k%32)/16][n%16][k%16] (the inverse of
    tools/benchmark/export_qwen36_dense_m1_capture.py:55-63)."""
    *lead, n, k = q.shape
    t = q.reshape(*lead, n // 16, 16, k // 32, 2, 16)
    nd = len(lead)
    t = t.transpose(*range(nd), nd, nd + 2, nd + 3, nd + 1, nd + 4)
    return np.ascontiguousarray(t).reshape(*lead, n, k)


def device_copy(src: torch.Tensor, dst: torch.Tensor) -> None:
    """Byte copy src -> dst (same size, GPU, 16-byte multiple) by the library's
    plain streaming kernel, on the current stream."""
    n = src.numel() * src.element_size()
    if not (src.is_cuda and dst.is_cuda and src.is_contiguous() and dst.is_contiguous()) or \
            n != dst.numel() * dst.element_size():
        raise ValueError("device_copy needs two contiguous GPU tensors of the same byte size")
    lib = bridge_library()
    rc = lib.netra_moe_copy(src.data_ptr(), dst.data_ptr(), n, torch.cuda.current_stream(src.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(f"netra_moe_copy failed ({rc}): {lib.netra_moe_last_error().decode()}")


def gu_order(nt: int) -> np.ndarray:
    """Stored row-tile order of a gate/up-interleaved W13 with nt row tiles:
    position 2t holds gate tile t, 2t + 1 holds up tile t (logical nt/2 + t)."""
    half = nt // 2
    return np.stack([np.arange(half), np.arange(half) + half], axis=1).reshape(-1)


def pack_tiles_host(q: np.ndarray, gate_up: bool = False) -> np.ndarray:
    """Host restatement of the tile16x128 layout: [G, N, K] ->
    [G, N/16, K/128, half, lane, 16 bytes] with lane = (k % 128) // 32 * 16 + n % 16
    and half = (k % 32) // 16 (returned with the original shape); with gate_up the
    row tiles are stored in gu_order."""
    g, n, k = q.shape
    t = q.reshape(g, n // 16, 16, k // 128, 4, 2, 16).transpose(0, 1, 3, 5, 4, 2, 6)
    t = np.ascontiguousarray(t)
    if gate_up:
        t = t[:, gu_order(n // 16)]
    return np.ascontiguousarray(t).reshape(g, n, k)


def unpack_tiles_host(q: np.ndarray, gate_up: bool = False) -> np.ndarray:
    """Inverse of pack_tiles_host: tile16x128 bytes [G, N, K] -> row-major."""
    g, n, k = q.shape
    t = q.reshape(g, n // 16, k // 128, 2, 4, 16, 16)
    if gate_up:
        t = t[:, np.argsort(gu_order(n // 16))]
    t = t.transpose(0, 1, 5, 2, 4, 3, 6)
    return np.ascontiguousarray(t).reshape(g, n, k)


def zipf_bias(E: int, seed: int, s: float = 1.1) -> np.ndarray:
    """bias[e] = log p(rank(e)), p(r) proportional to r^-s over r = 1..E."""
    ranks = np.arange(1, E + 1, dtype=np.float64)
    p = ranks ** (-s)
    p /= p.sum()
    perm = np.random.default_rng(seed).permutation(E)
    bias = np.empty(E, dtype=np.float32)
    bias[perm] = np.log(p).astype(np.float32)
    return bias


def synthetic_activations(cfg: MoEConfig, device: torch.device | str = "cpu") -> dict[str, torch.Tensor]:
    """x, router_w (router rows + shared-gate row), router_bias; generated on the CPU."""
    g = torch.Generator().manual_seed(cfg.seed)
    x = torch.randn((cfg.T, cfg.H), generator=g, dtype=torch.float32).to(torch.bfloat16)
    router_w = (torch.randn((cfg.router_rows, cfg.H), generator=g, dtype=torch.float32) * 0.02).to(torch.bfloat16)
    if cfg.router_bias == "zipf1.1":
        bias = torch.from_numpy(zipf_bias(cfg.E, cfg.seed))
    elif cfg.router_bias == "hot":  # every token picks experts 0..K-1: K experts hold all rows
        bias = torch.zeros(cfg.E, dtype=torch.float32)
        bias[:cfg.K] = 64.0
    else:
        bias = torch.zeros(cfg.E, dtype=torch.float32)
    return {"x": x.to(device), "router_w": router_w.to(device), "router_bias": bias.to(device)}


def synthetic_expert_weights_f32(cfg: MoEConfig, seed: int, device: torch.device | str) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 W13 [Etot, 2I, H] and W2 [Etot, H, I] ~ N(0, 0.02)."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    w13 = torch.randn((cfg.Etot, 2 * cfg.I, cfg.H), generator=g, device=dev, dtype=torch.float32)
    w13.mul_(0.02)
    w2 = torch.randn((cfg.Etot, cfg.H, cfg.I), generator=g, device=dev, dtype=torch.float32)
    w2.mul_(0.02)
    return w13, w2


def prepare_expert_weights(w13: torch.Tensor, w2: torch.Tensor, keep_row_major: bool = False):
    """fp32 W13 [Etot, 2I, H], W2 [Etot, H, I] on the GPU -> the layer's weight
    tensors (e4m3 in the tile16x128 layout, W13 gate/up-interleaved, + fp32
    128x128 block scales). With
    keep_row_major the row-major e4m3 bytes are returned as well."""
    q13, s13 = quantize_blocks(w13)
    q2, s2 = quantize_blocks(w2)
    out = {"w13": pack_tiles(q13, gate_up=True), "w13_scale": s13, "w2": pack_tiles(q2), "w2_scale": s2}
    if keep_row_major:
        out["w13_row_major"], out["w2_row_major"] = q13, q2
    return out


def synthetic_expert_weights(cfg: MoEConfig, seed: int, device: torch.device | str,
                             keep_row_major: bool = False) -> dict[str, torch.Tensor]:
    """Quantised, packed expert weights generated and prepared on the GPU."""
    w13, w2 = synthetic_expert_weights_f32(cfg, seed, device)
    out = prepare_expert_weights(w13, w2, keep_row_major)
    del w13, w2
    return out


def expert_bytes_touched(cfg: MoEConfig, topk_ids: np.ndarray) -> tuple[int, int]:
    """(distinct experts touched, their weight+scale bytes) for one call's routing."""
    touched = int(np.unique(topk_ids.reshape(-1)).size)
    return touched, touched * cfg.expert_bytes()


def flops_to_tflops(flops: int, seconds: float) -> float:
    return flops / seconds / 1e12 if seconds > 0 else math.nan
