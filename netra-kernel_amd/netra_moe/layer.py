"""Host side of one MoE layer: compile the engine, own its buffers, bind, launch.

PyTorch provides device memory and the stream only; all computation runs in the
engine's HIP kernels through the C ABI. The layer refuses to run without the
native library or a GPU (no CPU fallback exists in the product path).
"""
from __future__ import annotations

import hashlib
import json
import os
import tempfile
from pathlib import Path

import torch

from .config import MoEConfig
from .engine import compile_moe_engine, op_names, resolve_front, resolve_path, tensor_table
from .runtime import Engine, LaunchShape

TORCH_DTYPES = {"bf16": torch.bfloat16, "f32": torch.float32, "e4m3": torch.uint8,
                "i32": torch.int32, "u32": torch.int32, "u64": torch.int64}
WEIGHT_NAMES = ("router_w", "router_bias", "w13", "w13_scale", "w2", "w2_scale")


def _engine_cache_dir(cfg: MoEConfig, expose: tuple[str, ...], path: str, front: str) -> Path:
    root = Path(os.environ.get("NETRA_MOE_ENGINE_CACHE", Path(tempfile.gettempdir()) / "netra_moe_engines"))
    key = hashlib.sha256(json.dumps([cfg.to_dict(), sorted(expose), path, front],
                                    sort_keys=True).encode()).hexdigest()[:16]
    return root / f"{cfg.name}-{key}"


def check_tensor(name: str, t: torch.Tensor, dtype: str, shape: tuple[int, ...], device: torch.device) -> None:
    want = TORCH_DTYPES[dtype]
    if t.dtype != want or tuple(t.shape) != tuple(shape) or not t.is_contiguous() or t.device != device:
        raise ValueError(f"{name}: need {want} {tuple(shape)} contiguous on {device}, "
                         f"got {t.dtype} {tuple(t.shape)} contiguous={t.is_contiguous()} on {t.device}")


class MoELayer:
    def __init__(self, cfg: MoEConfig, weights: dict[str, torch.Tensor], *, device: int = 0,
                 expose: tuple[str, ...] = (), graph: bool = True, engine_dir: Path | None = None,
                 path: str = "auto", front: str = "auto"):
        if not torch.cuda.is_available():
            raise RuntimeError("MoELayer needs a ROCm GPU; there is no CPU fallback")
        self.cfg = cfg
        self.device = torch.device("cuda", device)
        self.expose = tuple(expose)
        self.path = resolve_path(cfg, path)
        self.front = resolve_front(cfg, self.path, front)
        self.op_names = op_names(cfg, self.path, self.front)
        self.engine_dir = Path(engine_dir) if engine_dir else _engine_cache_dir(cfg, self.expose, self.path,
                                                                                self.front)
        self.recipe = compile_moe_engine(cfg, self.engine_dir, expose=self.expose, path=self.path,
                                         front=self.front)
        self.specs = tensor_table(cfg, self.path, self.front)
        with torch.cuda.device(self.device):
            self.engine = Engine(self.engine_dir, device_id=device, graph_capture=graph)
        self.graph = graph
        self.buffers: dict[str, torch.Tensor] = {}
        for name in WEIGHT_NAMES:
            spec = self.specs[name]
            check_tensor(name, weights[name], spec.dtype, spec.shape, self.device)
            self.buffers[name] = weights[name]
        for name, info in self.recipe["tensors"].items():
            if info["storage"] == "binding" and name not in self.buffers:
                spec = self.specs[name]
                # zeroed: some temporaries (hand-off counters) must start at zero,
                # as the engine's own workspace does
                self.buffers[name] = torch.zeros(spec.shape, dtype=TORCH_DTYPES[spec.dtype], device=self.device)
        for name, slots in self.recipe["bindings"].items():
            ptr = self.buffers[name].data_ptr()
            for profile, op, arg in slots:
                self.engine.bind(profile, op, arg, ptr)
        self.engine.finalize()
        self.shape = LaunchShape(cfg.T, 1, 0, 1)
        self._prepared = False

    @property
    def x(self) -> torch.Tensor:
        return self.buffers["x"]

    @property
    def out(self) -> torch.Tensor:
        return self.buffers["out"]

    def buffer(self, name: str) -> torch.Tensor:
        if name not in self.buffers:
            raise KeyError(f"{name} is engine-internal; construct the layer with expose=('{name}',)")
        return self.buffers[name]

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def forward(self, x: torch.Tensor | None = None) -> torch.Tensor:
        """Run the layer on the current stream; returns the (reused) output buffer."""
        if x is not None and x.data_ptr() != self.x.data_ptr():
            check_tensor("x", x, "bf16", (self.cfg.T, self.cfg.H), self.device)
            self.x.copy_(x)
        stream = self._stream()
        if self.graph and not self._prepared:
            # Capture needs a non-legacy stream; the executable graph then
            # replays on whatever stream the caller launches it on.
            capture = torch.cuda.Stream(self.device)
            self.engine.prepare(0, capture.cuda_stream)
            self._capture_stream = capture
            self._prepared = True
        self.engine.launch(0, self.shape, stream)
        return self.out

    def run_operation(self, index_or_name: int | str) -> None:
        """Launch one operation (direct-launch engines only)."""
        idx = self.op_names.index(index_or_name) if isinstance(index_or_name, str) else int(index_or_name)
        self.engine.launch_operation(0, idx, self.shape, self._stream())

    def close(self) -> None:
        torch.cuda.synchronize(self.device)
        self.engine.destroy()
