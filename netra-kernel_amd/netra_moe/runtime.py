"""ctypes binding of the engine C ABI (include/netra_engine.h).

The reference's callers bind the same ABI from Python through ctypes (the
SGLang adapter; reference runtime/gfx950/engine/netra_engine.h:60-108). Errors
raise NetraError carrying the status and the engine's last_error text.
"""
from __future__ import annotations

import ctypes
import enum
from pathlib import Path

from . import paths


class Status(enum.IntEnum):
    OK = 0
    INVALID_ARGUMENT = 1
    IO = 2
    MANIFEST = 3
    UNSUPPORTED_TARGET = 4
    UNSUPPORTED_PROFILE = 5
    BINDING = 6
    HIP = 7
    BUSY = 8
    FALLBACK_REQUIRED = 9


class NetraError(RuntimeError):
    def __init__(self, status: int, message: str):
        self.status = Status(status)
        super().__init__(f"{self.status.name}: {message}")


class EngineOptions(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("device_id", ctypes.c_int32),
                ("enable_graph_capture", ctypes.c_uint32)]


class ProfileInfo(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("profile_id", ctypes.c_uint32),
                ("min_m", ctypes.c_uint32), ("max_m", ctypes.c_uint32),
                ("min_batch", ctypes.c_uint32), ("max_batch", ctypes.c_uint32),
                ("min_sequence", ctypes.c_uint64), ("max_sequence", ctypes.c_uint64),
                ("tensor_parallel", ctypes.c_uint32), ("workspace_bytes", ctypes.c_uint64),
                ("requires_fallback", ctypes.c_uint32)]


class LaunchShape(ctypes.Structure):
    _fields_ = [("m", ctypes.c_uint32), ("batch", ctypes.c_uint32),
                ("sequence", ctypes.c_uint64), ("tensor_parallel", ctypes.c_uint32)]


class PointerBinding(ctypes.Structure):
    _fields_ = [("argument_index", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("pointer", ctypes.c_void_p)]


ENGINE_SYMBOLS = (
    "netra_engine_create", "netra_engine_profile_count", "netra_engine_query_profile",
    "netra_engine_bind", "netra_engine_finalize_bindings", "netra_engine_prepare_profile",
    "netra_engine_launch", "netra_engine_launch_operation", "netra_engine_launch_operation_bound",
    "netra_engine_last_error", "netra_engine_destroy", "netra_engine_manifest_check",
)

_lib = None


def load_library(path: Path | None = None) -> ctypes.CDLL:
    """Load libnetra_engine.so (raises if it has not been built)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    path = Path(path) if path else paths.engine_library()
    if not path.is_file():
        raise FileNotFoundError(f"{path} is missing: build the native library first")
    lib = ctypes.CDLL(str(path))
    vp, u32, st = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int
    lib.netra_engine_create.argtypes = [ctypes.c_char_p, ctypes.POINTER(EngineOptions), ctypes.POINTER(vp)]
    lib.netra_engine_create.restype = st
    lib.netra_engine_profile_count.argtypes = [vp]
    lib.netra_engine_profile_count.restype = ctypes.c_size_t
    lib.netra_engine_query_profile.argtypes = [vp, u32, ctypes.POINTER(ProfileInfo)]
    lib.netra_engine_query_profile.restype = st
    lib.netra_engine_bind.argtypes = [vp, u32, u32, u32, vp]
    lib.netra_engine_bind.restype = st
    lib.netra_engine_finalize_bindings.argtypes = [vp]
    lib.netra_engine_finalize_bindings.restype = st
    lib.netra_engine_prepare_profile.argtypes = [vp, u32, vp]
    lib.netra_engine_prepare_profile.restype = st
    lib.netra_engine_launch.argtypes = [vp, u32, ctypes.POINTER(LaunchShape), vp]
    lib.netra_engine_launch.restype = st
    lib.netra_engine_launch_operation.argtypes = [vp, u32, u32, ctypes.POINTER(LaunchShape), vp]
    lib.netra_engine_launch_operation.restype = st
    lib.netra_engine_launch_operation_bound.argtypes = [vp, u32, u32, ctypes.POINTER(LaunchShape),
                                                        ctypes.POINTER(PointerBinding), u32, vp]
    lib.netra_engine_launch_operation_bound.restype = st
    lib.netra_engine_last_error.argtypes = [vp]
    lib.netra_engine_last_error.restype = ctypes.c_char_p
    lib.netra_engine_destroy.argtypes = [vp]
    lib.netra_engine_destroy.restype = st
    lib.netra_engine_manifest_check.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]
    lib.netra_engine_manifest_check.restype = st
    if path == paths.engine_library():
        _lib = lib
    return lib


def manifest_check(directory: Path) -> tuple[Status, str]:
    """Host-only validation of an engine directory (no GPU needed)."""
    lib = load_library()
    buf = ctypes.create_string_buffer(512)
    status = lib.netra_engine_manifest_check(str(directory).encode(), buf, len(buf))
    return Status(status), buf.value.decode()


class Engine:
    """One loaded engine (netra_engine_t*). Not thread-safe during binding."""

    def __init__(self, directory: Path, *, device_id: int = 0, graph_capture: bool = True):
        self.lib = load_library()
        self.directory = Path(directory)
        opts = EngineOptions(ctypes.sizeof(EngineOptions), device_id, 1 if graph_capture else 0)
        handle = ctypes.c_void_p()
        status = self.lib.netra_engine_create(str(self.directory).encode(), ctypes.byref(opts),
                                              ctypes.byref(handle))
        if status != Status.OK:
            detail = ""
            if status == Status.MANIFEST:
                _, detail = manifest_check(self.directory)
            raise NetraError(status, f"netra_engine_create({self.directory}) {detail}".strip())
        self.handle = handle

    def _check(self, status: int, what: str) -> None:
        if status != Status.OK:
            msg = self.lib.netra_engine_last_error(self.handle) or b""
            raise NetraError(status, f"{what}: {msg.decode()}")

    def profile_count(self) -> int:
        return int(self.lib.netra_engine_profile_count(self.handle))

    def query_profile(self, profile_id: int) -> ProfileInfo:
        info = ProfileInfo()
        info.struct_size = ctypes.sizeof(ProfileInfo)
        self._check(self.lib.netra_engine_query_profile(self.handle, profile_id, ctypes.byref(info)),
                    "query_profile")
        return info

    def bind(self, profile_id: int, op: int, arg: int, pointer: int) -> None:
        self._check(self.lib.netra_engine_bind(self.handle, profile_id, op, arg, ctypes.c_void_p(pointer)),
                    f"bind({profile_id},{op},{arg})")

    def finalize(self) -> None:
        self._check(self.lib.netra_engine_finalize_bindings(self.handle), "finalize_bindings")

    def prepare(self, profile_id: int, stream: int) -> None:
        self._check(self.lib.netra_engine_prepare_profile(self.handle, profile_id, ctypes.c_void_p(stream)),
                    "prepare_profile")

    def launch(self, profile_id: int, shape: LaunchShape, stream: int) -> None:
        self._check(self.lib.netra_engine_launch(self.handle, profile_id, ctypes.byref(shape),
                                                 ctypes.c_void_p(stream)), "launch")

    def launch_operation(self, profile_id: int, op: int, shape: LaunchShape, stream: int) -> None:
        self._check(self.lib.netra_engine_launch_operation(self.handle, profile_id, op, ctypes.byref(shape),
                                                           ctypes.c_void_p(stream)), f"launch_operation({op})")

    def launch_operation_bound(self, profile_id: int, op: int, shape: LaunchShape,
                               bindings: list[tuple[int, int]], stream: int) -> None:
        arr = (PointerBinding * max(1, len(bindings)))()
        for i, (arg, ptr) in enumerate(bindings):
            arr[i] = PointerBinding(arg, 0, ctypes.c_void_p(ptr))
        self._check(self.lib.netra_engine_launch_operation_bound(
            self.handle, profile_id, op, ctypes.byref(shape), arr, len(bindings), ctypes.c_void_p(stream)),
            f"launch_operation_bound({op})")

    def destroy(self) -> None:
        if getattr(self, "handle", None):
            self._check(self.lib.netra_engine_destroy(self.handle), "destroy")
            self.handle = None

    def __del__(self):  # best effort
        try:
            if getattr(self, "handle", None):
                self.lib.netra_engine_destroy(self.handle)
                self.handle = None
        except Exception:
            pass
