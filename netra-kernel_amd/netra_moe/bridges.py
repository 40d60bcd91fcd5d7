"""ctypes binding of the per-operation bridge ABIs (include/netra_qwen36_bridges.h,
libnetra_bridges.so), in the form the reference's Python callers bind its
bridges (the SGLang adapter loads each bridge library with ctypes and calls
load once before graph capture, then launch per step).

Every call returns the C status; `check` raises BridgeError with the family's
last_error text on a nonzero status.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

from . import paths

P, I32, U32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32

# family -> (argtypes of launch)
LAUNCH_ARGTYPES = {
    "netra_qwen36_router_bf16": [P, P, P, U32, P],
    "netra_qwen36_shared_gate_append": [P, P, P, P, P, P, U32, P],
    "netra_qwen36_moe_silu_mul_quant": [P, P, P, I32, P],
    "netra_qwen36_moe_down_reduce": [P, P, P, P, P, P, P, I32, P],
    "netra_qwen36_moe_gate_up": [P, P, P, P, P, P, I32, P],
    "netra_moe_prefill_m768": [P] * 14 + [P],
}
FAMILIES = tuple(LAUNCH_ARGTYPES)
BRIDGE_SYMBOLS = tuple(f"{fam}_{verb}" for fam in FAMILIES for verb in ("load", "launch", "unload", "last_error"))


class BridgeError(RuntimeError):
    def __init__(self, family: str, code: int, message: str):
        self.family, self.code = family, code
        super().__init__(f"{family}: status {code}: {message}")


_lib = None


def library() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        path = paths.ops_bridge_library()
        if not path.is_file():
            raise FileNotFoundError(f"{path} is missing: build the native library first")
        lib = ctypes.CDLL(str(path))
        for fam, argtypes in LAUNCH_ARGTYPES.items():
            load = getattr(lib, f"{fam}_load")
            load.argtypes = [ctypes.c_char_p, ctypes.c_char_p] if fam == "netra_moe_prefill_m768" else [ctypes.c_char_p]
            load.restype = ctypes.c_int
            launch = getattr(lib, f"{fam}_launch")
            launch.argtypes = argtypes
            launch.restype = ctypes.c_int
            getattr(lib, f"{fam}_unload").argtypes = []
            getattr(lib, f"{fam}_unload").restype = ctypes.c_int
            getattr(lib, f"{fam}_last_error").argtypes = []
            getattr(lib, f"{fam}_last_error").restype = ctypes.c_char_p
        _lib = lib
    return _lib


def last_error(family: str) -> str:
    return (getattr(library(), f"{family}_last_error")() or b"").decode()


def check(family: str, code: int) -> int:
    if code != 0:
        raise BridgeError(family, code, last_error(family))
    return code


def load(family: str, hsaco: Path | None = None) -> int:
    """Load this build's code object for one family (both paths for the prefill pair)."""
    path = str(hsaco or paths.hsaco_path()).encode()
    fn = getattr(library(), f"{family}_load")
    return fn(path, path) if family == "netra_moe_prefill_m768" else fn(path)


def launch(family: str, *args) -> int:
    return getattr(library(), f"{family}_launch")(*args)


def unload(family: str) -> int:
    return getattr(library(), f"{family}_unload")()
