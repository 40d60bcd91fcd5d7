"""MI355X-native (gfx950) FP8 E4M3 block-scaled routed-MoE behind the Netra
engine C ABI.

Host-side mirror of the reference's compiler surface for this path
(contracts, profiles, engine emission) plus the ctypes binding of the engine
runtime. Importing the package needs no GPU; running a layer does.
"""
from .config import BASELINE_CONFIGS, BLOCK_M, MoEConfig
from .contracts import HipKernelContract, Launch, canonical_json, stable_hash
from .engine import compile_moe_engine, operations, tensor_table
from .profiles import DimensionGuard, ShapeProfile, profile_for, select_profile
from .runtime import ENGINE_SYMBOLS, Engine, LaunchShape, NetraError, Status, manifest_check

__all__ = [
    "BASELINE_CONFIGS", "BLOCK_M", "MoEConfig", "HipKernelContract", "Launch", "canonical_json",
    "stable_hash", "compile_moe_engine", "operations", "tensor_table", "DimensionGuard",
    "ShapeProfile", "profile_for", "select_profile", "ENGINE_SYMBOLS", "Engine", "LaunchShape",
    "NetraError", "Status", "manifest_check",
]
