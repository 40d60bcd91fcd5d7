"""Locations of the in-tree built artefacts."""
from __future__ import annotations

from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent   # netra-kernel_amd/
REPO_ROOT = PKG_ROOT.parent
LIB_DIR = PKG_ROOT / "lib"


def hsaco_path() -> Path:
    return LIB_DIR / "netra_moe_gfx950.hsaco"


def engine_library() -> Path:
    return LIB_DIR / "libnetra_engine.so"


def bridge_library() -> Path:
    return LIB_DIR / "libnetra_moe.so"


def ops_bridge_library() -> Path:
    return LIB_DIR / "libnetra_bridges.so"


def header_paths() -> list[Path]:
    return sorted((REPO_ROOT / "include").glob("*.h"))
