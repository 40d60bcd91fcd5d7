"""Static check of the built gfx950 code object for one hazard the compiler
cannot see: a vector-memory instruction (buffer/global/flat) that reads an
SGPR fewer than five wait states after a VALU instruction wrote it
(v_readfirstlane, v_readlane, VALU compares and carry-outs). The hardware
needs those wait states; the compiler inserts them for its own instructions
but not around inline assembly, and several kernels issue their copies from
inline assembly. A missed case reads a stale resource descriptor or offset,
which can address memory outside every buffer.

Runs on the CPU over the disassembly of this repository's own build (the
ROCm llvm tools); skipped when the code object or the tools are absent.
"""
from __future__ import annotations

import re
import subprocess
import tempfile
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
HSACO = REPO / "netra-kernel_amd" / "lib" / "netra_moe_gfx950.hsaco"
LLVM = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
WAIT_STATES = 5

_SREG = re.compile(r"\bs\[(\d+):(\d+)\]|\bs(\d+)\b|\b(vcc|exec|m0)\b")
_VMEM = re.compile(r"^(buffer_|global_|flat_)")


def sgprs(text: str) -> set:
    out: set = set()
    for m in _SREG.finditer(text):
        if m.group(4):
            out.add(m.group(4))
        elif m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def valu_sgpr_writes(op: str, operands: list[str]) -> set:
    """SGPRs (and vcc/exec) a VALU instruction writes."""
    if op.startswith(("v_readfirstlane", "v_readlane")):
        return sgprs(operands[0])
    if op.startswith("v_cmpx"):
        return {"exec"} | (sgprs(operands[0]) if op.endswith("_e64") else set())
    if op.startswith("v_cmp"):
        return sgprs(operands[0]) if op.endswith("_e64") else {"vcc"}
    carry = re.match(r"v_(add|sub|subrev|addc|subb|subbrev)_co_|v_(addc|subb|subbrev)_|v_mad_[iu]64_|v_div_scale", op)
    if carry and len(operands) > 1:
        if op.endswith("_e32"):
            return {"vcc"}
        return sgprs(operands[1])
    return set()


def hazards(lines: list[str]) -> list[str]:
    found, recent = [], []  # recent: [wait states since, sgprs written]
    for text in lines:
        text = text.split("//")[0].strip()
        if not text or text.endswith(":"):
            continue
        op, _, rest = text.partition(" ")
        operands = [o.strip() for o in rest.split(",")]
        if _VMEM.match(op):
            read = sgprs(rest)
            for dist, written in recent:
                if read & written:
                    found.append(f"{text}  (VALU wrote {sorted(map(str, read & written))} {dist} wait states before)")
        step = int(rest, 0) + 1 if op == "s_nop" else 1  # s_nop N is N + 1 wait states
        recent = [(d + step, w) for d, w in recent if d + step < WAIT_STATES]
        if op.startswith("v_"):
            written = valu_sgpr_writes(op, operands)
            if written:
                recent.append((0, written))
    return found


def disassembly() -> dict[str, list[str]]:
    bundler, objdump = LLVM / "clang-offload-bundler", LLVM / "llvm-objdump"
    if not HSACO.exists() or not bundler.exists() or not objdump.exists():
        pytest.skip("built code object or ROCm llvm tools not present")
    with tempfile.TemporaryDirectory() as tmp:
        out = Path(tmp) / "gfx950.co"
        subprocess.run([str(bundler), "--unbundle", "--type=o", f"--input={HSACO}", f"--targets={TARGET}",
                        f"--output={out}"], check=True, capture_output=True)
        text = subprocess.run([str(objdump), "-d", "--mcpu=gfx950", str(out)], check=True,
                              capture_output=True, text=True).stdout
    funcs: dict[str, list[str]] = {}
    name = None
    for line in text.splitlines():
        m = re.match(r"^[0-9a-f]+ <([\w.]+)>:", line)
        if m:
            name = m.group(1)
            funcs[name] = []
        elif name:
            funcs[name].append(line)
    return funcs


def test_checker_flags_the_hazard_and_accepts_wait_states():
    bad = ["v_readlane_b32 s43, v209, 4", "buffer_store_dword v66, v67, s[40:43], 0 offen"]
    assert len(hazards(bad)) == 1
    ok = ["v_readlane_b32 s43, v209, 4", "s_nop 4", "buffer_store_dword v66, v67, s[40:43], 0 offen"]
    assert hazards(ok) == []
    assert hazards(["v_cmp_lt_u32_e64 s[4:5], v1, v2", "s_nop 3", "global_load_dword v1, v2, s[4:5]"])
    assert hazards(["v_add_co_u32_e64 v1, s[6:7], v2, v3", "buffer_load_dword v1, v2, s[4:7], 0 offen"])


def test_no_valu_sgpr_to_vmem_hazard_in_any_kernel():
    funcs = disassembly()
    kernels = {k: v for k, v in funcs.items() if k.startswith("netra_moe_")}
    assert kernels, "no netra_moe_ kernels in the code object"
    report = {k: h for k, v in kernels.items() if (h := hazards(v))}
    assert not report, "\n".join(f"{k}: {h[0]}" for k, h in report.items())
