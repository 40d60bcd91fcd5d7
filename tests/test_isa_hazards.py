"""Static checks of the built gfx950 code object for what the compiler
cannot see around inline assembly:

* a vector-memory instruction (buffer/global/flat) that reads an SGPR fewer
  than five wait states after a VALU instruction wrote it (v_readfirstlane,
  v_readlane, VALU compares and carry-outs). The hardware needs those wait
  states; the compiler inserts them for its own instructions but not around
  inline assembly, and several kernels issue their copies from inline
  assembly. A missed case reads a stale resource descriptor or offset, which
  can address memory outside every buffer.
* the LDS-ring gate/up kernels wait for "this step's copies landed" with
  s_waitcnt vmcnt(7): correct only while the seven buffer-to-LDS copies a wave
  issues per 128-K step are the only vector-memory operations in flight in
  the K loop. If the compiler ever turned the per-step weight-scale loads
  (uniform addresses, scalar loads today) into vector loads, the count would
  be off and a step would read a stage before its data arrived.

Runs on the CPU over the disassembly of this repository's own build (the
ROCm llvm tools): the engine's code object and the gfx950 device code
embedded in libnetra_moe.so (a separate compile of the kernels, which the
allocation-free prefill entry point launches); skipped when an artefact or the
tools are absent.
"""
from __future__ import annotations

import re
import subprocess
import tempfile
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
HSACO = REPO / "netra-kernel_amd" / "lib" / "netra_moe_gfx950.hsaco"
LIB_SO = REPO / "netra-kernel_amd" / "lib" / "libnetra_moe.so"
ARTEFACTS = {"hsaco": HSACO, "libnetra_moe.so": LIB_SO}
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


_CACHE: dict[str, dict[str, list[str]]] = {}


def disassembly(artefact: str = "hsaco") -> dict[str, list[str]]:
    """Per-function disassembly of the gfx950 code in one built artefact: the
    offload bundle itself (hsaco) or the .hip_fatbin section of a shared
    library."""
    if artefact in _CACHE:
        return _CACHE[artefact]
    src = ARTEFACTS[artefact]
    bundler, objdump, objcopy = LLVM / "clang-offload-bundler", LLVM / "llvm-objdump", LLVM / "llvm-objcopy"
    if not src.exists() or not bundler.exists() or not objdump.exists() or not objcopy.exists():
        pytest.skip("built artefact or ROCm llvm tools not present")
    with tempfile.TemporaryDirectory() as tmp:
        bundle = src
        if src.suffix == ".so":
            bundle = Path(tmp) / "fatbin"
            subprocess.run([str(objcopy), f"--dump-section=.hip_fatbin={bundle}", str(src), str(Path(tmp) / "so")],
                           check=True, capture_output=True)
        out = Path(tmp) / "gfx950.co"
        subprocess.run([str(bundler), "--unbundle", "--type=o", f"--input={bundle}", f"--targets={TARGET}",
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
    _CACHE[artefact] = funcs
    return funcs


def test_checker_flags_the_hazard_and_accepts_wait_states():
    bad = ["v_readlane_b32 s43, v209, 4", "buffer_store_dword v66, v67, s[40:43], 0 offen"]
    assert len(hazards(bad)) == 1
    ok = ["v_readlane_b32 s43, v209, 4", "s_nop 4", "buffer_store_dword v66, v67, s[40:43], 0 offen"]
    assert hazards(ok) == []
    assert hazards(["v_cmp_lt_u32_e64 s[4:5], v1, v2", "s_nop 3", "global_load_dword v1, v2, s[4:5]"])
    assert hazards(["v_add_co_u32_e64 v1, s[6:7], v2, v3", "buffer_load_dword v1, v2, s[4:7], 0 offen"])


@pytest.mark.parametrize("artefact", sorted(ARTEFACTS))
def test_no_valu_sgpr_to_vmem_hazard_in_any_kernel(artefact):
    funcs = disassembly(artefact)
    kernels = {k: v for k, v in funcs.items() if k.startswith("netra_moe_")}
    assert kernels, f"no netra_moe_ kernels in {artefact}"
    report = {k: h for k, v in kernels.items() if (h := hazards(v))}
    assert not report, "\n".join(f"{k}: {h[0]}" for k, h in report.items())


# vmcnt waits an LDS-ring kernel family may use inside its ring: 0 or the
# copies of one step (kCopiesPerWave in moe_gemm_lds.hip, kCopies in
# route_screen)
RING_WAITS = {"netra_moe_gate_up_lds_": {0, 6, 7}, "netra_moe_route_screen_": {0, 8, 16}}
KCOPIES = 7
_VMCNT = re.compile(r"vmcnt\((\d+)\)")
_VSTORE = re.compile(r"(global|buffer|flat)_store")


def ring_violations(lines: list[str], waits: set[int] | None = None) -> list[str]:
    """Vector-memory accounting of one LDS-ring kernel (instructions in address
    order): between its first and last buffer-to-LDS copy there is no other
    vector-memory load, every vmcnt wait is one of `waits`, and the first wait
    after a vector store is vmcnt(0) (stores may complete before older loads,
    so only a full drain is exact behind one); after the last copy, the first
    other vector-memory instruction comes behind a vmcnt(0)."""
    waits = {0, KCOPIES} if waits is None else waits
    text = [t.split("//")[0].strip() for t in lines]
    text = [t for t in text if t and not t.endswith(":")]
    is_copy = [bool(re.match(r"buffer_load_dword\w*\s.*\blds\b", t)) for t in text]
    copies = [i for i, c in enumerate(is_copy) if c]
    if not copies:
        return ["no buffer-to-LDS copies"]
    first, last = copies[0], copies[-1]
    bad = []
    store_pending = False
    for i in range(first, last + 1):
        t = text[i]
        if _VSTORE.match(t):
            store_pending = True
        elif _VMEM.match(t) and not is_copy[i]:
            bad.append(f"vector-memory op inside the copy ring: {t}")
        m = _VMCNT.search(t) if t.startswith("s_waitcnt") else None
        if m and int(m.group(1)) not in waits:
            bad.append(f"unexpected wait inside the copy ring: {t}")
        if m and store_pending:
            if int(m.group(1)) != 0:
                bad.append(f"partial wait behind a store inside the copy ring: {t}")
            store_pending = False
    drained = False
    for t in text[last + 1:]:
        m = _VMCNT.search(t) if t.startswith("s_waitcnt") else None
        if m:
            if store_pending and int(m.group(1)) != 0:
                bad.append(f"partial wait behind a store after the copy ring: {t}")
            store_pending = False
            if int(m.group(1)) == 0:
                drained = True
        if _VSTORE.match(t):  # stores may overlap copies still in flight; a drain must follow them
            store_pending = True
            continue
        if _VMEM.match(t):
            if not drained:
                bad.append(f"vector-memory op before the ring drains: {t}")
            break
    return bad


def test_ring_checker_flags_a_foreign_load():
    ring = ["buffer_load_dwordx4 v1, s[4:7], s1 offen lds", "s_waitcnt vmcnt(7)",
            "buffer_load_dwordx4 v2, s[4:7], s1 offen lds", "s_waitcnt vmcnt(0)",
            "global_store_dword v[0:1], v3, off"]
    assert ring_violations(ring) == []
    foreign = ring[:2] + ["global_load_dword v5, v[6:7], off"] + ring[2:]
    assert any("inside the copy ring" in v for v in ring_violations(foreign))
    early = ring[:3] + ["global_load_dword v4, v[0:1], off"]
    assert any("before the ring drains" in v for v in ring_violations(early))
    overlap = ring[:3] + ["global_store_dword v[0:1], v3, off", "s_waitcnt vmcnt(7)"]
    assert any("behind a store" in v for v in ring_violations(overlap))
    assert ring_violations(ring[:1] + ["s_waitcnt vmcnt(5)"] + ring[2:])
    stored = ring[:2] + ["global_store_dwordx4 v[0:1], v[4:7], off", "s_waitcnt vmcnt(7)"] + ring[2:]
    assert any("behind a store" in v for v in ring_violations(stored))
    drained = ring[:2] + ["global_store_dwordx4 v[0:1], v[4:7], off", "s_waitcnt vmcnt(0)"] + ring[2:]
    assert ring_violations(drained) == []


@pytest.mark.parametrize("artefact", sorted(ARTEFACTS))
@pytest.mark.parametrize("prefix", sorted(RING_WAITS))
def test_lds_ring_kernels_issue_only_their_copies(prefix, artefact):
    funcs = disassembly(artefact)
    ring = {k: v for k, v in funcs.items() if k.startswith(prefix)}
    assert ring, f"no {prefix} kernels in {artefact}"
    report = {k: b for k, v in ring.items() if (b := ring_violations(v, RING_WAITS[prefix]))}
    assert not report, "\n".join(f"{k}: {b[0]}" for k, b in report.items())
