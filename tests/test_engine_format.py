"""Engine directories against the reference's netra-engine-1 format.

tests/golden/engine_format.json holds the reference validator's verdicts on
this build's emitted directories (compiler/netra_compiler/validation.py:22-144,
written by tests/golden/make_engine_format.py in the development container)
and the required-field lists of schemas/netra-engine.schema.json and
schemas/netra-kernel-contract.schema.json. These tests re-emit every case and
check the same conditions against those lists, so a change to the emitter that
the reference would reject fails here without the reference present.
"""
import hashlib
import json
import re
from pathlib import Path

import pytest

import netra_moe as nm
from netra_moe.contracts import stable_hash
from netra_moe.planner import layer_semantics_request

GOLDEN = json.loads((Path(__file__).parent / "golden" / "engine_format.json").read_text())
CASES = {c["case"]: c for c in GOLDEN["cases"]}


def emit(case: str, out: Path) -> Path:
    c = CASES[case]
    kw = dict(c["options"])
    if kw.get("semantics") == "row_major":
        kw["semantics"] = layer_semantics_request(layouts="checkpoint_row_major.v1")
    nm.compile_moe_engine(nm.BASELINE_CONFIGS[c["config"]], out, **kw)
    return out


def variant_matches(contract: dict, variant: dict) -> bool:
    kind = variant["artifact_kind"]
    if kind is not None and contract.get("artifact_kind") != kind:
        return False
    return all(k in contract for k in variant["required"])


def format_errors(d: Path) -> list[str]:
    """The conditions validate_engine_directory and the two schemas impose,
    restated over the golden field lists."""
    err = []
    engine = json.loads((d / "engine.json").read_text())
    for k in set(GOLDEN["engine_required"]) | set(GOLDEN["validator_required"]):
        if k not in engine:
            err.append(f"engine.json lacks {k}")
    for k, v in GOLDEN["engine_const"].items():
        if engine.get(k) != v:
            err.append(f"engine.json {k} != {v!r}")
    if not re.search(GOLDEN["engine_id_pattern"], str(engine.get("engine_id", ""))):
        err.append("engine_id pattern")
    if not isinstance(engine.get("tensor_parallel"), int) or engine["tensor_parallel"] < 1:
        err.append("tensor_parallel")
    if not engine.get("profiles"):
        err.append("profiles empty")
    for rel in engine.get("artifact_files", []):
        if not (d / rel).is_file():
            err.append(f"missing artifact {rel}")
    cs = json.loads((d / "contracts.json").read_text())
    if cs.get("format") != "netra-contract-set-1":
        err.append("contract set format")
    for c in cs.get("contracts", []):
        for k in GOLDEN["contract_required"]:
            if k not in c:
                err.append(f"contract {c.get('id')} lacks {k}")
        if not re.search(GOLDEN["contract_id_pattern"], str(c.get("id", ""))):
            err.append(f"contract id {c.get('id')}")
        if "maturity" in c and c["maturity"] not in GOLDEN["contract_maturity"]:
            err.append(f"contract maturity {c['maturity']}")
        if sum(variant_matches(c, v) for v in GOLDEN["contract_variants"]) != 1:
            err.append(f"contract {c.get('id')} matches other than exactly one schema variant")
        if "launch" in c and any(k not in c["launch"] for k in GOLDEN["contract_launch_required"]):
            err.append("contract launch fields")
        if "workspace" in c and any(k not in c["workspace"] for k in GOLDEN["contract_workspace_required"]):
            err.append("contract workspace fields")
    sym = json.loads((d / "symbols.json").read_text())
    every = sym["selected"] + sym["candidates"]
    if len(every) != len(set(every)):
        err.append("duplicate kernel symbol")
    val = json.loads((d / "validation_plan.json").read_text())
    for cand in val.get("candidates", []):
        src = d / cand["source"]
        if not src.is_file() or cand["symbol"].encode() not in src.read_bytes():
            err.append(f"validation source lacks {cand['symbol']}")
    for op in engine.get("operations", []):
        if op.get("execution") != "kernel":
            continue
        args = op.get("arguments") or []
        if not args or len(args) > 32:
            err.append(f"{op['name']} argument count")
            continue
        spans = sorted((a["offset"], a["offset"] + (8 if a["kind"] == "pointer" else 4)) for a in args)
        if any(lo % min(hi - lo, 8) for lo, hi in spans) or any(a[1] > b[0] for a, b in zip(spans, spans[1:])):
            err.append(f"{op['name']} kernarg offsets")
        if (spans[-1][1] + 7) // 8 * 8 != op.get("kernarg_size"):
            err.append(f"{op['name']} kernarg size")
    return err


def test_golden_verdicts_are_all_valid():
    assert set(GOLDEN["verdicts"]) == set(CASES)
    bad = {c: v for c, v in GOLDEN["verdicts"].items() if not v["valid"]}
    assert not bad, bad
    # the five BASELINE configs and the fallback-only engine are among the cases
    assert set(nm.BASELINE_CONFIGS) <= set(CASES)
    fb = GOLDEN["verdicts"]["decode_t64.fallback_row_major"]["result"]
    assert fb["kernel_operations"] == 0 and fb["fallback_operations"] == 1


@pytest.mark.parametrize("case", sorted(CASES))
def test_emitted_directory_meets_the_reference_format(case, tmp_path):
    d = emit(case, tmp_path / case)
    assert format_errors(d) == []
    engine = json.loads((d / "engine.json").read_text())
    assert engine["artifact_files"] == ["contracts.json", "graph.json", "graph_recipe.json", "memory_plan.json",
                                        "layout_plan.json", "symbols.json", "validation_plan.json", "explain.json"]
    # engine_id is the hash of every other field (compiler/netra_compiler/engine.py:482)
    rest = {k: v for k, v in engine.items() if k != "engine_id"}
    assert engine["engine_id"] == "ne_" + stable_hash(rest)[:24]
    kernels = [op for op in engine["operations"] if op["execution"] == "kernel"]
    assert engine["kernel_symbols"] == sorted({op["kernel_symbol"] for op in kernels})
    ids = {c["id"] for c in json.loads((d / "contracts.json").read_text())["contracts"]}
    assert {op["contract_id"] for op in engine["operations"]} == ids
    assert nm.manifest_check(d)[0] == nm.Status.OK
    if kernels:
        sha = hashlib.sha256((d / kernels[0]["hsaco"]).read_bytes()).hexdigest()
        assert all(op["hsaco_sha256"] == sha for op in kernels)


def test_format_check_rejects_what_the_reference_rejects(tmp_path):
    """Each plausible emission mistake trips the restated check."""
    d = emit("decode_t64", tmp_path / "e")
    good = (d / "engine.json").read_text()

    def broken(mutate) -> list[str]:
        doc = json.loads(good)
        mutate(doc)
        (d / "engine.json").write_text(json.dumps(doc))
        try:
            return format_errors(d)
        finally:
            (d / "engine.json").write_text(good)

    assert broken(lambda e: e.pop("memory_plan"))
    assert broken(lambda e: e.update(engine_id="ne_123"))
    assert broken(lambda e: e["artifact_files"].append("missing.json"))
    assert broken(lambda e: e["operations"][1].update(kernarg_size=e["operations"][1]["kernarg_size"] + 8))
    assert broken(lambda e: e["operations"][0]["arguments"][1].update(offset=4))
    cs = (d / "contracts.json").read_text()
    doc = json.loads(cs)
    doc["contracts"][0].pop("fallback")
    (d / "contracts.json").write_text(json.dumps(doc))
    assert format_errors(d)
    doc = json.loads(cs)
    doc["contracts"][0]["artifact_kind"] = "framework_fallback"  # now two schema variants match
    (d / "contracts.json").write_text(json.dumps(doc))
    assert format_errors(d)
