"""Write tests/golden/engine_format.json: the reference's own verdict on the
engine directories this build emits.

Run in the development container only (it needs the reference checkout, which
the GPU host does not have):

    python tests/golden/make_engine_format.py [/root/reference]

For every case below it compiles this build's engine directory into a
temporary folder and passes it through the reference's
``validate_engine_directory`` (compiler/netra_compiler/validation.py:22-144,
schema checks of schemas/netra-engine.schema.json and
schemas/netra-kernel-contract.schema.json), recording the verdict. It also
records the required-field lists of those two schemas and of the validator, so
the CPU test can re-check freshly emitted directories against them without the
reference. Nothing of the reference is copied: the fixture holds field names
and verdicts.
"""
from __future__ import annotations

import json
import sys
import tempfile
from pathlib import Path

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO / "netra-kernel_amd"))

# (case name, config name, compile_moe_engine keyword arguments)
CASES = (
    ("cpu_small", "cpu_small", {}),
    ("decode_t64", "decode_t64", {}),
    ("decode_t1", "decode_t1", {}),
    ("verify_t512", "verify_t512", {}),
    ("prefill_t4096", "prefill_t4096", {}),
    ("decode_t64.stream", "decode_t64", {"path": "stream"}),
    ("verify_t512.tile_exact", "verify_t512", {"path": "tile", "front": "exact"}),
    ("decode_t64.fallback_row_major", "decode_t64", {"semantics": "row_major"}),
)


def main(reference: Path) -> int:
    sys.path.insert(0, str(reference / "compiler"))
    from netra_compiler.errors import ValidationError
    from netra_compiler.validation import REQUIRED_ENGINE_KEYS, validate_engine_directory

    import netra_moe as nm
    from netra_moe.planner import layer_semantics_request

    engine_schema = json.loads((reference / "schemas" / "netra-engine.schema.json").read_text())
    contract_schema = json.loads((reference / "schemas" / "netra-kernel-contract.schema.json").read_text())
    variants = []
    for v in contract_schema["oneOf"]:
        kind = v.get("properties", {}).get("artifact_kind", {}).get("const")
        variants.append({"required": sorted(v["required"]), "artifact_kind": kind})
    verdicts = {}
    with tempfile.TemporaryDirectory() as tmp:
        for case, cfg_name, kw in CASES:
            kw = dict(kw)
            if kw.get("semantics") == "row_major":
                kw["semantics"] = layer_semantics_request(layouts="checkpoint_row_major.v1")
            out = Path(tmp) / case
            nm.compile_moe_engine(nm.BASELINE_CONFIGS[cfg_name], out, **kw)
            try:
                res = validate_engine_directory(out, library_root=reference)
                verdicts[case] = {"valid": True, "result": res}
            except ValidationError as exc:
                verdicts[case] = {"valid": False, "error": str(exc)}
            print(f"{case}: {verdicts[case]}")
    doc = {
        "generator": "tests/golden/make_engine_format.py",
        "validator": "compiler/netra_compiler/validation.py:22-144 (validate_engine_directory)",
        "cases": [{"case": c, "config": n, "options": {k: v for k, v in kw.items()}} for c, n, kw in CASES],
        "verdicts": verdicts,
        "engine_required": sorted(engine_schema["required"]),
        "engine_const": {k: v["const"] for k, v in engine_schema["properties"].items() if "const" in v},
        "engine_id_pattern": engine_schema["properties"]["engine_id"]["pattern"],
        "validator_required": sorted(REQUIRED_ENGINE_KEYS),
        "contract_required": sorted(contract_schema["required"]),
        "contract_id_pattern": contract_schema["properties"]["id"]["pattern"],
        "contract_maturity": contract_schema["properties"]["maturity"]["enum"],
        "contract_variants": variants,
        "contract_launch_required": sorted(contract_schema["$defs"]["launch"]["required"]),
        "contract_workspace_required": sorted(contract_schema["$defs"]["workspace"]["required"]),
    }
    dst = Path(__file__).resolve().parent / "engine_format.json"
    dst.write_text(json.dumps(doc, indent=1, sort_keys=True) + "\n")
    print(f"wrote {dst.relative_to(REPO)}")
    return 0 if all(v["valid"] for v in verdicts.values()) else 1


if __name__ == "__main__":
    sys.exit(main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")))
