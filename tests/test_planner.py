"""Tactic catalog, planner fallback, explain.json and the packed workspace (no
GPU). Mirrors the reference compiler's planner checks: a request whose
dimensions match but whose layouts semantic differs must fall back, with the
reason recorded per candidate (tests/compiler/test_kernel_library.py:93-114);
the workspace shares bytes between temporaries whose lifetimes do not overlap
(compiler/netra_compiler/memory.py:56-112)."""
import json
from dataclasses import replace

import pytest

import netra_moe as nm
from netra_moe import planner
from netra_moe.engine import PERSISTENT_TENSORS, operations, resolve_front, resolve_path, tensor_table

CONFIGS = nm.BASELINE_CONFIGS


@pytest.fixture
def hsaco(tmp_path):
    f = tmp_path / "code.hsaco"
    f.write_bytes(b"\x7fELF stand-in code object for host-only emission")
    return f


@pytest.mark.parametrize("name,expected", [
    ("decode_t1", "gfx950.moe_fp8.fused_decode.exact"),
    ("decode_t64", "gfx950.moe_fp8.fused_decode.exact"),
    ("verify_t512", "gfx950.moe_fp8.tile.screen"),
    ("prefill_t4096", "gfx950.moe_fp8.tile.screen"),
])
def test_default_request_takes_the_best_ranked_tactic(name, expected):
    plan = planner.plan_layer(planner.layer_request(CONFIGS[name]))
    assert plan.execution == "kernel" and plan.selected.name == expected
    first = plan.candidates[0]
    assert first == {"tactic": expected, "selected": True, "reasons": []}
    assert sum(c["selected"] for c in plan.candidates) == 1


def test_auto_resolution_follows_the_planner():
    for cfg in CONFIGS.values():
        sel = planner.plan_layer(planner.layer_request(cfg)).selected
        assert (resolve_path(cfg), resolve_front(cfg)) == (sel.path, sel.front)


def test_row_major_layouts_fall_back_with_the_reason(tmp_path, hsaco):
    cfg = CONFIGS["decode_t64"]
    out = tmp_path / "engine"
    sem = planner.layer_semantics_request(layouts="checkpoint_row_major.v1")
    recipe = nm.compile_moe_engine(cfg, out, hsaco=hsaco, semantics=sem)
    assert recipe["execution"] == "fallback" and recipe["operations"] == []
    engine = json.loads((out / "engine.json").read_text())
    kinds = [op["execution"] for op in engine["operations"]]
    assert kinds.count("kernel") == 0 and kinds.count("fallback") == 1
    assert engine["fallbacks"] == {"moe.layer": "framework"} and engine["workspace_bytes"] == 0
    explanation = json.loads((out / "explain.json").read_text())
    selected = explanation["operations"][0]
    assert selected["selected"] is None and selected["execution"] == "fallback"
    assert all("layouts semantic mismatch" in c["reasons"] for c in selected["candidates"])
    # the native parser accepts the fallback-only engine
    assert nm.manifest_check(out)[0] == nm.Status.OK


def test_matching_request_emits_kernels_and_an_explanation(tmp_path, hsaco):
    cfg = CONFIGS["verify_t512"]
    out = tmp_path / "engine"
    nm.compile_moe_engine(cfg, out, hsaco=hsaco)
    engine = json.loads((out / "engine.json").read_text())
    assert engine["selected_tactics"] == ["gfx950.moe_fp8.tile.screen"]
    assert {op["execution"] for op in engine["operations"]} == {"kernel"}
    assert all(op["tactic"] == "gfx950.moe_fp8.tile.screen" for op in engine["operations"])
    explanation = json.loads((out / "explain.json").read_text())["operations"][0]
    assert explanation["selected"] == "gfx950.moe_fp8.tile.screen"
    rejected = {c["tactic"]: c["reasons"] for c in explanation["candidates"] if not c["selected"]}
    assert "T mismatch" in rejected["gfx950.moe_fp8.fused_decode.exact"]
    assert "T mismatch" in rejected["gfx950.moe_fp8.stream.exact"]
    assert rejected["gfx950.moe_fp8.tile.exact"] == []  # compatible, ranked lower


def test_numerical_and_path_requests_steer_the_choice():
    cfg = CONFIGS["prefill_t4096"]
    from netra_moe.engine import NUMERICS
    exact = planner.plan_layer(planner.layer_request(
        cfg, semantics=planner.layer_semantics_request(numerical=NUMERICS["exact"])))
    assert exact.selected.name == "gfx950.moe_fp8.tile.exact"
    screen = next(c for c in exact.candidates if c["tactic"] == "gfx950.moe_fp8.tile.screen")
    assert screen["reasons"] == ["numerical semantic mismatch"]
    forced = planner.plan_layer(planner.layer_request(CONFIGS["decode_t64"], path="stream"))
    assert forced.selected.name == "gfx950.moe_fp8.stream.exact"
    fused = next(c for c in forced.candidates if c["tactic"].startswith("gfx950.moe_fp8.fused"))
    assert "gemm-path mismatch" in fused["reasons"]


def test_unsupported_shapes_and_fields_are_named():
    cfg = replace(CONFIGS["decode_t64"], H=3072)
    plan = planner.plan_layer(planner.layer_request(cfg))
    assert plan.execution == "fallback"
    assert all("H mismatch" in c["reasons"] for c in plan.candidates)
    req = planner.layer_request(CONFIGS["decode_t64"])
    req["constants"]["BLOCK_N"] = 64
    req["semantics"]["scales"] = "per_tensor"
    req["target"] = "gfx942"
    why = planner.catalog()[0].rejection_reasons(req)
    assert {"target mismatch", "undeclared semantic field scales",
            "undeclared compile-time constant BLOCK_N"} <= set(why)
    del req["constants"]
    assert "compile-time constants missing" in planner.catalog()[0].rejection_reasons(req)


def test_buffer_offset_limit_names_the_bound():
    big = replace(CONFIGS["prefill_t4096"], T=1 << 19)  # bf16 x of 2 GiB
    plan = planner.plan_layer(planner.layer_request(big))
    screen = next(c for c in plan.candidates if c["tactic"] == "gfx950.moe_fp8.tile.screen")
    assert screen["reasons"] == [f"x_bytes exceeds {(1 << 31) - 1}"]
    assert plan.selected.name == "gfx950.moe_fp8.tile.exact"


def test_maturity_gates_experimental_tactics():
    exp = replace(planner.catalog()[0], name="gfx950.trial", maturity="experiment", rank=1)
    req = planner.layer_request(CONFIGS["decode_t1"])
    assert "experimental tactics are disabled" in exp.rejection_reasons(req)
    assert planner.plan_layer(req, tactics=(exp,)).execution == "fallback"
    assert planner.plan_layer(req, tactics=(exp,), allow_experimental=True).selected is exp
    dead = replace(exp, maturity="rejected")
    assert "maturity is rejected" in dead.rejection_reasons(req, allow_experimental=True)
    tie = replace(exp, name="gfx950.trial2")
    with pytest.raises(ValueError, match="ambiguous"):
        planner.plan_layer(req, tactics=(exp, tie), allow_experimental=True)


PATHS = [(n, p) for n in ("decode_t1", "decode_t64", "verify_t512", "prefill_t4096")
         for p in ("fused", "stream", "tile") if p != "fused" or CONFIGS[n].T <= 64]


@pytest.mark.parametrize("name,path", PATHS)
def test_packed_workspace_never_overlaps_live_tensors(name, path):
    cfg = CONFIGS[name]
    front = resolve_front(cfg, path)
    ops = operations(cfg, path, front)
    sizes = {n: s.nbytes for n, s in tensor_table(cfg, path, front).items() if s.role == "temporary"}
    top, slots = planner.pack_workspace(sizes, ops, set(PERSISTENT_TENSORS))
    by = {s.name: s for s in slots}
    assert set(by) == set(sizes)
    for s in slots:
        assert s.offset % 256 == 0 and s.size >= sizes[s.name] and s.offset + s.size <= top
    for a in slots:
        for b in slots:
            if a.name >= b.name:
                continue
            alive = not (a.last_use < b.first_use or b.last_use < a.first_use) or a.persistent or b.persistent
            apart = a.offset + a.size <= b.offset or b.offset + b.size <= a.offset
            assert apart or not alive, (a, b)
    # every pointer an operation takes lives over that operation
    for i, op in enumerate(ops):
        for arg in op["args"]:
            if isinstance(arg, str) and arg in by:
                assert by[arg].first_use <= i <= by[arg].last_use
    unpacked = sum((v + 255) // 256 * 256 for v in sizes.values())
    assert top <= unpacked
    if path == "tile":  # prefill: the big temporaries share bytes
        assert top < unpacked


def test_packer_refuses_state_it_was_not_told_about():
    ops = [dict(args=["a", "b"], reads=["a"], writes=["b"])]
    with pytest.raises(ValueError, match="read before"):
        planner.pack_workspace({"a": 512, "b": 512}, ops, set())
    top, slots = planner.pack_workspace({"a": 512, "b": 512}, ops, {"a"})
    assert top == 1024 and {s.name: s.persistent for s in slots} == {"a": True, "b": False}


def test_disjoint_lifetimes_share_bytes():
    ops = [dict(args=["x", "y"], reads=[], writes=["x", "y"]),
           dict(args=["y", "z"], reads=["y"], writes=["z"]),
           dict(args=["z", "w"], reads=["z"], writes=["w"])]
    top, slots = planner.pack_workspace({"x": 1000, "y": 300, "z": 1000, "w": 256}, ops, set())
    by = {s.name: s for s in slots}
    assert by["x"].offset == by["z"].offset or by["x"].offset == by["w"].offset  # x dies after op 0
    assert top < 1024 + 512 + 1024 + 256
