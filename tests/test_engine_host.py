"""Host-side boundary tests (no GPU): the C-ABI libraries load and export every
declared entry point, the ctypes structs match the C header's layout, the
engine manifest contract is enforced by the native parser, engine emission is
deterministic, and profiles select/refuse shapes the way the reference's
planner does (compiler/netra_compiler/profiles.py:70-77)."""
import ctypes
import json
import re
import shutil
import subprocess
from pathlib import Path

import pytest

import netra_moe as nm
from netra_moe import paths, runtime
from netra_moe.engine import op_names, operations

REPO = Path(__file__).resolve().parent.parent


def declared(header: Path) -> list[str]:
    text = header.read_text()
    return sorted(set(re.findall(r"^[A-Za-z_][\w \*]*?\b(netra_\w+)\(", text, flags=re.M)))


def test_headers_declare_the_reference_engine_abi():
    names = declared(REPO / "include" / "netra_engine.h")
    ref = ["netra_engine_create", "netra_engine_profile_count", "netra_engine_query_profile",
           "netra_engine_bind", "netra_engine_finalize_bindings", "netra_engine_prepare_profile",
           "netra_engine_launch", "netra_engine_launch_operation", "netra_engine_launch_operation_bound",
           "netra_engine_last_error", "netra_engine_destroy"]
    assert set(ref) <= set(names)
    assert set(names) == set(runtime.ENGINE_SYMBOLS)


LIBRARIES = {"engine": paths.engine_library, "bridge": paths.bridge_library, "ops": paths.ops_bridge_library}


@pytest.mark.parametrize("header,lib", [("netra_engine.h", "engine"), ("netra_moe.h", "bridge"),
                                        ("netra_qwen36_bridges.h", "ops")])
def test_libraries_load_and_export_every_declared_symbol(header, lib):
    path = LIBRARIES[lib]()
    dll = ctypes.CDLL(str(path))
    for name in declared(REPO / "include" / header):
        assert hasattr(dll, name), f"{path.name} does not export {name}"


def test_ctypes_structs_match_the_c_header(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(r"""
#include <stdio.h>
#include <stddef.h>
#include "netra_engine.h"
int main(void) {
  printf("%zu %zu %zu %zu\n", sizeof(netra_engine_options_t), sizeof(netra_profile_info_t),
         sizeof(netra_launch_shape_t), sizeof(netra_pointer_binding_t));
  printf("%zu %zu %zu\n", offsetof(netra_profile_info_t, min_sequence),
         offsetof(netra_profile_info_t, workspace_bytes), offsetof(netra_profile_info_t, requires_fallback));
  printf("%d %d %d\n", NETRA_STATUS_BINDING, NETRA_STATUS_BUSY, NETRA_STATUS_FALLBACK_REQUIRED);
  return 0;
}
""")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-D__HIP_PLATFORM_AMD__", f"-I{REPO / 'include'}", "-I/opt/rocm/include",
                    str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    sizes = [int(v) for v in out[0].split()]
    assert sizes == [ctypes.sizeof(runtime.EngineOptions), ctypes.sizeof(runtime.ProfileInfo),
                     ctypes.sizeof(runtime.LaunchShape), ctypes.sizeof(runtime.PointerBinding)]
    offs = [int(v) for v in out[1].split()]
    assert offs == [runtime.ProfileInfo.min_sequence.offset, runtime.ProfileInfo.workspace_bytes.offset,
                    runtime.ProfileInfo.requires_fallback.offset]
    assert [int(v) for v in out[2].split()] == [runtime.Status.BINDING, runtime.Status.BUSY,
                                               runtime.Status.FALLBACK_REQUIRED]


@pytest.fixture()
def engine_dir(tmp_path):
    cfg = nm.BASELINE_CONFIGS["decode_t64"]
    d = tmp_path / "eng"
    nm.compile_moe_engine(cfg, d)
    return d


def test_emitted_engine_passes_the_native_manifest_check(engine_dir):
    st, msg = nm.manifest_check(engine_dir)
    assert st == nm.Status.OK, msg
    doc = json.loads((engine_dir / "engine.json").read_text())
    assert [op["name"] for op in doc["operations"]] == [f"moe.{n}" for n in op_names(nm.BASELINE_CONFIGS["decode_t64"])]
    assert op_names(nm.BASELINE_CONFIGS["decode_t64"]) == ("route", "gate_up", "combine")  # down per tile in gate/up
    wide17 = nm.MoEConfig("wide17", T=17, H=2048, E=256, K=8, I=512, S=1, seed=1)
    assert op_names(wide17) == ("route", "gate_up", "down", "combine")
    assert op_names(nm.BASELINE_CONFIGS["decode_t1"]) == ("route", "gate_up", "down")
    assert op_names(nm.BASELINE_CONFIGS["decode_t64"], path="stream") == ("route", "sort", "gate_up", "down", "combine")


def _corrupt(engine_dir: Path, mutate) -> tuple:
    doc = json.loads((engine_dir / "engine.json").read_text())
    mutate(doc)
    (engine_dir / "engine.json").write_text(json.dumps(doc))
    return nm.manifest_check(engine_dir)


@pytest.mark.parametrize("mutate,needle", [
    (lambda d: d.update(format_version="netra-engine-0"), "format_version"),
    (lambda d: d.update(target="gfx942"), "target"),
    (lambda d: d.update(wave_size=32), "wave_size"),
    (lambda d: d["required_rocm"].update(code_object_version=5), "code object"),
    (lambda d: d["required_rocm"].update(minimum="7"), "MAJOR.MINOR"),
    (lambda d: d["operations"][0].update(hsaco="hsaco/../engine.json"), "hsaco"),
    (lambda d: d["operations"][0].update(hsaco="/abs/x.hsaco"), "hsaco"),
    (lambda d: d["operations"][0]["launch"].update(grid=[0, 1, 1]), "nonzero"),
    (lambda d: d["operations"][0]["launch"].update(block=[2048, 1, 1]), "1024"),
    (lambda d: d["operations"][-1].update(launch={**d["operations"][-1]["launch"], "dynamic_lds_bytes": 200000}), "LDS"),
    (lambda d: d["operations"][0]["arguments"].append({"kind": "pointer", "source": "workspace",
                                                       "workspace_offset": d["workspace_bytes"]}), "workspace"),
    (lambda d: d["operations"][0]["arguments"].extend([{"kind": "u32_constant", "value": 1}] * 40), "32"),
    (lambda d: d["operations"][0]["arguments"].append({"kind": "f64_constant", "value": 1}), "kind"),
    (lambda d: d["profiles"][0]["guards"]["m"].update(min=9, max=3), "min > max"),
])
def test_manifest_violations_are_refused(engine_dir, mutate, needle):
    st, msg = _corrupt(engine_dir, mutate)
    assert st == nm.Status.MANIFEST
    assert needle.lower() in msg.lower(), msg


def test_manifest_parser_rejects_malformed_json(engine_dir):
    (engine_dir / "engine.json").write_text('{"a": 1, "a": 2}')
    st, msg = nm.manifest_check(engine_dir)
    assert st == nm.Status.MANIFEST and "duplicate" in msg
    (engine_dir / "engine.json").write_text('{"a": [1, 2')
    assert nm.manifest_check(engine_dir)[0] == nm.Status.MANIFEST
    shutil.rmtree(engine_dir)
    assert nm.manifest_check(engine_dir)[0] == nm.Status.IO


def test_engine_emission_is_deterministic_and_contract_ids_track_shape(tmp_path):
    cfg = nm.BASELINE_CONFIGS["verify_t512"]
    a, b = tmp_path / "a", tmp_path / "b"
    nm.compile_moe_engine(cfg, a)
    nm.compile_moe_engine(cfg, b)
    for f in ("engine.json", "contracts.json", "graph_recipe.json", "memory_plan.json"):
        assert (a / f).read_bytes() == (b / f).read_bytes()
    ids_a = [c["id"] for c in json.loads((a / "contracts.json").read_text())["contracts"]]
    c2 = nm.BASELINE_CONFIGS["prefill_t4096"]
    nm.compile_moe_engine(c2, tmp_path / "c")
    ids_c = [c["id"] for c in json.loads((tmp_path / "c" / "contracts.json").read_text())["contracts"]]
    assert all(i.startswith("nk_") and len(i) == 27 for i in ids_a)
    assert len(set(ids_a) & set(ids_c)) == 0


def test_every_emitted_kernel_symbol_is_in_the_code_object():
    blob = paths.hsaco_path().read_bytes()
    for cfg in nm.BASELINE_CONFIGS.values():
        for path, front in (("stream", "exact"), ("tile", "exact"), ("tile", "auto")):
            for op in operations(cfg, path, front):
                assert op["symbol"].encode() in blob, op["symbol"]


def test_prefill_engines_use_the_screen_front_end(tmp_path):
    cfg = nm.BASELINE_CONFIGS["prefill_t4096"]
    nm.compile_moe_engine(cfg, tmp_path / "p")
    doc = json.loads((tmp_path / "p" / "engine.json").read_text())
    assert doc["front_end"] == "screen" and doc["gemm_path"] == "tile"
    assert [op["name"] for op in doc["operations"]] == [f"moe.{n}" for n in op_names(cfg)]
    assert op_names(cfg) == ("route_screen", "route_select", "sort_route", "gate_up", "down", "combine")
    assert nm.manifest_check(tmp_path / "p")[0] == nm.Status.OK
    screen, select = doc["operations"][0], doc["operations"][1]
    assert screen["launch"]["grid"] == [32, 2, 4]  # 4096 / 128 tokens x 256 / 128 expert rows x 4 K splits
    # one token per wave, 8-wave workgroups at T=4096
    assert select["launch"]["grid"] == [512, 1, 1] and select["launch"]["block"] == [512, 1, 1]
    assert select["launch"]["lds_bytes"] <= 160 * 1024
    sort = doc["operations"][2]
    assert sort["launch"]["grid"] == [257, 1, 1]  # one workgroup per expert (256 routed + shared)
    gate_up = doc["operations"][3]
    assert gate_up["kernel_symbol"] == "netra_moe_gate_up_lds_h2048_gfx950"
    assert gate_up["launch"]["block"] == [512, 1, 1] and gate_up["launch"]["lds_bytes"] <= 160 * 1024


@pytest.mark.parametrize("T,H,E,shape", [
    (4096, 2048, 256, (8, 1)), (2048, 2048, 256, (8, 1)), (1024, 2048, 256, (8, 2)), (512, 2048, 256, (8, 4)),
    (300, 2048, 256, (8, 4)), (512, 1024, 256, (8, 2)), (512, 512, 256, (4, 1)), (768, 2048, 384, (8, 2)),
])
def test_route_select_waves_per_token(T, H, E, shape):
    """Waves per token: the most of 1, 2, 4 that keeps T * WPT <= 2048 and
    WPT <= H / 512; the kernel symbol, block, grid and the per-workgroup list
    tensors follow from (W, WPT)."""
    from netra_moe.config import MoEConfig
    from netra_moe.engine import screen_groups, screen_tokens, screen_waves, screen_waves_per_token, tensor_table
    cfg = MoEConfig(f"wpt_t{T}_h{H}_e{E}", T=T, H=H, E=E, K=8, I=512, S=1, seed=1)
    assert (screen_waves(cfg), screen_waves_per_token(cfg)) == shape
    W, WPT = shape
    sel = next(o for o in operations(cfg, "tile", "screen") if o["name"] == "moe.route_select")
    emax = 256 if E <= 256 else 512
    assert sel["symbol"] == f"netra_moe_route_select_h{H}_e{emax}_w{W}x{WPT}_gfx950"
    assert sel["block"] == (64 * W, 1, 1) and sel["grid"] == (screen_groups(cfg), 1, 1)
    assert screen_tokens(cfg) == W // WPT and screen_groups(cfg) == -(-T // (W // WPT))
    tt = tensor_table(cfg, "tile", "screen")
    assert tt["route_hist"].shape == (screen_groups(cfg), cfg.Etot + 1)
    assert tt["route_bucket"].shape == (screen_groups(cfg), screen_tokens(cfg) * cfg.Ktot)
    assert tt["route_slices"].shape == (cfg.Etot, 8)
    sort = next(o for o in operations(cfg, "tile", "screen") if o["name"] == "moe.sort_route")
    assert sort["grid"] == (cfg.Etot, 1, 1)  # the kernel's unused-block stride assumes exactly Etot


def test_profiles_select_exact_shapes_and_refuse_neighbours():
    p64 = nm.profile_for(nm.BASELINE_CONFIGS["decode_t64"])
    p1 = nm.profile_for(nm.BASELINE_CONFIGS["decode_t1"])
    sel = nm.select_profile((p64, p1), {"m": 64, "batch": 1, "sequence": 0})
    assert sel.supported and sel.profile is p64
    miss = nm.select_profile((p64, p1), {"m": 63, "batch": 1, "sequence": 0})
    assert not miss.supported and "fallback" in miss.reason
    assert not nm.select_profile((p64,), {"m": 64, "batch": 1, "sequence": 0}, tensor_parallel=2).supported
    # netra-profile-1 JSON round trip, as in manifests/gfx950/profiles/decode_m1.json
    doc = {"format": "netra-profile-1", "name": "decode_m1", "guards": {"m": {"min": 1, "max": 1},
           "batch": {"min": 1, "max": 64}, "sequence": {"min": 0, "max": 1048576}},
           "quantization": "fp8_block128", "tensor_parallel": "deployment", "priority": 30}
    prof = nm.ShapeProfile.from_dict(doc)
    assert prof.guard("m").matches(1) and not prof.guard("m").matches(2) and prof.priority == 30


def test_engine_create_without_a_gpu_reports_a_status():
    import torch
    if torch.cuda.is_available():
        pytest.skip("host-only behaviour")
    d = Path(paths.PKG_ROOT) / "lib"
    with pytest.raises(nm.NetraError) as err:
        nm.Engine(d)
    assert err.value.status in (nm.Status.HIP, nm.Status.UNSUPPORTED_TARGET)


def test_op_bridges_declare_the_reference_bridge_abis():
    """Every load/launch/unload/last_error entry point of the reference's four
    bridge headers (runtime/gfx950/fp8/moe/qwen36_moe_silu_mul_quant_bridge.h:14-64,
    moe_prefill_m768_bridge.h:10-23, routing/verify/qwen36_router_bf16_bridge.h:10-21,
    routing/decode/qwen36_shared_gate_append_bridge.h:10-24) is declared, and the
    ctypes binding covers exactly those."""
    from netra_moe import bridges
    names = declared(REPO / "include" / "netra_qwen36_bridges.h")
    assert sorted(names) == sorted(bridges.BRIDGE_SYMBOLS)
    assert len(names) == 24


def test_merged_decode_ffn_follows_the_expected_tile_count():
    """The fused path merges each tile's down into gate/up only when a call is
    expected to have enough 16-row tiles to keep the chip streaming (the
    expected count under uniform routing: E (1 - (1 - K/E)^T) + S ceil(T/16),
    checked against a direct sum over experts), and splits gate/up's K over
    the waves from a larger count; few-expert shapes keep the separate down."""
    from netra_moe.engine import (MERGED_KSPLIT_MIN_TILES, MERGED_MIN_TILES, down_variant,
                                  expected_tiles)

    import numpy as np

    def sampled(T, E, K, S, trials=400):  # touched experts of random uniform top-K routings
        rng = np.random.default_rng(T * 1000 + E)
        touched = [len(np.unique(np.argsort(rng.random((T, E)), axis=1)[:, :K])) for _ in range(trials)]
        return float(np.mean(touched)) + S * ((T + 15) // 16)

    def cfg(T, H, E, K, I, S=1):
        return nm.MoEConfig(f"t{T}_h{H}_e{E}", T=T, H=H, E=E, K=K, I=I, S=S, seed=7)

    for T, E, K, S in ((21, 256, 8, 1), (64, 64, 4, 1), (40, 16, 2, 0), (64, 384, 12, 1)):
        assert expected_tiles(cfg(T, 2048, E, K, 512, S)) == pytest.approx(sampled(T, E, K, S), rel=0.01)
    assert MERGED_MIN_TILES[(2048, 512)] < MERGED_KSPLIT_MIN_TILES[(2048, 512)]
    sym = lambda c: next(op["symbol"] for op in operations(c) if op["name"] == "moe.gate_up")  # noqa: E731
    # H 2048, E 256, K 8: wide at T = 21 (126.6 tiles), merged from T = 22 (130.7), K split from T = 28
    assert down_variant(cfg(21, 2048, 256, 8, 512)) == "wide"
    assert op_names(cfg(21, 2048, 256, 8, 512)) == ("route", "gate_up", "down", "combine")
    assert sym(cfg(22, 2048, 256, 8, 512)) == "netra_moe_ffn_gate_up_down_h2048_i512_gfx950"
    assert op_names(cfg(22, 2048, 256, 8, 512)) == ("route", "gate_up", "combine")
    assert sym(cfg(27, 2048, 256, 8, 512)) == "netra_moe_ffn_gate_up_down_h2048_i512_gfx950"
    assert sym(cfg(28, 2048, 256, 8, 512)) == "netra_moe_ffn_gate_up_down_h2048_i512_ksplit_gfx950"
    # few experts at H 2048 (~67 tiles): the separate down
    assert down_variant(cfg(64, 2048, 64, 4, 512)) == "wide"
    # H 512: merged at every wide T; H 4096 and (1024, 1024): never; narrow T: never
    assert down_variant(cfg(17, 512, 16, 2, 256, 0)) == "merged"
    assert down_variant(cfg(64, 4096, 256, 8, 256)) == "wide"
    assert down_variant(cfg(40, 1024, 24, 3, 1024)) == "wide"
    assert down_variant(cfg(16, 2048, 256, 8, 512)) == "rows"
