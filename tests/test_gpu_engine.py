"""Engine C-ABI behaviour on the GPU, through ctypes on the cpu_small layer.

* A manifest whose launch does not fit the compiled kernel (a block beyond the
  kernel's flat work-group bound) is refused at create with MANIFEST, as the
  reference runtime refuses malformed manifests
  (runtime/gfx950/engine/netra_engine.hip:273-383).
* netra_engine_launch_operation_bound, op by op with every pointer slot given
  by the caller, computes the same bytes as netra_engine_launch.
* The refusal statuses of the reference runtime's state model
  (runtime/gfx950/engine/netra_engine.hip:406-566, and the checks of
  harness/gfx950/engine/netra_engine_smoke.hip:20-36): bind after finalize and
  single-operation launches after graph preparation are BUSY, a shape outside
  the profile guards is UNSUPPORTED_PROFILE, a framework-fallback operation is
  FALLBACK_REQUIRED, malformed bound launches are BINDING, a direct launch
  before finalize is BINDING.
"""
import ctypes
import json

import numpy as np
import pytest
import torch

import netra_moe as nm
from conftest import gpu_available
from moe_case import bf16_bits, make_inputs
from netra_moe.layer import TORCH_DTYPES
from netra_moe.runtime import LaunchShape, PointerBinding, Status

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

DEV = torch.device("cuda", 0)
CFG = nm.BASELINE_CONFIGS["cpu_small"]


def test_block_beyond_kernel_bound_is_refused(tmp_path):
    d = tmp_path / "eng"
    nm.compile_moe_engine(CFG, d, path="tile")
    eng = nm.Engine(d)  # the emitted engine loads
    eng.destroy()
    doc = json.loads((d / "engine.json").read_text())
    op = next(o for o in doc["operations"] if o["name"] == "moe.gate_up")
    op["launch"]["block"] = [1024, 1, 1]
    (d / "engine.json").write_text(json.dumps(doc))
    with pytest.raises(nm.NetraError) as err:
        nm.Engine(d)
    assert err.value.status == Status.MANIFEST


@pytest.fixture(scope="module")
def layer_inputs():
    x, gpu_w, _ = make_inputs(CFG, DEV)
    return x, gpu_w


def _buffers(recipe, specs, x, weights):
    bufs = {"x": x.to(DEV).contiguous(), **weights}
    for name, info in recipe["tensors"].items():
        if info["storage"] == "binding" and name not in bufs:
            spec = specs[name]
            bufs[name] = torch.zeros(spec.shape, dtype=TORCH_DTYPES[spec.dtype], device=DEV)
    return bufs


def _engine(tmp_path, name, layer_inputs, graph):
    d = tmp_path / name
    recipe = nm.compile_moe_engine(CFG, d)
    specs = nm.engine.tensor_table(CFG)
    bufs = _buffers(recipe, specs, *layer_inputs)
    eng = nm.Engine(d, graph_capture=graph)
    return eng, recipe, bufs


def _bind_all(eng, recipe, bufs):
    for name, slots in recipe["bindings"].items():
        for profile, op, arg in slots:
            eng.bind(profile, op, arg, bufs[name].data_ptr())


def _slots_by_op(recipe, bufs):
    per_op: dict[int, list[tuple[int, int]]] = {}
    for name, slots in recipe["bindings"].items():
        for _, op, arg in slots:
            per_op.setdefault(op, []).append((arg, bufs[name].data_ptr()))
    return per_op


def _status(eng, fn, *args):
    return Status(fn(eng.handle, *args))


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)


def test_bound_launches_equal_the_profile_launch(tmp_path, layer_inputs):
    shape = LaunchShape(CFG.T, 1, 0, 1)
    a, recipe, bufs_a = _engine(tmp_path, "a", layer_inputs, graph=False)
    _bind_all(a, recipe, bufs_a)
    a.finalize()
    a.launch(0, shape, torch.cuda.current_stream(DEV).cuda_stream)
    b, recipe_b, bufs_b = _engine(tmp_path, "b", layer_inputs, graph=False)
    per_op = _slots_by_op(recipe_b, bufs_b)
    for op in range(len(recipe_b["operations"])):
        b.launch_operation_bound(0, op, shape, per_op.get(op, []), torch.cuda.current_stream(DEV).cuda_stream)
    torch.cuda.synchronize(DEV)
    out_a, out_b = bf16_bits(bufs_a["out"]), bf16_bits(bufs_b["out"])
    assert np.any(out_a != 0)
    np.testing.assert_array_equal(out_a, out_b)
    a.destroy()
    b.destroy()


def test_bound_launch_refusals(tmp_path, layer_inputs):
    eng, recipe, bufs = _engine(tmp_path, "c", layer_inputs, graph=False)
    lib, shape = eng.lib, LaunchShape(CFG.T, 1, 0, 1)
    per_op = _slots_by_op(recipe, bufs)
    op = 0
    slots = per_op[op]

    def bound(entries, count=None):
        arr = (PointerBinding * max(1, len(entries)))()
        for i, (arg, ptr, reserved) in enumerate(entries):
            arr[i] = PointerBinding(arg, reserved, ctypes.c_void_p(ptr))
        n = len(entries) if count is None else count
        return _status(eng, lib.netra_engine_launch_operation_bound, 0, op, ctypes.byref(shape), arr, n, _stream())

    full = [(arg, ptr, 0) for arg, ptr in slots]
    assert bound(full[:-1]) == Status.BINDING                      # a slot missing
    assert bound(full[:-1] + [full[0]]) == Status.BINDING           # a slot twice
    assert bound([(full[0][0], full[0][1], 1)] + full[1:]) == Status.BINDING  # reserved field set
    constant = next(i for i, a in enumerate(json.loads((tmp_path / "c" / "engine.json").read_text())
                                            ["operations"][op]["arguments"]) if a["kind"] == "u32_constant")
    assert bound(full[:-1] + [(constant, full[-1][1], 0)]) == Status.BINDING  # not a pointer slot
    assert bound(full, count=17) == Status.INVALID_ARGUMENT
    wrong = LaunchShape(CFG.T + 1, 1, 0, 1)
    arr = (PointerBinding * len(full))(*[PointerBinding(a, 0, ctypes.c_void_p(p)) for a, p, _ in full])
    assert _status(eng, lib.netra_engine_launch_operation_bound, 0, op, ctypes.byref(wrong), arr,
                   len(full), _stream()) == Status.UNSUPPORTED_PROFILE
    assert bound(full) == Status.OK
    torch.cuda.synchronize(DEV)
    eng.destroy()


def test_state_model_refusals(tmp_path, layer_inputs):
    eng, recipe, bufs = _engine(tmp_path, "d", layer_inputs, graph=True)
    lib = eng.lib
    shape, wrong = LaunchShape(CFG.T, 1, 0, 1), LaunchShape(CFG.T + 1, 1, 0, 1)
    # a direct launch before finalize
    assert _status(eng, lib.netra_engine_launch, 0, ctypes.byref(shape), _stream()) == Status.BINDING
    # finalize with an unbound slot
    assert _status(eng, lib.netra_engine_finalize_bindings) == Status.BINDING
    _bind_all(eng, recipe, bufs)
    eng.finalize()
    any_slot = next(iter(recipe["bindings"].values()))[0]
    st = _status(eng, lib.netra_engine_bind, *any_slot, ctypes.c_void_p(bufs["x"].data_ptr()))
    assert st == Status.BUSY
    assert lib.netra_engine_last_error(eng.handle).decode() == "bindings are finalized and immutable"
    # a shape outside the guards (the reference smoke harness's check)
    assert _status(eng, lib.netra_engine_launch, 0, ctypes.byref(wrong), _stream()) == Status.UNSUPPORTED_PROFILE
    assert _status(eng, lib.netra_engine_launch_operation, 0, 0, ctypes.byref(wrong), _stream()) \
        == Status.UNSUPPORTED_PROFILE
    assert _status(eng, lib.netra_engine_launch, 7, ctypes.byref(shape), _stream()) == Status.INVALID_ARGUMENT
    capture = torch.cuda.Stream(DEV)
    eng.prepare(0, capture.cuda_stream)
    assert _status(eng, lib.netra_engine_launch_operation, 0, 0, ctypes.byref(shape), _stream()) == Status.BUSY
    per_op = _slots_by_op(recipe, bufs)
    arr = (PointerBinding * len(per_op[0]))(*[PointerBinding(a, 0, ctypes.c_void_p(p)) for a, p in per_op[0]])
    assert _status(eng, lib.netra_engine_launch_operation_bound, 0, 0, ctypes.byref(shape), arr,
                   len(per_op[0]), _stream()) == Status.BUSY
    eng.launch(0, shape, torch.cuda.current_stream(DEV).cuda_stream)
    torch.cuda.synchronize(DEV)
    assert np.any(bf16_bits(bufs["out"]) != 0)
    eng.destroy()


def test_fallback_operation_refusals(tmp_path, layer_inputs):
    d = tmp_path / "fb"
    recipe = nm.compile_moe_engine(CFG, d)
    doc = json.loads((d / "engine.json").read_text())
    fb = len(doc["operations"]) - 1  # the combine becomes a framework-fallback operation
    doc["operations"][fb] = {"name": "moe.combine", "execution": "framework_fallback"}
    (d / "engine.json").write_text(json.dumps(doc))
    eng = nm.Engine(d, graph_capture=True)
    lib = eng.lib
    assert eng.query_profile(0).requires_fallback == 1
    shape = LaunchShape(CFG.T, 1, 0, 1)
    bufs = _buffers(recipe, nm.engine.tensor_table(CFG), *layer_inputs)
    for name, slots in recipe["bindings"].items():
        for profile, op, arg in slots:
            if op != fb:
                eng.bind(profile, op, arg, bufs[name].data_ptr())
    eng.finalize()
    assert _status(eng, lib.netra_engine_launch, 0, ctypes.byref(shape), _stream()) == Status.FALLBACK_REQUIRED
    assert _status(eng, lib.netra_engine_launch_operation, 0, fb, ctypes.byref(shape), _stream()) \
        == Status.FALLBACK_REQUIRED
    assert _status(eng, lib.netra_engine_prepare_profile, 0, _stream()) == Status.FALLBACK_REQUIRED
    # the kernel operations before it still launch one by one
    for op in range(fb):
        eng.launch_operation(0, op, shape, torch.cuda.current_stream(DEV).cuda_stream)
    torch.cuda.synchronize(DEV)
    eng.destroy()
