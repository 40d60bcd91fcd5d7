"""Weight prep on the CPU: the oracle's stacking restatement is pinned, and the
product's step plan and input checks follow the reference's layout plan
(compiler/netra_compiler/layouts.py:109-206)."""
import numpy as np
import pytest
import torch

import oracle
from netra_moe import prep
from netra_moe import weights as W
from netra_moe.config import MoEConfig
from prep_case import PREFIX, synthetic_checkpoint

CFG = MoEConfig("prep", T=1, H=256, E=6, K=2, I=256, S=1)


@pytest.mark.parametrize("gate_up", [False, True])
def test_oracle_tile_placement_matches_the_documented_permutation(gate_up):
    # two formulations of one layout: per-element destinations (oracle) and the
    # reshape/transpose restatement pinned byte by byte in test_layouts.py
    q = np.random.default_rng(1).integers(0, 256, size=(3, 64, 256), dtype=np.uint8)
    np.testing.assert_array_equal(oracle.tile16x128(q, gate_up), W.pack_tiles_host(q, gate_up))


def test_oracle_stacking_places_shards_shared_expert_and_scales():
    ck = synthetic_checkpoint(CFG.E, CFG.S, CFG.H, CFG.I)
    st = oracle.stack_checkpoint(ck, CFG.E, CFG.S, CFG.H, CFG.I, PREFIX)
    w13 = W.unpack_tiles_host(st["w13"], gate_up=True)
    w2 = W.unpack_tiles_host(st["w2"])
    for slot, owner in [(0, "experts.0"), (3, "experts.3"), (CFG.E, "shared_expert")]:
        gate = ck[f"{PREFIX}.{owner}.gate_proj.weight"]
        gate = np.concatenate(gate) if isinstance(gate, list) else gate
        np.testing.assert_array_equal(w13[slot, :CFG.I], gate)
        down = ck[f"{PREFIX}.{owner}.down_proj.weight"]
        down = np.concatenate(down) if isinstance(down, list) else down
        np.testing.assert_array_equal(w2[slot], down)
    # even experts carry bf16 scales: the fp32 bits are the bf16 bits shifted up
    sc = ck[f"{PREFIX}.experts.2.up_proj.weight_scale_inv"]
    bits = (np.concatenate(sc) if isinstance(sc, list) else sc).astype(np.uint32) << 16
    np.testing.assert_array_equal(st["w13_scale"][2, CFG.I // 128:].view(np.uint32), bits)
    assert st["w13_scale"].dtype == np.float32 and st["w13_scale"].shape == (CFG.Etot, 4, 2)


def _torch_checkpoint(ck):
    def conv(a, i):
        t = torch.from_numpy(np.ascontiguousarray(a))
        if a.dtype == np.uint16:
            return t.view(torch.bfloat16)
        if a.dtype == np.uint8 and i % 2:
            return t.view(torch.float8_e4m3fn)
        return t
    return {k: ([conv(a, i) for i, a in enumerate(v)] if isinstance(v, list) else conv(v, 1))
            for k, v in ck.items()}


def test_plan_lists_the_reference_steps():
    steps = [s.to_dict() for s in prep.plan_checkpoint(CFG, _torch_checkpoint(synthetic_checkpoint(
        CFG.E, CFG.S, CFG.H, CFG.I)), PREFIX)]
    assert {"tensor": "w13", "transform": "concatenate_output_shards", "parameters": {"axis": 0, "shards": 2}} in steps
    assert {"tensor": "w13_scale", "transform": "widen_bf16_to_fp32_exact", "parameters": {}} in steps
    assert {"tensor": "w2", "transform": "stack_experts", "parameters": {"routed": 6, "shared": 1}} in steps
    assert steps[-1] == {"tensor": "w2", "transform": "tile16x128", "parameters": {}}


def test_missing_and_malformed_tensors_are_named():
    ck = _torch_checkpoint(synthetic_checkpoint(CFG.E, CFG.S, CFG.H, CFG.I))
    del ck[f"{PREFIX}.shared_expert.up_proj.weight"]
    with pytest.raises(KeyError, match="shared_expert.up_proj.weight"):
        prep.plan_checkpoint(CFG, ck, PREFIX)
    bad = {"x": [torch.zeros((100, 256), dtype=torch.uint8), torch.zeros((100, 256), dtype=torch.uint8)]}
    with pytest.raises(ValueError, match="expected 256"):
        prep._weight(bad, "x", 256, 256, "cpu")
    with pytest.raises(ValueError, match="bf16 or fp32"):
        prep._scale({"s": torch.zeros((2, 2), dtype=torch.float16)}, "s", 2, 2, "cpu")
