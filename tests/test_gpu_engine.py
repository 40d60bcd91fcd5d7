"""Engine runtime checks that need a GPU but launch nothing: the runtime refuses
a manifest whose launch does not fit the compiled kernel (a block beyond the
kernel's flat work-group bound) with a MANIFEST status, as the reference
runtime refuses malformed manifests at create time
(runtime/gfx950/engine/netra_engine.hip:273-383)."""
import json

import pytest

import netra_moe as nm
from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def test_block_beyond_kernel_bound_is_refused(tmp_path):
    cfg = nm.BASELINE_CONFIGS["cpu_small"]
    d = tmp_path / "eng"
    nm.compile_moe_engine(cfg, d, path="tile")
    eng = nm.Engine(d)  # the emitted engine loads
    eng.destroy()
    doc = json.loads((d / "engine.json").read_text())
    op = next(o for o in doc["operations"] if o["name"] == "moe.gate_up")
    op["launch"]["block"] = [1024, 1, 1]
    (d / "engine.json").write_text(json.dumps(doc))
    with pytest.raises(nm.NetraError) as err:
        nm.Engine(d)
    assert err.value.status == nm.Status.MANIFEST
