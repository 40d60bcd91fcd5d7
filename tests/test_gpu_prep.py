"""Weight prep on the GPU: a sharded per-expert checkpoint with bf16 and fp32
scales and a shared expert, stacked and packed by netra_moe.prep, is bit for
bit the oracle's stacking of the same tensors."""
import numpy as np
import pytest
import torch

import oracle
from netra_moe import prep
from prep_case import PREFIX, synthetic_checkpoint
from test_prep_oracle import CFG, _torch_checkpoint

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("source", ["host", "device"])
def test_stacked_checkpoint_is_bit_exact(source):
    dev = torch.device("cuda", 0)
    ck = synthetic_checkpoint(CFG.E, CFG.S, CFG.H, CFG.I)
    tensors = _torch_checkpoint(ck)
    if source == "device":
        tensors = {k: ([t.to(dev) for t in v] if isinstance(v, list) else v.to(dev)) for k, v in tensors.items()}
    got = prep.stack_checkpoint(CFG, tensors, PREFIX, dev)
    torch.cuda.synchronize()
    want = oracle.stack_checkpoint(ck, CFG.E, CFG.S, CFG.H, CFG.I, PREFIX)
    for name in ("w13", "w2"):
        np.testing.assert_array_equal(got[name].cpu().numpy(), want[name], err_msg=name)
    for name in ("w13_scale", "w2_scale"):
        np.testing.assert_array_equal(got[name].cpu().numpy().view(np.uint32), want[name].view(np.uint32),
                                      err_msg=name)
