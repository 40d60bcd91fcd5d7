"""Device numerics: the E4M3 encoders and the weight-prep quantiser.

The hot kernels convert with the gfx950 instruction; the contract (shared with
the CPU oracle) is an integer RNE encoder with saturation at 448. Both are
swept over a dense grid of fp32 bit patterns and compared with each other and
with torch's float8_e4m3fn conversion (an independent implementation).
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import gpu_available
from netra_moe import weights as W

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]
DEV = torch.device("cuda", 0)


def _sweep() -> np.ndarray:
    # every 97th fp32 bit pattern from 0 up to 480.0, every e4m3 value and every
    # rounding midpoint with its two fp32 neighbours, both signs, plus specials
    pos = np.arange(0, 0x43F00000, 97, dtype=np.uint32)
    vals = np.array([oracle.lib().orc_f32_from_e4m3(c) for c in range(0x7F)], dtype=np.float32)
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32).view(np.uint32)
    around = np.concatenate([vals.view(np.uint32), mids, mids - 1, mids + 1])
    edges = np.array([0x43E00000, 0x43E00001, 0x43E7FFFF, 0x43E80000, 0x7F7FFFFF, 0x7F800000,
                      0x3B000000, 0x3B800000, 0x3C800000, 0x00000001], dtype=np.uint32)
    bits = np.concatenate([pos, around.astype(np.uint32), edges])
    bits = np.concatenate([bits, bits | 0x80000000])
    return bits.view(np.float32)


def test_hw_conversion_matches_contract_encoder():
    x = _sweep()
    xt = torch.from_numpy(x).to(DEV)
    sw = torch.empty(x.size, dtype=torch.uint8, device=DEV)
    hw = torch.empty_like(sw)
    lib = W.bridge_library()
    rc = lib.netra_moe_e4m3_check(xt.data_ptr(), sw.data_ptr(), hw.data_ptr(), x.size,
                                  torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.netra_moe_last_error()
    torch.cuda.synchronize()
    sw, hw = sw.cpu().numpy(), hw.cpu().numpy()
    bad = np.nonzero(sw != hw)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[bad[:5]]} sw={sw[bad[:5]]} hw={hw[bad[:5]]}"
    # the contract encoder agrees with torch's RNE conversion inside the finite range
    finite = np.abs(x) <= 448.0
    ref = torch.from_numpy(x[finite]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(sw[finite], ref)
    # and saturates above it
    assert np.all((sw[~finite] & 0x7F) == 0x7E)


def test_weight_prep_kernel_bit_exact_vs_oracle():
    g = torch.Generator().manual_seed(5)
    w = torch.randn((3, 256, 384), generator=g) * 0.02
    w[1, :128, :128] *= 1000.0          # a block with a very different scale
    w[2, 128:, 256:] = 0.0              # an all-zero block (amax floor)
    q_ref, s_ref = oracle.quant_blocks_f32(w.numpy())
    q, s = W.quantize_blocks(w.to(DEV).contiguous())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


def test_pack_tiles_kernel_matches_host_layout():
    g = np.random.default_rng(3)
    q = g.integers(0, 256, size=(3, 64, 384), dtype=np.uint8)
    out = W.pack_tiles(torch.from_numpy(q).to(DEV))
    out_gu = W.pack_tiles(torch.from_numpy(q).to(DEV), gate_up=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), W.pack_tiles_host(q))
    np.testing.assert_array_equal(out_gu.cpu().numpy(), W.pack_tiles_host(q, gate_up=True))


@pytest.mark.parametrize("n,k,gate_up", [(64, 256, False), (1024, 512, True), (2048, 512, False), (96, 384, True)])
def test_pack_from_aiter_equals_pack_from_row_major(n, k, gate_up):
    """Weights in the reference's AITER 16x16 shuffle convert to exactly the
    bytes the row-major packer writes."""
    rng = np.random.default_rng(n + k)
    q = rng.integers(0, 256, size=(3, n, k), dtype=np.uint8)
    src = torch.from_numpy(W.aiter_shuffle_host(q)).to(DEV)
    got = W.pack_tiles_from_aiter(src, gate_up=gate_up)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), W.pack_tiles_host(q, gate_up=gate_up))
