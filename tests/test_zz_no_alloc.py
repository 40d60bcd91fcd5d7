"""netra_moe_prefill_launch_noalloc (libnetra_moe.so, include/netra_moe.h):
the allocation-free variant of netra_moe_prefill_m768_launch
(libnetra_bridges.so), checked against that entry point through the C ABI.

Two calls in a row on one process: 768 tokens, then 300 tokens (a smaller
input, so the shared static scratch is reused with a smaller capacity). Each
token's output depends only on its own routes (rows of an MFMA tile are
independent, and every per-row sum keeps its order whatever block the row
sits in), so:
* the 768-token call equals the existing entry point's output, h scales and
  fp16 partials bit for bit;
* the 300-token call equals the existing entry point's output on the same
  300 tokens (the first 300 of its 768-token input) bit for bit, and the
  oracle within the layer tolerance;
* rows outside 1..768 are refused with a message, and nothing is launched.
"""
import numpy as np
import pytest
import torch

import oracle
from bridge_case import (DEV, H, I, KTOT, M768, build_model, prefill_args, prefill_buffers, prefill_inputs,
                         stream, tokens)
from conftest import gpu_available
from moe_case import bf16_bits
from netra_moe import bridges as B
from netra_moe import weights as W

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

SMALL = 300


def noalloc(model, d, rows):
    lib = W.bridge_library()
    rc = lib.netra_moe_prefill_launch_noalloc(*prefill_args(model, d), rows, stream())
    return rc, lib.netra_moe_last_error().decode()


def test_noalloc_prefill_matches_the_bridge_on_two_calls():
    print("\n[no-alloc] building weights", flush=True)
    model = build_model()
    x, xb = tokens(M768, 90)
    big = prefill_inputs(model, xb)
    small = prefill_inputs(model, xb[:SMALL])

    # the existing entry point (module-loaded code object, scratch from load)
    B.check("netra_moe_prefill_m768", B.load("netra_moe_prefill_m768"))
    ref = prefill_buffers(big)
    B.check("netra_moe_prefill_m768", B.launch("netra_moe_prefill_m768", *prefill_args(model, ref), stream()))
    torch.cuda.synchronize()
    B.check("netra_moe_prefill_m768", B.unload("netra_moe_prefill_m768"))

    # call 1: 768 tokens
    print("[no-alloc] call 1: rows=768", flush=True)
    d1 = prefill_buffers(big)
    rc, msg = noalloc(model, d1, M768)
    assert rc == 0, msg
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bf16_bits(d1["out"]), bf16_bits(ref["out"]))
    sid = big["sid"]
    valid_rows = np.nonzero((sid & 0xFFFFFF) < M768)[0]
    np.testing.assert_array_equal(d1["rs"].cpu().numpy()[valid_rows].view(np.uint32),
                                  ref["rs"].cpu().numpy()[valid_rows].view(np.uint32))
    routes = M768 * KTOT
    np.testing.assert_array_equal(d1["parts"][:, :routes].cpu().numpy().view(np.uint16),
                                  ref["parts"][:, :routes].cpu().numpy().view(np.uint16))

    # call 2: 300 tokens, right after
    print(f"[no-alloc] call 2: rows={SMALL}", flush=True)
    d2 = prefill_buffers(small)
    rc, msg = noalloc(model, d2, SMALL)
    assert rc == 0, msg
    torch.cuda.synchronize()
    out2 = bf16_bits(d2["out"])
    np.testing.assert_array_equal(out2, bf16_bits(ref["out"])[:SMALL])
    h = model["host"]
    toks = np.arange(0, SMALL, 3, dtype=np.int64)
    ref_f, _ = oracle.moe_tokens(small["x_q"], small["x_s"], h["w13"], h["w13_scale"], h["w2"], h["w2_scale"],
                                 small["ids"], small["wts"], toks, H, I)
    err = oracle.max_abs_rel(oracle.f32_from_bf16(out2[toks]), ref_f)
    print(f"[no-alloc] rows={SMALL} output max_abs_rel {err:.2e} against the oracle")
    assert err <= 2e-2

    # sizes beyond the static scratch are refused before anything is launched
    for rows in (0, M768 + 1):
        rc, msg = noalloc(model, d2, rows)
        assert rc == -1 and "1..768" in msg, (rows, rc, msg)
