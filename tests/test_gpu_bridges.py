"""The reference's per-operation bridge ABIs (include/netra_qwen36_bridges.h,
libnetra_bridges.so) on the GPU, called through ctypes with the reference's
exact signatures and argument formats, against the CPU oracle on the same
seeded inputs.

Shape: the reference's Qwen3.6-35B-A3B layer (hidden 2048, 256 routed experts
+ the shared expert as expert 256, top-8 + 1, intermediate 512), weights in
the AITER 16x16 shuffle with fp32 128x128 block scales.

Bars: router logits, the shared-gate append and the SiLU-quant outputs are
bit-exact (the layer's numeric contract); per-route gate/up fp32 outputs are
within 1e-4 of each route's maximum (fp32 partial sums over K quarters against
float64); down-reduce and the whole decode chain, and the M768 prefill output,
are within the layer tolerance max|y - y_ref| / max|y_ref| <= 2e-2 of the
float64 oracle; the M768 h scales are within one bf16 step (2^-7) and each
split-K2 fp16 partial half within 5e-2 of its float64 half. (The halves are
intermediates computed from the GPU's own h, which may sit one E4M3 step from
the oracle's h on some elements, and a single route row has no slot average
to smooth that out; a swapped half, a wrong K range or a misplaced route row
shows as an error of order 1.)
"""
import numpy as np
import pytest
import torch

import oracle
from bridge_case import (DEV, E, ETOT, H, I, K, KTOT, M768, build_model, capacity, half_rows, prefill_args,
                         prefill_buffers, prefill_inputs, ptr, routing, stream, tokens)
from conftest import gpu_available
from moe_case import bf16_bits
from netra_moe import bridges as B

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

TOL = 2e-2


@pytest.fixture(scope="module")
def model():
    print(f"\n[bridges] building weights H={H} E={ETOT} I={I}", flush=True)
    m = build_model()
    for fam in B.FAMILIES:
        B.check(fam, B.load(fam))
    yield m
    torch.cuda.synchronize()
    for fam in B.FAMILIES:
        B.check(fam, B.unload(fam))


@pytest.mark.parametrize("rows", [1, 16])
def test_router_bridge_bit_exact(model, rows):
    x, xb = tokens(rows, 10 + rows)
    xd = x.to(DEV)
    out = torch.empty((rows, E), dtype=torch.bfloat16, device=DEV)
    B.check("netra_qwen36_router_bf16",
            B.launch("netra_qwen36_router_bf16", ptr(out), ptr(xd), ptr(model["router_w"]), rows, stream()))
    torch.cuda.synchronize()
    ref = oracle.router_logits(xb, model["host"]["router"][:E])
    np.testing.assert_array_equal(bf16_bits(out), ref)


@pytest.mark.parametrize("rows", [1, 16])
def test_shared_gate_append_bridge_bit_exact(model, rows):
    x, xb = tokens(rows, 20 + rows)
    _, ids, wts = routing(model, xb)
    xd = x.to(DEV)
    rid = torch.from_numpy(np.ascontiguousarray(ids[:, :K])).to(DEV)
    rw = torch.from_numpy(np.ascontiguousarray(wts[:, :K])).to(DEV)
    out_ids = torch.empty((rows, KTOT), dtype=torch.int32, device=DEV)
    out_w = torch.empty((rows, KTOT), dtype=torch.float32, device=DEV)
    B.check("netra_qwen36_shared_gate_append",
            B.launch("netra_qwen36_shared_gate_append", ptr(out_ids), ptr(out_w), ptr(xd), ptr(model["shared_w"]),
                     ptr(rid), ptr(rw), rows, stream()))
    torch.cuda.synchronize()
    ref_ids, ref_w = oracle.shared_gate_append(xb, model["host"]["router"][E], ids[:, :K], wts[:, :K], E)
    np.testing.assert_array_equal(out_ids.cpu().numpy(), ref_ids)
    np.testing.assert_array_equal(out_w.cpu().numpy().view(np.uint32), ref_w.view(np.uint32))
    # the same bits as the layer's own top-k shared slot
    np.testing.assert_array_equal(ref_w.view(np.uint32), wts.view(np.uint32))


def decode_inputs(model, rows, seed):
    x, xb = tokens(rows, seed)
    _, ids, wts = routing(model, xb)
    x_q, x_s = oracle.quant_rows_bf16(xb)
    return x_q, x_s, ids, wts


@pytest.mark.parametrize("rows", [1, 4])
def test_gate_up_bridge(model, rows):
    x_q, x_s, ids, _ = decode_inputs(model, rows, 30 + rows)
    out = torch.empty((rows * KTOT, 2 * I), dtype=torch.float32, device=DEV)
    dq, ds, di = (torch.from_numpy(a).to(DEV) for a in (x_q, x_s, ids))
    B.check("netra_qwen36_moe_gate_up",
            B.launch("netra_qwen36_moe_gate_up", ptr(dq), ptr(ds), ptr(model["w13"]), ptr(model["w13_scale"]),
                     ptr(di), ptr(out), rows, stream()))
    torch.cuda.synchronize()
    h = model["host"]
    ref = oracle.stage1_routes(x_q, x_s, h["w13"], h["w13_scale"], ids, ETOT, I)
    got = out.cpu().numpy()
    err = np.max(np.abs(got - ref), axis=1) / np.max(np.abs(ref), axis=1)
    print(f"[bridges] gate/up rows={rows} worst route rel err {err.max():.2e}")
    assert np.all(np.isfinite(got)) and err.max() <= 1e-4


@pytest.mark.parametrize("rows", [9, 36])
def test_silu_mul_quant_bridge_bit_exact(model, rows):
    rng = np.random.default_rng(40 + rows)
    gu = (rng.standard_normal((rows, 2 * I)) * 3).astype(np.float32)
    gu[0, :128] = 0.0  # a group with h == 0 everywhere: floor scale
    din = torch.from_numpy(gu).to(DEV)
    q = torch.empty((rows, I), dtype=torch.uint8, device=DEV)
    s = torch.empty((rows, I // 128), dtype=torch.float32, device=DEV)
    B.check("netra_qwen36_moe_silu_mul_quant",
            B.launch("netra_qwen36_moe_silu_mul_quant", ptr(din), ptr(q), ptr(s), rows, stream()))
    torch.cuda.synchronize()
    rq, rs = oracle.silu_mul_quant(gu)
    np.testing.assert_array_equal(q.cpu().numpy(), rq)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("rows", [1, 4])
def test_down_reduce_bridge(model, rows):
    x_q, x_s, ids, wts = decode_inputs(model, rows, 50 + rows)
    h = model["host"]
    hq, hs = oracle.silu_mul_quant(oracle.stage1_routes(x_q, x_s, h["w13"], h["w13_scale"], ids, ETOT, I))
    dq, ds, dw, di = (torch.from_numpy(a).to(DEV) for a in (hq, hs, wts, ids))
    out = torch.empty((rows, H), dtype=torch.bfloat16, device=DEV)
    B.check("netra_qwen36_moe_down_reduce",
            B.launch("netra_qwen36_moe_down_reduce", ptr(dq), ptr(ds), ptr(model["w2"]), ptr(model["w2_scale"]),
                     ptr(dw), ptr(di), ptr(out), rows, stream()))
    torch.cuda.synchronize()
    ref_f, _ = oracle.down_reduce_routes(hq, hs, h["w2"], h["w2_scale"], ids, wts, ETOT)
    err = oracle.max_abs_rel(oracle.f32_from_bf16(bf16_bits(out)), ref_f)
    print(f"[bridges] down-reduce rows={rows} max_abs_rel {err:.2e}")
    assert err <= TOL


def test_decode_chain_through_the_bridges(model):
    """router -> (oracle top-k) -> shared-gate append -> gate/up -> SiLU-quant ->
    down-reduce, every step on the GPU through its bridge, against the oracle's
    whole expert path."""
    rows = 16
    x, xb = tokens(rows, 60)
    xd = x.to(DEV)
    logits = torch.empty((rows, E), dtype=torch.bfloat16, device=DEV)
    B.check("netra_qwen36_router_bf16",
            B.launch("netra_qwen36_router_bf16", ptr(logits), ptr(xd), ptr(model["router_w"]), rows, stream()))
    torch.cuda.synchronize()
    # the reference takes top-k from SGLang; the oracle's contract stands in
    ids8, w8 = oracle.topk(bf16_bits(logits), None, E, K, 0)
    rid, rw = torch.from_numpy(ids8).to(DEV), torch.from_numpy(w8).to(DEV)
    ids = torch.empty((rows, KTOT), dtype=torch.int32, device=DEV)
    wts = torch.empty((rows, KTOT), dtype=torch.float32, device=DEV)
    B.check("netra_qwen36_shared_gate_append",
            B.launch("netra_qwen36_shared_gate_append", ptr(ids), ptr(wts), ptr(xd), ptr(model["shared_w"]),
                     ptr(rid), ptr(rw), rows, stream()))
    x_q, x_s = oracle.quant_rows_bf16(xb)  # the reference's AITER input quant stands outside the bridges
    dq, ds = torch.from_numpy(x_q).to(DEV), torch.from_numpy(x_s).to(DEV)
    gu = torch.empty((rows * KTOT, 2 * I), dtype=torch.float32, device=DEV)
    B.check("netra_qwen36_moe_gate_up",
            B.launch("netra_qwen36_moe_gate_up", ptr(dq), ptr(ds), ptr(model["w13"]), ptr(model["w13_scale"]),
                     ptr(ids), ptr(gu), rows, stream()))
    hq = torch.empty((rows * KTOT, I), dtype=torch.uint8, device=DEV)
    hs = torch.empty((rows * KTOT, I // 128), dtype=torch.float32, device=DEV)
    B.check("netra_qwen36_moe_silu_mul_quant",
            B.launch("netra_qwen36_moe_silu_mul_quant", ptr(gu), ptr(hq), ptr(hs), rows * KTOT, stream()))
    out = torch.empty((rows, H), dtype=torch.bfloat16, device=DEV)
    B.check("netra_qwen36_moe_down_reduce",
            B.launch("netra_qwen36_moe_down_reduce", ptr(hq), ptr(hs), ptr(model["w2"]), ptr(model["w2_scale"]),
                     ptr(wts), ptr(ids), ptr(out), rows, stream()))
    torch.cuda.synchronize()
    ref_logits, ref_ids, ref_w = routing(model, xb)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref_ids)
    np.testing.assert_array_equal(wts.cpu().numpy().view(np.uint32), ref_w.view(np.uint32))
    h = model["host"]
    ref_f, _ = oracle.moe_tokens(x_q, x_s, h["w13"], h["w13_scale"], h["w2"], h["w2_scale"], ref_ids, ref_w,
                                 np.arange(rows, dtype=np.int64), H, I)
    err = oracle.max_abs_rel(oracle.f32_from_bf16(bf16_bits(out)), ref_f)
    print(f"[bridges] decode chain rows={rows} max_abs_rel {err:.2e}")
    assert err <= TOL


CAP = capacity(M768)      # 365 blocks
HALF = half_rows(M768)    # 7277 rows between the split-K2 halves


def run_m768(model, inp):
    d = prefill_buffers(inp)
    rc = B.launch("netra_moe_prefill_m768", *prefill_args(model, d), stream())
    torch.cuda.synchronize()
    return rc, d["out"], d["rs"], d["parts"]


def test_prefill_m768_bridge(model):
    inp = prefill_inputs(model, tokens(M768, 70)[1])
    x_q, x_s, ids, wts, sid, sexp, nv = (inp[k] for k in ("x_q", "x_s", "ids", "wts", "sid", "sexp", "nv"))
    print(f"[bridges] m768: {int(nv[0])} sorted rows of {CAP * 64}", flush=True)
    rc, out, rs, parts = run_m768(model, inp)
    B.check("netra_moe_prefill_m768", rc)
    h = model["host"]
    # output on a seeded sample of tokens
    rng = np.random.default_rng(71)
    toks = np.unique(np.concatenate([[0, M768 - 1], rng.choice(M768, 190, replace=False)])).astype(np.int64)
    ref_f, _ = oracle.moe_tokens(x_q, x_s, h["w13"], h["w13_scale"], h["w2"], h["w2_scale"], ids, wts, toks, H, I)
    y = oracle.f32_from_bf16(bf16_bits(out))
    err = oracle.max_abs_rel(y[toks], ref_f)
    print(f"[bridges] m768 output max_abs_rel {err:.2e} over {toks.size} tokens")
    assert np.all(np.isfinite(y)) and err <= TOL
    # h scales (route_scale_workspace) on sampled sorted rows
    nvr = int(nv[0])
    rows = np.unique(np.concatenate([rng.choice(nvr, 512, replace=False), np.arange(64), np.arange(nvr - 64, nvr)]))
    rows = rows[(sid[rows] & 0xFFFFFF) < M768]
    hq_ref, hs_ref = oracle.gate_up_rows(x_q, x_s, h["w13"], h["w13_scale"], sid, sexp, rows, M768, H, I)
    got_s = rs.cpu().numpy()[rows].astype(np.float64)
    srel = float(np.max(np.abs(got_s - hs_ref) / hs_ref))
    print(f"[bridges] m768 h scales worst rel {srel:.2e} over {rows.size} rows")
    assert srel <= 2.0 ** -7
    # split-K2 halves on sampled routes, from the oracle's h
    pick = rows[:48]
    t, s = sid[pick] & 0xFFFFFF, sid[pick] >> 24
    p0, p1 = oracle.stage2_split_halves(hq_ref[:48], hs_ref[:48].astype(np.float32), h["w2"], h["w2_scale"],
                                        sexp[pick // 64])
    pp = parts.float().cpu().numpy()
    g0, g1 = pp[0][t * KTOT + s], pp[1][t * KTOT + s]
    e0 = float(np.max(np.abs(g0 - p0)) / np.max(np.abs(p0)))
    e1 = float(np.max(np.abs(g1 - p1)) / np.max(np.abs(p1)))
    print(f"[bridges] m768 split-K2 halves rel err {e0:.2e} {e1:.2e}")
    assert e0 <= 5e-2 and e1 <= 5e-2
    # a second launch is bitwise identical
    rc2, out2, _, _ = run_m768(model, inp)
    B.check("netra_moe_prefill_m768", rc2)
    np.testing.assert_array_equal(bf16_bits(out2), bf16_bits(out))


def test_bridge_refusals(model):
    lib = B.library()
    fam = "netra_qwen36_moe_gate_up"
    dummy = torch.zeros(16, dtype=torch.float32, device=DEV)
    p = ptr(dummy)
    # rows <= 0 and null pointers
    assert B.launch(fam, p, p, p, p, p, p, 0, stream()) == -1
    assert "rows" in B.last_error(fam)
    assert B.launch(fam, p, None, p, p, p, p, 1, stream()) == -1
    assert "nonnull" in B.last_error(fam)
    # the router and shared gate take 1 or 16 rows, as in the reference
    assert B.launch("netra_qwen36_router_bf16", p, p, p, 2, stream()) == -1
    # loading a different code object without unloading first
    assert lib.netra_qwen36_moe_gate_up_load(b"/nonexistent/other.hsaco") == -1
    assert "unload" in B.last_error(fam)
    # unload, launch refused, reload
    assert B.unload(fam) == 0
    assert B.launch(fam, p, p, p, p, p, p, 1, stream()) == -1
    assert "not loaded" in B.last_error(fam)
    assert B.load(fam) == 0
    assert B.last_error(fam) == ""
    # the prefill pair loads one module when both paths name the same code
    # object; unloading it releases that module once and leaves no HIP error
    # behind for the caller's next call
    pre = "netra_moe_prefill_m768"
    assert B.unload(pre) == 0, B.last_error(pre)
    torch.cuda.synchronize()
    assert float(torch.ones(4, device=DEV).sum()) == 4.0
    assert B.load(pre) == 0, B.last_error(pre)
