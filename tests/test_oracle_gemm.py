"""Pins the oracle's grouped GEMMs and the end-to-end layer.

Stage 1 and stage 2 are compared with dense float64 numpy matrix products of
the dequantised operands (a different formulation: whole-matrix products with
the block scales expanded, no loops over K blocks); the token-major and
sorted-order drivers must agree exactly; and a one-expert, top-1 layer must
reduce to the textbook SwiGLU FFN y = W2 (silu(Wg x) * (Wu x)) computed by
torch in float64 on the unquantised weights, within the layer tolerance.
"""
import numpy as np
import torch

import oracle

bits = oracle.bf16_from_f32
val = oracle.f32_from_bf16


def make(T=12, H=256, E=4, K=2, I=128, seed=0):
    rng = np.random.default_rng(seed)
    x = val(bits(rng.standard_normal((T, H)).astype(np.float32)))
    w13 = (rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float32)
    w2 = (rng.standard_normal((E, H, I)) * 0.02).astype(np.float32)
    router = val(bits((rng.standard_normal((E, H)) * 0.02).astype(np.float32)))
    q13, s13 = oracle.quant_blocks_f32(w13, threads=2)
    q2, s2 = oracle.quant_blocks_f32(w2, threads=2)
    return x, router, w13, w2, q13, s13, q2, s2


def dequant_blocks(q, s):
    table = oracle.e4m3_table().astype(np.float64)
    return table[q] * np.repeat(np.repeat(s.astype(np.float64), 128, axis=1), 128, axis=2)


def dequant_rows(q, s):
    table = oracle.e4m3_table().astype(np.float64)
    return table[q] * np.repeat(s.astype(np.float64), 128, axis=1)


def test_stage1_and_stage2_match_dense_float64():
    T, H, E, K, I = 12, 256, 4, 2, 128
    x, router, _, _, q13, s13, q2, s2 = make(T, H, E, K, I)
    r = oracle.moe_layer(bits(x), bits(router), None, q13, s13, q2, s2, E, K, 0, I, threads=2)
    xd = dequant_rows(r["x_q"], r["x_scale"])
    W13 = dequant_blocks(q13, s13)
    W2 = dequant_blocks(q2, s2)
    nv = int(r["num_valid"][0])
    sid, sexp = r["sorted_ids"][:nv], r["sorted_expert"]
    for p in range(nv):
        t, s = sid[p] & 0xFFFFFF, sid[p] >> 24
        if t >= T:
            continue
        e = sexp[p // 64]
        gu = W13[e] @ xd[t]
        g, u = gu[:I].astype(np.float32), gu[I:].astype(np.float32)
        h_ref = g / (1 + np.exp(-g.astype(np.float64))) * u
        h = val(r["h_bf16"][p]).astype(np.float64)
        assert np.max(np.abs(h - h_ref)) <= 2.0 ** -7 * np.max(np.abs(h_ref)) + 1e-6
        hd = dequant_rows(r["h_q"][p:p + 1], r["h_scale"][p:p + 1])[0]
        np.testing.assert_allclose(r["partial"][t * K + s], W2[e] @ hd, rtol=1e-5, atol=1e-7)
    out_ref = np.zeros((T, H))
    for t in range(T):
        for s in range(K):
            out_ref[t] += r["topk_weights"][t, s] * r["partial"][t * K + s].astype(np.float64)
    np.testing.assert_allclose(r["out_f32"], out_ref, rtol=1e-5, atol=1e-7)
    np.testing.assert_array_equal(r["out"], bits(r["out_f32"]))


def test_token_major_and_sorted_drivers_agree():
    T, H, E, K, I = 12, 256, 4, 2, 128
    x, router, _, _, q13, s13, q2, s2 = make(T, H, E, K, I, seed=1)
    r = oracle.moe_layer(bits(x), bits(router), None, q13, s13, q2, s2, E, K, 0, I, threads=2)
    tok = np.array([0, 5, 11], np.int64)
    out_f, out = oracle.moe_tokens(r["x_q"], r["x_scale"], q13, s13, q2, s2, r["topk_ids"],
                                   r["topk_weights"], tok, H, I, threads=2)
    np.testing.assert_array_equal(out_f, r["out_f32"][tok])
    np.testing.assert_array_equal(out, r["out"][tok])


def test_single_expert_layer_is_the_swiglu_ffn():
    T, H, E, K, I = 8, 512, 1, 1, 256
    x, router, w13, w2, q13, s13, q2, s2 = make(T, H, E, K, I, seed=2)
    r = oracle.moe_layer(bits(x), bits(router), None, q13, s13, q2, s2, E, K, 0, I, threads=2)
    assert np.all(r["topk_ids"] == 0) and np.all(r["topk_weights"] == 1.0)
    xt = torch.from_numpy(x.astype(np.float64))
    wg, wu = torch.from_numpy(w13[0, :I].astype(np.float64)), torch.from_numpy(w13[0, I:].astype(np.float64))
    y = torch.nn.functional.silu(xt @ wg.T) * (xt @ wu.T) @ torch.from_numpy(w2[0].astype(np.float64)).T
    # FP8 quantisation of x, the weights and h (three E4M3 roundings, 3-bit
    # mantissas) is the only difference from the unquantised textbook FFN
    def cos(a, b):
        a, b = a.reshape(-1), b.reshape(-1)
        return float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))
    assert cos(r["out_f32"].astype(np.float64), y.numpy()) > 0.995
    assert oracle.max_abs_rel(r["out_f32"], y.numpy()) < 0.1
    # while gate and up swapped, or the down weights transposed per block, are far off
    bad = (torch.nn.functional.silu(xt @ wu.T) * (xt @ wg.T)) @ torch.from_numpy(w2[0].astype(np.float64)).T
    assert cos(r["out_f32"].astype(np.float64), bad.numpy()) < 0.9


def test_gate_up_rows_equals_the_sorted_pass_on_a_selection():
    """gate_up_rows (the row-sampled driver the GPU parity test uses at large T)
    returns exactly the sorted pass's rows, in the order asked."""
    T, H, E, K, I = 40, 256, 6, 3, 128
    x, router, _, _, q13, s13, q2, s2 = make(T, H, E, K, I, seed=3)
    r = oracle.moe_layer(bits(x), bits(router), None, q13, s13, q2, s2, E, K, 0, I, threads=2)
    nv = int(r["num_valid"][0])
    rows = np.array([nv - 1, 0, 5, 64, 63, nv // 2], dtype=np.int64)
    hq, hs = oracle.gate_up_rows(r["x_q"], r["x_scale"], q13, s13, r["sorted_ids"], r["sorted_expert"],
                                 rows, T, H, I, threads=2)
    valid = (r["sorted_ids"][rows] & 0xFFFFFF) < T
    np.testing.assert_array_equal(hq[valid], r["h_q"][rows][valid])
    np.testing.assert_array_equal(hs[valid].view(np.uint32), r["h_scale"][rows][valid].view(np.uint32))
