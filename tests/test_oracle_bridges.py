"""Pins the oracle functions behind the per-operation bridge tests (CPU).

Each bridge contract is a re-cut of stages the oracle already computes on the
layer path, so each new function is checked against an independent
formulation of the same numbers:

* stage1_routes (per-route gate/up before SiLU) against dense float64 numpy
  products of the dequantised operands, and, composed with silu_mul_quant,
  bit-exactly against the fused sorted-order gate_up (whose h is pinned by
  tests/test_oracle_gemm.py);
* silu_mul_quant against closed forms (a zero row quantises to zero codes with
  the 1e-10 floor scale; a row whose maximum |h| is 448 * s has scale s) and
  the composition above;
* down_reduce_routes bit-exactly against the sorted-order down_combine;
* shared_gate_append against top-k's shared-expert slot (router row E);
* stage2_split_halves: the two halves sum to the down partial, and each half
  equals a dense product over its own K range.
"""
import numpy as np

import oracle

bits = oracle.bf16_from_f32
val = oracle.f32_from_bf16


def quantised_case(T=6, H=256, E=5, K=3, I=256, seed=11):
    rng = np.random.default_rng(seed)
    x = bits(rng.standard_normal((T, H)).astype(np.float32))
    w13 = (rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float32)
    w2 = (rng.standard_normal((E, H, I)) * 0.02).astype(np.float32)
    q13, s13 = oracle.quant_blocks_f32(w13, threads=2)
    q2, s2 = oracle.quant_blocks_f32(w2, threads=2)
    x_q, x_s = oracle.quant_rows_bf16(x)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    wts = rng.random((T, K)).astype(np.float32)
    wts /= wts.sum(axis=1, keepdims=True)
    return x, x_q, x_s, q13, s13, q2, s2, ids, wts


def dequant_blocks(q, s):
    table = oracle.e4m3_table().astype(np.float64)
    return table[q] * np.repeat(np.repeat(s.astype(np.float64), 128, axis=1), 128, axis=2)


def dequant_rows(q, s):
    table = oracle.e4m3_table().astype(np.float64)
    return table[q] * np.repeat(s.astype(np.float64), 128, axis=1)


def test_stage1_routes_matches_dense_float64():
    x, x_q, x_s, q13, s13, q2, s2, ids, wts = quantised_case()
    T, K = ids.shape
    I = q13.shape[1] // 2
    out = oracle.stage1_routes(x_q, x_s, q13, s13, ids, q13.shape[0], I, threads=2)
    W13 = dequant_blocks(q13, s13)
    xd = dequant_rows(x_q, x_s)
    for r in range(T * K):
        ref = W13[ids.reshape(-1)[r]] @ xd[r // K]
        np.testing.assert_allclose(out[r], ref, rtol=2e-6, atol=1e-7)
    bad = ids.copy()
    bad[0, 0] = 99  # an expert id out of range gives a zero row
    assert not np.any(oracle.stage1_routes(x_q, x_s, q13, s13, bad, q13.shape[0], I, threads=2)[0])


def test_silu_mul_quant_of_stage1_equals_the_fused_gate_up():
    x, x_q, x_s, q13, s13, q2, s2, ids, wts = quantised_case()
    T, K = ids.shape
    E, I, H = q13.shape[0], q13.shape[1] // 2, x_q.shape[1]
    hq, hs = oracle.silu_mul_quant(oracle.stage1_routes(x_q, x_s, q13, s13, ids, E, I, threads=2))
    # the fused path over one-row "blocks" in route order
    sid = np.array([(r % K) << 24 | (r // K) for r in range(T * K)], dtype=np.int32)
    fq, fs, _ = oracle.gate_up(x_q, x_s, q13, s13, sid, ids.reshape(-1), T * K, T, H, I, threads=2, bm=1)
    np.testing.assert_array_equal(hq, fq)
    np.testing.assert_array_equal(hs.view(np.uint32), fs.view(np.uint32))


def test_silu_mul_quant_closed_forms():
    I = 256
    q, s = oracle.silu_mul_quant(np.zeros((1, 2 * I), np.float32))
    assert not np.any(q)
    np.testing.assert_array_equal(s, np.float32(1e-10) * np.float32(np.frombuffer(
        np.uint32(0x3B124925).tobytes(), np.float32)[0]))
    # a large gate makes silu(g) == g exactly in fp32: h = bf16(g * u); with
    # g * u = 448 * 2^-4 the row maximum is 28 and the scale 28 * (1/448)
    gu = np.zeros((1, 2 * I), np.float32)
    gu[0, 0], gu[0, I] = 112.0, 0.25
    q, s = oracle.silu_mul_quant(gu)
    inv448 = np.frombuffer(np.uint32(0x3B124925).tobytes(), np.float32)[0]
    assert s[0, 0] == np.float32(28.0) * inv448
    assert q[0, 0] == 0x7E  # 448 in e4m3 (the group maximum maps to the top code)
    assert not np.any(q[0, 1:])


def test_down_reduce_routes_equals_sorted_down_combine():
    x, x_q, x_s, q13, s13, q2, s2, ids, wts = quantised_case()
    T, K = ids.shape
    E, I, H = q13.shape[0], q13.shape[1] // 2, x_q.shape[1]
    hq, hs = oracle.silu_mul_quant(oracle.stage1_routes(x_q, x_s, q13, s13, ids, E, I, threads=2))
    out_f, out = oracle.down_reduce_routes(hq, hs, q2, s2, ids, wts, E, threads=2)
    sid, sexp, nv, _ = oracle.sort(ids, E)
    # h in sorted order from the route-major rows
    t, s = sid & 0xFFFFFF, sid >> 24
    valid = t < T
    h_sorted = np.zeros((sid.size, I), np.uint8)
    s_sorted = np.zeros((sid.size, I // 128), np.float32)
    h_sorted[valid] = hq[t[valid] * K + s[valid]]
    s_sorted[valid] = hs[t[valid] * K + s[valid]]
    _, ref_f, ref = oracle.down_combine(h_sorted, s_sorted, q2, s2, sid, sexp, nv[0], wts, T, H, I, threads=2)
    np.testing.assert_array_equal(out, ref)
    np.testing.assert_array_equal(out_f.view(np.uint32), ref_f.view(np.uint32))


def test_shared_gate_append_equals_topk_shared_slot():
    rng = np.random.default_rng(5)
    T, H, E, K = 7, 512, 16, 3
    x = bits(rng.standard_normal((T, H)).astype(np.float32))
    router = bits((rng.standard_normal((E + 1, H)) * 0.02).astype(np.float32))
    logits = oracle.router_logits(x, router)
    ids, wts = oracle.topk(logits, None, E, K, 1)
    out_ids, out_w = oracle.shared_gate_append(x, router[E], ids[:, :K], wts[:, :K], E)
    np.testing.assert_array_equal(out_ids, ids)
    np.testing.assert_array_equal(out_w.view(np.uint32), wts.view(np.uint32))


def test_stage2_split_halves_sum_to_the_partial():
    x, x_q, x_s, q13, s13, q2, s2, ids, wts = quantised_case(I=512)
    T, K = ids.shape
    E, I, H = q13.shape[0], q13.shape[1] // 2, x_q.shape[1]
    hq, hs = oracle.silu_mul_quant(oracle.stage1_routes(x_q, x_s, q13, s13, ids, E, I, threads=2))
    experts = ids.reshape(-1)
    p0, p1 = oracle.stage2_split_halves(hq, hs, q2, s2, experts)
    W2 = dequant_blocks(q2, s2)
    hd = dequant_rows(hq, hs)
    for r in range(T * K):
        ref0 = W2[experts[r]][:, : I // 2] @ hd[r, : I // 2]
        ref1 = W2[experts[r]][:, I // 2:] @ hd[r, I // 2:]
        np.testing.assert_allclose(p0[r], ref0, rtol=1e-9, atol=1e-12)
        np.testing.assert_allclose(p1[r], ref1, rtol=1e-9, atol=1e-12)
