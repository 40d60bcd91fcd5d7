"""Pins the oracle's router, top-k and sort.

Router: known answers that only the contract's summation order produces
(slice membership 128 j + 8 s + i and the +8/+4/+2/+1 tree), exactness on
integer-valued inputs, and a bound against an fp64 dot product. Top-k: special
cases (equal logits, ties, one-hot, bias), an independent numpy selection and
fp64 softmax. Sort: a brute-force Python sort, invariants, and the
reference's own capacity figure (365 blocks for 768 tokens x 9 slots over 257
experts, manifests/gfx950/models/qwen36-35b-c64-fp8.json:43-49).
"""
import math

import numpy as np
import pytest

import oracle

bits = oracle.bf16_from_f32
val = oracle.f32_from_bf16


def logit(x, w):
    return float(val(oracle.router_logits(bits(np.asarray(x, np.float32)[None]),
                                          bits(np.asarray(w, np.float32)[None])))[0, 0])


def test_router_order_known_answers():
    A = 2.0 ** 25  # fp32 spacing at A is 4: +1 is absorbed
    # slice 0 = elements 0..7 (j = 0): A, six ones, -A -> the ones are absorbed
    x = np.zeros(128, np.float32); w = np.ones(128, np.float32)
    x[0], x[1:7], x[7] = A, 1.0, -A
    assert logit(x, w) == 0.0
    # the same six ones in slice 1 (elements 8..13) survive: the tree adds p1 = 6
    x = np.zeros(128, np.float32)
    x[0], x[8:14], x[7] = A, 1.0, -A
    assert logit(x, w) == 6.0
    # H = 256: slice 0 also owns elements 128..135 (j = 1), after 0..7
    x = np.zeros(256, np.float32); w = np.ones(256, np.float32)
    x[0], x[1:7], x[128] = A, 1.0, -A
    assert logit(x, w) == 0.0
    # tree: p0 = A, p8 = -A meet first (+8 step), so p1 = 6 survives;
    # a left-to-right fold over slices would absorb it
    x = np.zeros(128, np.float32)
    x[0], x[64], x[8:14] = A, -A, 1.0
    assert logit(x, w) == 6.0
    # slice 1 = A, slice 9 = -A: tree pairs them, slice 2's ones survive
    x = np.zeros(128, np.float32)
    x[8], x[72], x[16:22] = A, -A, 1.0
    assert logit(x, w) == 6.0


def test_router_exact_on_small_integers_and_bounded_otherwise():
    rng = np.random.default_rng(7)
    x = rng.integers(-3, 4, size=(8, 512)).astype(np.float32)
    w = rng.integers(-3, 4, size=(40, 512)).astype(np.float32)
    got = val(oracle.router_logits(bits(x), bits(w)))
    exact = x.astype(np.float64) @ w.T.astype(np.float64)  # every partial sum is an exact integer
    np.testing.assert_array_equal(got, val(bits(exact.astype(np.float32))))
    x = val(bits(rng.standard_normal((16, 2048)).astype(np.float32)))
    w = val(bits((rng.standard_normal((64, 2048)) * 0.02).astype(np.float32)))
    got = val(oracle.router_logits(bits(x), bits(w))).astype(np.float64)
    ref = x.astype(np.float64) @ w.T.astype(np.float64)
    mag = np.abs(x).astype(np.float64) @ np.abs(w).T.astype(np.float64)
    bound = 2048 * 2.0 ** -24 * mag + np.abs(ref) * 2.0 ** -8  # fp32 sum + bf16 rounding
    assert np.all(np.abs(got - ref) <= bound)


def _topk(logits_f32, E, K, S=0, bias=None):
    rows = E + S
    assert logits_f32.shape[1] == rows
    return oracle.topk(bits(logits_f32), bias, E, K, S)


def test_topk_special_cases():
    # all equal -> ids 0..k-1, weights exactly 1/k
    ids, w = _topk(np.full((1, 16), 0.5, np.float32), 16, 4)
    assert ids.tolist() == [[0, 1, 2, 3]] and w.tolist() == [[0.25] * 4]
    # ties resolve to the lower index, slots in descending logit
    l = np.array([[0.0, 2.0, 1.0, 2.0, 1.0, -1.0]], np.float32)
    ids, w = _topk(l, 6, 4)
    assert ids.tolist() == [[1, 3, 2, 4]]
    # one-hot dominance: weight 1 (exp underflows to 0 for the rest)
    l = np.full((1, 8), -100.0, np.float32); l[0, 5] = 100.0
    ids, w = _topk(l, 8, 2)
    assert ids[0, 0] == 5 and w[0, 0] == 1.0 and w[0, 1] == 0.0
    # bias shifts selection; weights use the biased logits
    l = np.zeros((1, 4), np.float32)
    ids, w = _topk(l, 4, 1, bias=np.array([0, 0, 0.5, 0], np.float32))
    assert ids.tolist() == [[2]] and w.tolist() == [[1.0]]
    # shared expert: id E at slot K, weight bf16(sigmoid(logit_E))
    l = np.zeros((1, 5), np.float32); l[0, 4] = 0.75
    ids, w = _topk(l, 4, 2, S=1)
    assert ids[0, 2] == 4
    assert w[0, 2] == val(bits(np.array([1 / (1 + math.exp(-0.75))], np.float32)))[0]


def test_topk_matches_independent_selection_and_softmax():
    rng = np.random.default_rng(9)
    E, K, T = 256, 8, 64
    l = val(bits(rng.standard_normal((T, E)).astype(np.float32)))
    # coarse logits force many ties
    l[: T // 2] = np.round(l[: T // 2] * 4) / 4
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    ids, w = _topk(l, E, K, bias=bias)
    z = (l + bias).astype(np.float32)
    for t in range(T):
        order = np.lexsort((np.arange(E), -z[t].astype(np.float64)))[:K]
        assert ids[t].tolist() == order.tolist()
        zs = z[t, order].astype(np.float64)
        p = np.exp(zs - zs[0]); p /= p.sum()
        assert np.max(np.abs(w[t] - p) / p) < 4e-7
        assert abs(float(w[t].astype(np.float64).sum()) - 1.0) < 1e-6


def _brute_sort(ids, Etot, bm=64):
    T, Ktot = ids.shape
    counts = [0] * Etot
    for e in ids.reshape(-1):
        counts[e] += 1
    rows, experts, tiles, pairs = [], [], [], []
    for e in range(Etot):
        mine = sorted((t, s) for t in range(T) for s in range(Ktot) if ids[t, s] == e)
        nb = -(-len(mine) // bm)
        first = len(experts)
        for b in range(nb):
            experts.append(e)
        for j in range(-(-len(mine) // 16)):
            tiles.append(first * (bm // 16) + j)
        pairs += list(range(first, first + nb, 2))  # consecutive blocks of e, two at a time
        ent = [(s << 24) | t for t, s in mine]
        rows += ent + [(Ktot << 24) | T] * (nb * bm - len(ent))
    return rows, experts, counts, tiles, pairs


@pytest.mark.parametrize("T,K,E,S,seed", [(16, 2, 16, 0, 1), (64, 8, 256, 1, 2), (5, 3, 7, 1, 3), (1, 8, 256, 1, 4)])
def test_sort_matches_brute_force(T, K, E, S, seed):
    rng = np.random.default_rng(seed)
    ids = np.stack([np.concatenate([rng.choice(E, K, replace=False), [E] * S]) for _ in range(T)]).astype(np.int32)
    Etot, Ktot = E + S, K + S
    sid, sexp, nv, counts, tmap, pmap = oracle.sort(ids, Etot, with_tiles=True)
    rows, experts, cnt, tiles, pairs = _brute_sort(ids, Etot)
    assert counts.tolist() == cnt and sum(cnt) == T * Ktot
    assert nv.tolist() == [len(rows), T * Ktot, len(tiles), len(pairs)]
    assert pmap[: len(pairs)].tolist() == pairs
    assert sid[: len(rows)].tolist() == rows
    assert np.all(sid[len(rows):] == ((Ktot << 24) | T))
    assert sexp[: len(experts)].tolist() == experts and np.all(sexp[len(experts):] == -1)
    assert tmap[: len(tiles)].tolist() == tiles
    # every route appears exactly once
    valid = sid[(sid & 0xFFFFFF) < T]
    assert sorted(((v >> 24), v & 0xFFFFFF) for v in valid.tolist()) == sorted(
        (s, t) for t in range(T) for s in range(Ktot))


def test_capacity_matches_reference_manifest():
    # qwen36-35b-c64-fp8.json: 768 routes-rows x 9 slots, 257 experts -> 365 x 64 = 23360
    assert oracle.capacity_blocks(768, 9, 257) == 365
    assert oracle.capacity_blocks(768, 9, 257) * 64 == 23360
