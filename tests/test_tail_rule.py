"""The prefill gate/up's work-item rule for expert tails, restated on the CPU
over the oracle's sorted layouts (netra-kernel_amd/csrc/kernels/
moe_gemm_lds.hip, gate_up_lds): item p covers the 64-row blocks pair_map[p]
and, when they belong to the same expert, pair_map[p] + 1; it also covers
block pair_map[p] + 2 when that block is its expert's last, holds at most 16
rows (its row 16 is padding) and follows the pair; the item of such a block
exits. Every block with rows must be computed by exactly one item, whatever
the routing."""
import numpy as np
import pytest

import oracle

BM = 64


def items_cover(sid: np.ndarray, sexp: np.ndarray, nv: np.ndarray, pmap: np.ndarray, T: int, Ktot: int):
    nblocks = int(nv[0]) // BM

    def pad(b: int, r: int) -> bool:  # row r of block b holds no route
        v = int(sid[b * BM + r])
        return v < 0 or (v & 0xFFFFFF) >= T or (v >> 24) >= Ktot

    def expert(b: int) -> int:
        return int(sexp[b]) if 0 <= b < nblocks else -1

    covered: list[int] = []
    absorbed: list[int] = []
    for p in range(int(nv[3])):
        b0 = int(pmap[p])
        e = expert(b0)
        two = expert(b0 + 1) == e
        if not two and expert(b0 - 1) == e and pad(b0, 16):
            continue  # the pair before it takes this tail
        covered.append(b0)
        if two:
            covered.append(b0 + 1)
            if expert(b0 + 2) == e and expert(b0 + 3) != e and pad(b0 + 2, 16):
                covered.append(b0 + 2)
                absorbed.append(b0 + 2)
    return nblocks, covered, absorbed


def _check(ids: np.ndarray, Etot: int):
    T, Ktot = ids.shape
    sid, sexp, nv, counts, _tmap, pmap = oracle.sort(ids, Etot, with_tiles=True)
    nblocks, covered, absorbed = items_cover(sid, sexp, nv, pmap, T, Ktot)
    with_rows = [b for b in range(nblocks) if not all(
        (int(sid[b * BM + r]) & 0xFFFFFF) >= T for r in range(BM))]
    assert sorted(covered) == with_rows  # each block with rows exactly once
    for b in absorbed:
        rows = sum(1 for r in range(BM) if (int(sid[b * BM + r]) & 0xFFFFFF) < T)
        assert 1 <= rows <= 16
        assert int(sexp[b - 1]) == int(sexp[b - 2]) == int(sexp[b])
    return absorbed


@pytest.mark.parametrize("T", [129, 144, 145, 272, 300])
def test_hot_routing_tails(T):
    """Every token on experts 0, 1 and the shared expert 2: T rows each."""
    ids = np.tile(np.array([0, 1, 2], np.int32), (T, 1))
    absorbed = _check(ids, 3)
    tail = T % BM
    blocks = -(-T // BM)
    expect = 3 if (blocks % 2 == 1 and blocks >= 3 and 1 <= tail <= 16) else 0
    assert len(absorbed) == expect


@pytest.mark.parametrize("seed", range(6))
def test_random_routing_tails(seed):
    rng = np.random.default_rng(seed)
    T, E, K = int(rng.integers(200, 3000)), int(rng.integers(4, 40)), 4
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
    ids = np.concatenate([ids, np.full((T, 1), E, np.int32)], axis=1)  # the shared expert at slot K
    _check(ids, E + 1)
