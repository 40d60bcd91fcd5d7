"""Host restatements of the kernels' data layouts (CPU).

The packed weight layout and the AITER 16x16 shuffle the reference's kernels
consume are pure permutations; these tests pin the host restatements against
element-by-element definitions (independent index arithmetic, and the
reference's own inverse of the shuffle) so the GPU tests that rely on them
compare like with like.
"""
import numpy as np
import pytest
import torch

from netra_moe import weights as W


def test_pack_tiles_host_is_the_documented_permutation():
    rng = np.random.default_rng(0)
    G, N, K = 2, 32, 256
    q = rng.integers(0, 256, size=(G, N, K), dtype=np.uint8)
    p = W.pack_tiles_host(q).reshape(-1)
    for g in range(G):
        for n in range(0, N, 5):
            for k in range(0, K, 7):
                tile = (g * (N // 16) + n // 16) * (K // 128) + k // 128
                lane = ((k % 128) // 32) * 16 + n % 16
                half = (k % 32) // 16
                off = tile * 2048 + half * 1024 + lane * 16 + k % 16
                assert p[off] == q[g, n, k]
    assert sorted(p.tolist()) == sorted(q.reshape(-1).tolist())


def test_pack_tiles_gate_up_interleaves_the_row_tiles():
    # W13 [G, 2I, K]: logical row tile t (gate t < I/16, up t >= I/16) is stored at
    # 2t (gate) or 2(t - I/16) + 1 (up); inside a tile the plain layout holds
    rng = np.random.default_rng(1)
    G, N, K = 2, 64, 256  # I = 32: two gate tiles, two up tiles
    q = rng.integers(0, 256, size=(G, N, K), dtype=np.uint8)
    p = W.pack_tiles_host(q, gate_up=True).reshape(-1)
    half = N // 32
    for g in range(G):
        for n in range(0, N, 3):
            for k in range(0, K, 11):
                t = n // 16
                pt = 2 * t if t < half else 2 * (t - half) + 1
                tile = (g * (N // 16) + pt) * (K // 128) + k // 128
                lane = ((k % 128) // 32) * 16 + n % 16
                off = tile * 2048 + ((k % 32) // 16) * 1024 + lane * 16 + k % 16
                assert p[off] == q[g, n, k]
    np.testing.assert_array_equal(W.unpack_tiles_host(p.reshape(G, N, K), gate_up=True), q)
    np.testing.assert_array_equal(W.unpack_tiles_host(W.pack_tiles_host(q)), q)


def _reference_unshuffle(shuffled: np.ndarray) -> np.ndarray:
    """The reference's inverse of the AITER 16x16 shuffle, as its capture tool
    states it (tools/benchmark/export_qwen36_dense_m1_capture.py:55-63):
    view(n/16, k/32, 2, 16, 16).permute(0, 3, 1, 2, 4), per matrix."""
    n, k = shuffled.shape
    return torch.from_numpy(shuffled).view(n // 16, k // 32, 2, 16, 16).permute(0, 3, 1, 2, 4) \
        .contiguous().view(n, k).numpy()


@pytest.mark.parametrize("n,k", [(16, 128), (64, 256), (96, 384)])
def test_aiter_shuffle_is_inverted_by_the_reference_unshuffle(n, k):
    rng = np.random.default_rng(n * 1000 + k)
    q = rng.integers(0, 256, size=(2, n, k), dtype=np.uint8)
    s = W.aiter_shuffle_host(q)
    for g in range(2):
        np.testing.assert_array_equal(_reference_unshuffle(s[g]), q[g])
    # the reference decode kernel's addressing: row tile * 32 KiB (k = 2048)
    # generalises to row tile * 16 k; lane (n % 16) * 16; 16-column fragment
    # ((k % 128) // 16) * 256 within a 128-column block (gate_up_mfma.inc:47-55)
    flat = s.reshape(2, -1)
    for (nn, kk) in [(0, 0), (n - 1, k - 1), (n // 2 + 3, 37), (5, k // 2 + 17)]:
        off = (nn // 16) * 16 * k + (kk // 32) * 512 + ((kk % 32) // 16) * 256 + (nn % 16) * 16 + kk % 16
        assert flat[1, off] == q[1, nn, kk]
