"""Host restatements of the kernels' data layouts (CPU).

The packed weight layout and the tiled h layout are pure permutations; these
tests pin the host restatements against element-by-element definitions
(independent index arithmetic) so the GPU tests that rely on them compare like
with like.
"""
import numpy as np

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
