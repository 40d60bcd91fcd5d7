"""Pins the oracle's scalar numerics against independent implementations.

bf16 and E4M3 conversions are checked against torch's own dtype conversions
(library code, not this build's), the contract exp against math.exp within a
stated ulp bound, and the 1x128 / 128x128 quantisers against closed-form
cases and a numpy restatement that uses torch's E4M3 encoder.
"""
import math
import struct

import numpy as np
import pytest
import torch

import oracle


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def ulp_distance(a: float, b: float) -> int:
    ia = struct.unpack("<i", struct.pack("<f", a))[0]
    ib = struct.unpack("<i", struct.pack("<f", b))[0]
    ia = ia if ia >= 0 else -(ia & 0x7FFFFFFF)
    ib = ib if ib >= 0 else -(ib & 0x7FFFFFFF)
    return abs(ia - ib)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 3,
        rng.standard_normal(2000).astype(np.float32) * 1e-30,
        # exact halfway cases between bf16 neighbours, both parities
        (np.arange(1, 2000, dtype=np.uint32) * 0x10000 + 0x8000).view(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, 3.3895314e38, 1e-45], np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(oracle.bf16_from_f32(x), ref)
    L = oracle.lib()
    for v in x[::37]:
        assert L.orc_bf16_from_f32(float(v)) == oracle.bf16_from_f32(np.array([v]))[0]


def test_e4m3_decode_table_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    got = oracle.e4m3_table()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert nan.sum() == 2  # 0x7f and 0xff only
    np.testing.assert_array_equal(got[~nan], ref[~nan])
    # closed forms: max finite, min normal, min subnormal
    assert got[0x7E] == 448.0 and got[0x08] == 2.0 ** -6 and got[0x01] == 2.0 ** -9


def test_e4m3_encode_matches_torch_and_saturates():
    L = oracle.lib()
    rng = np.random.default_rng(2)
    table = oracle.e4m3_table()
    vals = table[:0x7F].astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    x = np.concatenate([
        rng.uniform(-460, 460, 4000), rng.standard_normal(4000) * 0.01,
        mids, -mids, np.nextafter(mids.astype(np.float32), np.float32(0)),
        np.nextafter(mids.astype(np.float32), np.float32(1000)),
    ]).astype(np.float32)
    got = np.array([L.orc_e4m3_from_f32(float(v)) for v in x], dtype=np.uint8)
    inside = np.abs(x) <= 448
    ref = torch.from_numpy(x[inside]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(got[inside], ref)
    assert np.all((got[~inside] & 0x7F) == 0x7E)
    assert L.orc_e4m3_from_f32(float("inf")) == 0x7E
    assert L.orc_e4m3_from_f32(float("-inf")) == 0xFE
    assert L.orc_e4m3_from_f32(float("nan")) & 0x7F == 0x7F


def test_contract_exp_is_accurate_and_exact_at_zero():
    L = oracle.lib()
    assert L.orc_exp(0.0) == 1.0
    assert L.orc_exp(-100.0) == 0.0
    assert math.isinf(L.orc_exp(100.0))
    xs = np.linspace(-87.0, 88.0, 40001, dtype=np.float32)
    worst = 0
    for x in xs:
        got = L.orc_exp(float(x))
        want = f32(math.exp(float(x)))
        worst = max(worst, ulp_distance(got, want))
    assert worst <= 2, worst
    # silu / sigmoid are the textbook forms around the contract exp
    for g in (-20.0, -3.5, -0.25, 0.0, 0.5, 4.0, 30.0):
        assert abs(L.orc_silu(g) - g / (1 + math.exp(-g))) <= 4e-7 * max(1.0, abs(g))
        assert abs(L.orc_sigmoid(g) - 1 / (1 + math.exp(-g))) <= 3e-7


def _quant_rows_reference(x: np.ndarray):
    """Reference rule restated in numpy with torch's E4M3 encoder."""
    c = np.uint32(0x3B124925).view(np.float32)
    g = x.reshape(x.shape[0], -1, 128)
    amax = np.maximum(np.float32(1e-10), np.abs(g).max(axis=2)).astype(np.float32)
    scale = (amax * c).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    v = (g * inv[:, :, None]).astype(np.float32)
    q = torch.from_numpy(np.clip(v, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return q.reshape(x.shape), scale


def test_activation_quant_closed_forms_and_reference_rule():
    # closed forms: a group whose max is 448 gets scale 448 * RN(1/448) and the
    # max maps back to 448; an all-zero group gets the 1e-10 floor and zeros
    row = np.zeros((1, 256), np.float32)
    row[0, 3] = 448.0
    row[0, 7] = -224.0
    q, s = oracle.quant_rows_bf16(oracle.bf16_from_f32(row))
    assert s[0, 0] == np.float32(448.0) * np.uint32(0x3B124925).view(np.float32)
    assert q[0, 3] == 0x7E and q[0, 7] == 0xF6  # -224 = -1.75 * 2^7
    assert s[0, 1] == np.float32(1e-10) * np.uint32(0x3B124925).view(np.float32)
    assert not q[0, 128:].any()
    rng = np.random.default_rng(4)
    x = oracle.f32_from_bf16(oracle.bf16_from_f32(rng.standard_normal((16, 512)).astype(np.float32)))
    q, s = oracle.quant_rows_bf16(oracle.bf16_from_f32(x))
    q_ref, s_ref = _quant_rows_reference(x)
    np.testing.assert_array_equal(s, s_ref)
    np.testing.assert_array_equal(q, q_ref)


def test_weight_block_quant_matches_rule_per_block():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((2, 256, 384)) * 0.02).astype(np.float32)
    w[1, 128:, :128] *= 50
    q, s = oracle.quant_blocks_f32(w, threads=2)
    for g in range(2):
        for bn in range(2):
            for bk in range(3):
                blk = w[g, bn * 128:(bn + 1) * 128, bk * 128:(bk + 1) * 128]
                q_ref, s_ref = _quant_rows_reference(blk.reshape(1, -1))
                assert s[g, bn, bk] == s_ref[0].max()  # one scale per block
                # same rule, one amax over the whole block
                c = np.uint32(0x3B124925).view(np.float32)
                scale = np.float32(max(np.float32(1e-10), np.abs(blk).max()) * c)
                assert s[g, bn, bk] == scale
                inv = np.float32(1.0) / scale
                ref = torch.from_numpy(np.clip(blk * inv, -448, 448).astype(np.float32)).to(
                    torch.float8_e4m3fn).view(torch.uint8).numpy()
                np.testing.assert_array_equal(q[g, bn * 128:(bn + 1) * 128, bk * 128:(bk + 1) * 128], ref)
