"""Pins the low-bit oracle (CPU): reference shape KATs and round-trip bounds, numpy's
packbits as the bitstream routine, per-element brute force."""

from __future__ import annotations

import numpy as np

from oracle import lowbit as ol


def test_reference_int3_roundtrip_kat():
    # reference tests/test_qstore_int3.py:10-21
    rng = np.random.default_rng(0)
    W = rng.standard_normal((5, 17)).astype(np.float32)
    packed, scales = ol.quant_row_int3(W, G=4)
    assert packed.dtype == np.uint8 and packed.shape == (5, (17 * 3 + 7) // 8)
    assert scales.shape == (5, 5)
    deq = ol.dequant(packed, scales, 17, 3, 4)
    step = np.repeat(scales, 4, axis=1)[:, :17]
    assert np.all(np.abs(W - deq) <= step * 0.51 + 1e-6)


def test_reference_int2_roundtrip_kat():
    # reference tests/test_qstore_int2.py:10-23
    rng = np.random.default_rng(0)
    W = rng.standard_normal((5, 17)).astype(np.float32)
    packed, scales = ol.quant_row_int2(W, G=4)
    assert packed.shape == (5, (17 * 2 + 7) // 8) and scales.shape == (5, 5)
    deq = ol.dequant(packed, scales, 17, 2, 4)
    ratio = deq / np.repeat(scales, 4, axis=1)[:, :17]
    r = np.round(ratio).astype(np.int8)
    assert np.allclose(ratio, r, atol=1e-6) and set(np.unique(r)).issubset({-1, 0, 1})


def test_bitstream_brute_force():
    rng = np.random.default_rng(1)
    for bits in (2, 3):
        codes = rng.integers(0, 1 << bits, size=(4, 37), dtype=np.uint8)
        packed = ol.pack_codes(codes, bits)
        for n in range(4):
            for k in range(37):
                v = 0
                for i in range(bits):
                    bit = k * bits + i
                    v |= ((int(packed[n, bit // 8]) >> (bit % 8)) & 1) << i
                assert v == codes[n, k]
        assert np.array_equal(ol.unpack_codes(packed, 37, bits), codes)


def test_dequant_closed_form_and_zero_points():
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 8, size=(3, 128), dtype=np.uint8)
    packed = ol.pack_codes(codes, 3)
    s = rng.uniform(0.5, 1.5, size=(3, 2)).astype(np.float16)
    z = rng.uniform(0, 7, size=(3, 2)).astype(np.float16)
    w = ol.dequant(packed, s, 128, 3, 64, zeros=z)
    for n in range(3):
        for k in range(128):
            g = k // 64
            exp = np.float32(np.float32(codes[n, k]) - np.float32(z[n, g])) * np.float32(s[n, g])
            assert w[n, k] == exp
    # symmetric default: offset 4 (int3) / 1 (int2)
    assert np.array_equal(ol.dequant(packed, s.astype(np.float32), 128, 3, 64),
                          ((codes.astype(np.float32) - 4.0) * np.repeat(s.astype(np.float32), 64, axis=1)).astype(np.float32))


def test_asym_codec_roundtrip():
    rng = np.random.default_rng(3)
    W = rng.standard_normal((6, 128)).astype(np.float32)
    for bits in (2, 3):
        packed, s, z = ol.quant_row_asym(W, bits, 64)
        deq = ol.dequant(packed, s, 128, bits, 64, zeros=z)
        step = np.repeat(s.astype(np.float32), 64, axis=1)
        assert np.all(np.abs(W - deq) <= step * 0.51 + 2e-3 * np.abs(W).max())
