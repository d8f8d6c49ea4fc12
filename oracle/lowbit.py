"""Oracle: packed int3 / int2 QStore codecs, dequant and matmul (numpy, CPU).

Restates (reference paths relative to /root/reference):
* ``pack_codes``          -- ``_pack_int3_codes`` / ``_pack_int2_codes``
                             src/mrun/engine/kernels/qstore_int3.py:30-39, qstore_int2.py:24-33
* ``quant_row_int3``      -- ``_quant_row_int3``  qstore_int3.py:42-56
* ``quant_row_int2``      -- ``_quant_row_int2``  qstore_int2.py:36-63
* ``dequant``             -- ``_dequant_int3`` / ``_dequant_int2`` qstore.py:441-456
                             (``(code - offset) * scale``, fp32), extended to a per-group
                             zero point for the asymmetric G=64 variant
* ``lowbit_matmul``       -- ``QStoreInt3.matmul`` / ``QStoreInt2.matmul`` qstore.py:1318-1341,
                             1451-1474 (x in fp32, chunked dequant, ``x @ W.T``)
* ``quant_row_asym``      -- builder convention for the asymmetric G=64 fp16 scale/zero
                             variant.  The reference has this codec only
                             through MLX (third-party ``mlx.core.quantize``, mlx 0.32.3,
                             src/mrun/decompiler/mlx_lowbit.py:99-105, 300-348), which is not
                             installed: **parity unpinned** for the affine variant's codec
                             beyond the closed form and round-trip checks below.

Pinned by (tests/test_oracle_lowbit.py): the reference's shape KATs and round-trip bounds
(test_qstore_int3.py:10-21, test_qstore_int2.py:10-23), numpy ``packbits`` as the library
routine behind the bitstream, per-element brute-force unpacking, and golden vectors from
the reference codecs when present under tests/golden/.
"""

from __future__ import annotations

import numpy as np

OFFSET = {3: 4.0, 2: 1.0}


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """uint codes [out, in] -> LSB-first row bitstreams [out, ceil(in*bits/8)] uint8."""
    codes = np.asarray(codes, dtype=np.uint8)
    out, inn = codes.shape
    b = ((codes[:, :, None] >> np.arange(bits, dtype=np.uint8)) & 1).reshape(out, inn * bits)
    row_bits = inn * bits
    pad = ((row_bits + 7) // 8) * 8 - row_bits
    if pad:
        b = np.concatenate([b, np.zeros((out, pad), np.uint8)], axis=1)
    return np.packbits(b, axis=1, bitorder="little")


def unpack_codes(packed: np.ndarray, inn: int, bits: int) -> np.ndarray:
    b = np.unpackbits(np.asarray(packed, np.uint8), axis=1, bitorder="little")[:, : inn * bits]
    b = b.reshape(packed.shape[0], inn, bits).astype(np.uint8)
    code = np.zeros((packed.shape[0], inn), np.uint8)
    for i in range(bits):
        code |= b[:, :, i] << i
    return code


def quant_row_int3(W: np.ndarray, G: int = 128):
    W = np.asarray(W, np.float32)
    out, inn = W.shape
    ng = (inn + G - 1) // G
    scales = np.empty((out, ng), np.float32)
    q = np.empty((out, inn), np.int8)
    for g in range(ng):
        c0, c1 = g * G, min((g + 1) * G, inn)
        blk = W[:, c0:c1]
        s = np.abs(blk).max(axis=1) / 3.0
        s = np.where(s == 0.0, 1.0, s).astype(np.float32)
        scales[:, g] = s
        q[:, c0:c1] = np.round(blk / s[:, None]).clip(-3, 3).astype(np.int8)
    return pack_codes((q + 4).astype(np.uint8), 3), scales


def quant_row_int2(W: np.ndarray, G: int = 128):
    W = np.asarray(W, np.float32)
    out, inn = W.shape
    ng = (inn + G - 1) // G
    scales = np.empty((out, ng), np.float32)
    q = np.empty((out, inn), np.int8)
    for g in range(ng):
        c0, c1 = g * G, min((g + 1) * G, inn)
        blk = W[:, c0:c1]
        a = np.abs(blk)
        active = a >= (0.7 * a.mean(axis=1))[:, None]
        count = active.sum(axis=1)
        weighted = (a * active).sum(axis=1)
        s = np.divide(weighted, count, out=np.ones_like(weighted, dtype=np.float32), where=count > 0)
        s = np.where(s == 0.0, 1.0, s).astype(np.float32)
        scales[:, g] = s
        q[:, c0:c1] = np.where(active, np.sign(blk), 0).astype(np.int8)
    return pack_codes((q + 1).astype(np.uint8), 2), scales


def quant_row_asym(W: np.ndarray, bits: int, G: int = 64):
    """Affine per-group codec: s = (max-min)/(2^b-1), z = -min/s (fp16), code = clip(rint(w/s + z))."""
    W = np.asarray(W, np.float32)
    out, inn = W.shape
    ng = inn // G
    lvl = (1 << bits) - 1
    blk = W.reshape(out, ng, G)
    lo, hi = blk.min(axis=2), blk.max(axis=2)
    s = ((hi - lo) / lvl).astype(np.float32)
    s = np.where(s == 0, np.float32(1.0), s).astype(np.float16)
    z = (-lo / s.astype(np.float32)).astype(np.float16)
    code = np.clip(np.rint(blk / s.astype(np.float32)[..., None] + z.astype(np.float32)[..., None]), 0, lvl)
    return pack_codes(code.reshape(out, inn).astype(np.uint8), bits), s, z


def dequant(packed, scales, inn: int, bits: int, G: int, zeros=None, offset: float | None = None) -> np.ndarray:
    """``(float(code) - zero) * scale`` in fp32 (reference order: subtract, then multiply)."""
    code = unpack_codes(packed, inn, bits).astype(np.float32)
    col = lambda a: np.repeat(np.asarray(a, np.float32), G, axis=1)[:, :inn]  # noqa: E731
    z = col(zeros) if zeros is not None else np.float32(OFFSET[bits] if offset is None else offset)
    return ((code - z).astype(np.float32) * col(scales)).astype(np.float32)


def lowbit_matmul(packed, scales, x, inn: int, bits: int, G: int, zeros=None, offset=None) -> np.ndarray:
    W = dequant(packed, scales, inn, bits, G, zeros, offset)
    x2 = np.asarray(x, np.float32).reshape(-1, inn)
    y = (x2.astype(np.float64) @ W.T.astype(np.float64)).astype(np.float32)
    return y.reshape(*np.asarray(x).shape[:-1], W.shape[0])
