"""Oracle: int8 row-scaled (qrow) codec, dequant and matmul contracts (numpy, CPU).

Restates (reference paths relative to /root/reference):
* ``quant_row_int8``    -- ``_quant_row_int8``       src/mrun/engine/kernels/qstore_build.py:496-501
* ``dequant_qrow``      -- ``_dequant_qrow``          src/mrun/engine/kernels/qstore.py:385-399
* ``qrow_matmul_f32``   -- ``QStore.matmul`` (fp32)   qstore.py:1082-1092
* ``qrow_matmul_w8a16`` -- ``_qrow_w8a16_kernel`` / ``dequantized_reference_matmul``
                           src/mrun/engine/kernels/dense_qstore_cuda.py:467-512, 1003-1013
* ``qrow_swiglu``       -- ``fused_qrow_swiglu_reference`` dense_qstore_cuda.py:1037-1050

Pinned by (tests/test_oracle_qrow.py):
* the reference's own KATs: test_dense_qstore_cuda.py:72-96 (compact qrow, exact) and the
  paired-SwiGLU KAT operands of :99-124;
* ``round_bf16`` / ``round_f16`` against torch's CPU casts (library routine) incl. ties,
  subnormals, inf and NaN;
* ``quant_row_int8`` against brute force per element (ties to even, the zero row -> 1);
* matmuls against float64 brute force on small shapes, row-stable vs batched equality.
"""

from __future__ import annotations

import numpy as np


def round_bf16(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 round-to-nearest-even, returned widened back to fp32 (NaN kept)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out = out.copy()
        out[nan] = np.float32("nan")
    return out


def round_f16(a: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 (IEEE RNE), widened back to fp32."""
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def quant_row_int8(W: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric int8: ``s = max|W_row|/127`` (0 -> 1), ``q = clip(rint(W/s), ±127)``.

    qstore_build.py:496-501.  Division and rounding in fp32 (numpy ``np.round`` is
    round-half-to-even).
    """
    W = np.asarray(W, dtype=np.float32)
    scale = np.abs(W).max(axis=1, keepdims=True) / np.float32(127.0)
    scale = np.where(scale == 0.0, np.float32(1.0), scale).astype(np.float32)
    q = np.round(W / scale).clip(-127, 127).astype(np.int8)
    return q, scale[:, 0].astype(np.float32)


def dequant_qrow(q: np.ndarray, sc: np.ndarray) -> np.ndarray:
    """``float32(q) * sc[:, None]`` -- exact widen, one IEEE single multiply (qstore.py:396-399)."""
    return np.asarray(q).astype(np.float32) * np.asarray(sc, dtype=np.float32)[:, None]


def qrow_weight(q: np.ndarray, sc: np.ndarray, dtype: str = "fp32") -> np.ndarray:
    """``QStore.weight``: fp32 dequant then narrow to the compute dtype (qstore.py:1076-1077)."""
    W = dequant_qrow(q, sc)
    if dtype == "bf16":
        return round_bf16(W)
    if dtype == "fp16":
        return round_f16(W)
    return W


def qrow_matmul_f32(q: np.ndarray, sc: np.ndarray, x: np.ndarray) -> np.ndarray:
    """``x.float() @ W.T`` in fp32 (QStore.matmul with an fp32 compute dtype)."""
    W = dequant_qrow(q, sc)
    return np.asarray(x, dtype=np.float32) @ W.T


def qrow_matmul_w8a16(
    q: np.ndarray, sc: np.ndarray, x: np.ndarray, dtype: str = "bf16"
) -> np.ndarray:
    """W8A16: ``W = dtype(float(q)*s)``, fp32-exact products, fp32 sum, output in ``dtype``.

    ``x`` must already hold values representable in ``dtype`` (as float32).  The sum is
    formed in float64 and rounded once to fp32 before the final narrowing; the reference's
    accumulation order is an fp32 tile order, so this is compared by tolerance.
    """
    rnd = round_bf16 if dtype == "bf16" else round_f16
    W = rnd(dequant_qrow(q, sc)).astype(np.float64)
    acc = (np.asarray(x, dtype=np.float64) @ W.T).astype(np.float32)
    return rnd(acc)


def silu_f32(g: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        sig = (np.float32(1.0) / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
    return (g * sig).astype(np.float32)


def qrow_swiglu(
    gq: np.ndarray, gs: np.ndarray, uq: np.ndarray, us: np.ndarray, x: np.ndarray
) -> np.ndarray:
    """``bf16(float(bf16(silu(g))) * float(u))`` with g, u the bf16 W8A16 projections
    (dense_qstore_cuda.py:1037-1050)."""
    g = qrow_matmul_w8a16(gq, gs, x)
    u = qrow_matmul_w8a16(uq, us, x)
    s = round_bf16(silu_f32(g))
    return round_bf16(s * u)


def rel_l2(got: np.ndarray, ref: np.ndarray) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = float(np.linalg.norm(ref))
    num = float(np.linalg.norm(got - ref))
    return num / den if den > 0 else num
