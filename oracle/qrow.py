"""Oracle: int8 row-scaled (qrow) codec, dequant and matmul contracts (numpy, CPU).

Restates (reference paths relative to /root/reference):
* ``quant_row_int8``    -- ``_quant_row_int8``       src/mrun/engine/kernels/qstore_build.py:496-501
* ``dequant_qrow``      -- ``_dequant_qrow``          src/mrun/engine/kernels/qstore.py:385-399
* ``qrow_matmul_f32``   -- ``QStore.matmul`` (fp32)   qstore.py:1082-1092
* ``qrow_matmul_w8a16`` -- ``_qrow_w8a16_kernel`` / ``dequantized_reference_matmul``
                           src/mrun/engine/kernels/dense_qstore_cuda.py:467-512, 1003-1013
* ``qrow_swiglu``       -- ``fused_qrow_swiglu_reference`` dense_qstore_cuda.py:1037-1050
* ``head_logits`` / ``qrow_top2`` -- the fused head's logits (W8A16 or fp32 weights, fp32
                           sums) and its block top-2 order, ``_qrow_w8a16_block_top2_kernel``
                           + ``_reduce_top2_blocks_kernel`` dense_qstore_cuda.py:578-674
* ``rerank_fp32``       -- ``_rerank_qrow_candidates_fp32`` dense_qstore_cuda.py:1189-1236

Pinned by (tests/test_oracle_qrow.py):
* the reference's own KATs: test_dense_qstore_cuda.py:72-96 (compact qrow, exact) and the
  paired-SwiGLU KAT operands of :99-124;
* ``round_bf16`` / ``round_f16`` against torch's CPU casts (library routine) incl. ties,
  subnormals, inf and NaN;
* ``quant_row_int8`` against brute force per element (ties to even, the zero row -> 1);
* matmuls against float64 brute force on small shapes, row-stable vs batched equality;
* ``qrow_top2`` / ``rerank_fp32``: the reference's KATs test_dense_qstore_cuda.py:246-287
  (candidates, values, reranked winners) and :289-311 (the semantic row count masks
  padding rows), and a full stable sort of the logits on random inputs.
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


def head_logits(q: np.ndarray, sc: np.ndarray, x: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """fp32 logits of the fused head: weights ``dtype(float(q)*s)`` (``fp32``: no narrowing),
    products exact, the sum formed in float64 and rounded once to fp32 (the kernels' fp32
    tile order is compared by tolerance or on inputs whose sums are exact)."""
    W = dequant_qrow(q, sc)
    if dtype == "bf16":
        W = round_bf16(W)
    elif dtype == "fp16":
        W = round_f16(W)
    return (np.asarray(x, dtype=np.float64) @ W.astype(np.float64).T).astype(np.float32)


def qrow_top2(logits: np.ndarray, start_row: int = 0, row_count: int | None = None):
    """Top two rows per logit row over the first ``row_count`` columns: the first is the
    largest (lowest index on ties), the second the largest of the others (lowest index on
    ties), as the block kernel and its reduction select (dense_qstore_cuda.py:620-674).
    Returns ``(indices int32 [M, 2], values fp32 [M, 2])`` with global row indices."""
    L = np.asarray(logits, dtype=np.float32)
    n = L.shape[1] if row_count is None else int(row_count)
    idx = np.zeros((L.shape[0], 2), dtype=np.int32)
    val = np.zeros((L.shape[0], 2), dtype=np.float32)
    for m in range(L.shape[0]):
        row = L[m, :n]
        first = int(np.flatnonzero(row == row.max())[0])
        rest = row.copy()
        rest[first] = -np.inf
        second = int(np.flatnonzero(rest == rest.max())[0])
        idx[m] = (start_row + first, start_row + second)
        val[m] = (row[first], row[second])
    return idx, val


def rerank_fp32(q: np.ndarray, sc: np.ndarray, x: np.ndarray, candidates: np.ndarray, start_row: int = 0):
    """fp32 rerank: ``score = sum float(x) * (float(q) * s)`` (products as fp32, the sum in
    float64 rounded once), best score, lowest index on ties (dense_qstore_cuda.py:1216-1236).
    Returns ``(indices int64 [M], values fp32 [M])``."""
    x = np.asarray(x, dtype=np.float32)
    cand = np.asarray(candidates, dtype=np.int64).reshape(x.shape[0], -1)
    W = dequant_qrow(q, sc)
    out_i = np.zeros(x.shape[0], dtype=np.int64)
    out_v = np.zeros(x.shape[0], dtype=np.float32)
    for m in range(x.shape[0]):
        local = cand[m] - start_row
        prods = (x[m][None, :] * W[local]).astype(np.float32)
        scores = prods.astype(np.float64).sum(axis=1).astype(np.float32)
        best = scores.max()
        out_i[m] = int(cand[m][scores == best].min())
        out_v[m] = best
    return out_i, out_v
