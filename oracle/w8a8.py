"""Oracle: W8A8 per-token int8 GEMM with the fp32 outlier side path (numpy, CPU).

Restates src/mrun/engine/kernels/w8a8.py (reference paths relative to /root/reference):
* ``int8_gemm``      -- ``_int8_gemm``       w8a8.py:33-64  (exact int32 accumulation)
* ``act_quant``      -- activation recipe    w8a8.py:118-121
* ``protect_topk``   -- outlier columns      w8a8.py:98-102
* ``w8a8_matmul``    -- full contract        w8a8.py:67-125

Pinned by (tests/test_oracle_w8a8.py):
* int8_gemm against brute-force Python int arithmetic and numpy int64 (closed form);
* act_quant against torch's own ops composed exactly as the reference writes them
  (library routines: ``torch.round``, ``amax``, IEEE division) on random, tie and
  all-zero rows;
* w8a8_matmul against the reference's published test properties (test_w8a8.py:34-64:
  error bounds with/without protection, argmax, static list == top-k) and, where the
  side path is absent, bit-equality with the closed-form epilogue
  ``(float(acc) * act_scale) * w_scale``;
* golden vectors written from the reference in this container (tests/golden/), when
  present.
"""

from __future__ import annotations

import numpy as np


def int8_gemm(qx: np.ndarray, qw: np.ndarray) -> np.ndarray:
    """``[T,K] int8 @ [N,K] int8^T -> [T,N] int32`` (exact).

    Evaluated as a float64 GEMM: every product is at most 128*128 = 2^14 in magnitude and
    every partial sum of K terms at most K * 2^14, so for K <= 2^38 each partial sum is an
    integer below 2^53 and the float64 evaluation is exact in any summation order (this
    lets the config-3 sizes run through BLAS in seconds; numpy's int64 matmul has no BLAS).
    """
    qx = np.asarray(qx, dtype=np.int8)
    qw = np.asarray(qw, dtype=np.int8)
    assert qx.shape[-1] <= 2**38
    acc = qx.astype(np.float64) @ qw.astype(np.float64).T
    assert np.abs(acc).max(initial=0) < 2**31
    return acc.astype(np.int32)


def act_quant(x: np.ndarray, keep: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Per-row ``s = max|x*keep|/127`` (0 -> 1); ``q = clamp(round_half_even(x*keep/s), ±127)``."""
    x = np.asarray(x, dtype=np.float32)
    src = x if keep is None else (x * np.asarray(keep, dtype=np.float32)[None, :]).astype(np.float32)
    scale = (np.abs(src).max(axis=1, keepdims=True) / np.float32(127.0)).astype(np.float32)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    q = np.clip(np.round((src / scale).astype(np.float32)), -127, 127).astype(np.int8)
    return q, scale[:, 0]


def protect_topk(x: np.ndarray, k: int) -> np.ndarray:
    """Indices of the ``k`` largest column maxima of ``|x|`` (ties -> lower index)."""
    colmax = np.abs(np.asarray(x, dtype=np.float32)).max(axis=0)
    order = np.lexsort((np.arange(colmax.size), -colmax))
    return order[: min(k, colmax.size)].astype(np.int64)


def w8a8_matmul(
    q_w: np.ndarray,
    sc_w: np.ndarray,
    x: np.ndarray,
    *,
    protect_idx: np.ndarray | None = None,
    protect_k: int = 0,
) -> np.ndarray:
    """``x @ (q_w * sc_w[:, None]).T`` through int8 x int8 plus the fp32 side path; fp32 out."""
    q_w = np.asarray(q_w, dtype=np.int8)
    sc_w = np.asarray(sc_w, dtype=np.float32)
    out, inn = q_w.shape
    x2 = np.asarray(x, dtype=np.float32).reshape(-1, inn)
    T = x2.shape[0]
    if protect_idx is None and protect_k > 0:
        protect_idx = protect_topk(x2, protect_k)
    if protect_idx is not None and np.asarray(protect_idx).size == 0:
        protect_idx = None
    y = np.zeros((T, out), dtype=np.float32)
    keep = None
    if protect_idx is not None:
        pidx = np.asarray(protect_idx, dtype=np.int64)
        Wp = (q_w[:, pidx].astype(np.float32) * sc_w[:, None]).astype(np.float32)
        y = (y + (x2[:, pidx].astype(np.float64) @ Wp.T.astype(np.float64)).astype(np.float32)).astype(np.float32)
        keep = np.ones(inn, dtype=np.float32)
        keep[pidx] = 0.0
    q_x, act_scale = act_quant(x2, keep)
    acc = int8_gemm(q_x, q_w)
    y = (y + (acc.astype(np.float32) * act_scale[:, None]).astype(np.float32) * sc_w[None, :]).astype(np.float32)
    return y.reshape(*np.asarray(x).shape[:-1], out)
