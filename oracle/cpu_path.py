"""CPU baseline: the reference's own CPU qrow path, restated with torch CPU ops -- TEST /
BASELINE INFRASTRUCTURE ONLY (imported by ``bench.py``'s ``cpu_baseline`` leg and tests).

Follows the reference step for step:
* dequant ``torch.from_numpy(q).to(float32).mul_(sc[:, None])``   qstore.py:385-399
* narrow to the compute dtype (bf16, RNE)                          qstore.py:1076-1077
* ``x.to(W.dtype) @ W.T`` (torch CPU GEMM)                         qstore.py:1082-1092

Pinned by tests/test_oracle_cpu_path.py against ``oracle.qrow`` (bit-exact dequant and
bf16 narrowing; matmul within the fp32-accumulation tolerance).
"""

from __future__ import annotations

import numpy as np
import torch


def dequant_qrow(q: np.ndarray, sc: np.ndarray) -> torch.Tensor:
    W = torch.from_numpy(q).to(torch.float32)
    W.mul_(torch.from_numpy(sc)[:, None])
    return W


def qstore_matmul(q: np.ndarray, sc: np.ndarray, x: torch.Tensor, compute_dtype=torch.bfloat16) -> torch.Tensor:
    W = dequant_qrow(q, sc)
    if compute_dtype is not torch.float32:
        W = W.to(compute_dtype)
    if x.dtype is not W.dtype:
        x = x.to(W.dtype)
    return x @ W.T


# ---- the reference's other CPU paths, for the per-config CPU baselines -------------------


def w8a8_matmul(q_w: torch.Tensor, sc_w: torch.Tensor, x: torch.Tensor, protect_k: int = 8) -> torch.Tensor:
    """CPU ``w8a8_matmul`` (w8a8.py:67-125 with ``_int8_gemm``'s CPU ``torch._int_mm``,
    :33-64): fp32 outlier side path over the top-k columns, per-token int8 quantisation,
    int32 GEMM, rescale."""
    out, inn = q_w.shape
    x2 = x.reshape(-1, inn).float()
    y = torch.zeros((x2.shape[0], out), dtype=torch.float32)
    keep = torch.ones(inn, dtype=torch.float32)
    if protect_k > 0:
        idx = x2.abs().amax(dim=0).topk(protect_k).indices
        Wp = q_w[:, idx].float() * sc_w[:, None]
        y += x2[:, idx] @ Wp.T
        keep[idx] = 0.0
    src = x2 * keep
    act_scale = src.abs().amax(dim=1, keepdim=True) / 127.0
    act_scale = torch.where(act_scale == 0, torch.ones_like(act_scale), act_scale)
    q_x = torch.round(src / act_scale).clamp_(-127, 127).to(torch.int8)
    acc = torch._int_mm(q_x.contiguous(), q_w.t().contiguous())
    y += acc.to(torch.float32) * act_scale * sc_w[None, :]
    return y


def lowbit_matmul(packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray | None, x: torch.Tensor, inn: int,
                  bits: int, G: int, offset: float, chunk_rows: int = 1024) -> torch.Tensor:
    """CPU ``QStoreInt3/Int2.matmul`` (qstore.py:1318-1341, dequant :441-456): per chunk of
    output rows, ``np.unpackbits`` of the LSB-first streams, ``(code - zero) * scale`` in
    fp32, then ``x @ W.T``."""
    out = packed.shape[0]
    x2 = x.reshape(-1, inn).to(torch.float32)
    y = torch.empty((x2.shape[0], out), dtype=torch.float32)
    for s in range(0, out, chunk_rows):
        e = min(s + chunk_rows, out)
        b = np.unpackbits(packed[s:e], axis=1, bitorder="little")[:, : inn * bits].reshape(e - s, inn, bits)
        code = np.zeros((e - s, inn), dtype=np.float32)
        for j in range(bits):
            code += b[:, :, j].astype(np.float32) * float(1 << j)
        sc = np.repeat(scales[s:e].astype(np.float32), G, axis=1)[:, :inn]
        z = offset if zeros is None else np.repeat(zeros[s:e].astype(np.float32), G, axis=1)[:, :inn]
        W = ((code - z) * sc).astype(np.float32)
        y[:, s:e] = x2 @ torch.from_numpy(W).T
    return y


def moe_layer(source: torch.Tensor, top_idx: torch.Tensor, top_w: torch.Tensor, gu_q: np.ndarray, gu_s: np.ndarray,
              dn_q: np.ndarray, dn_s: np.ndarray, experts=None) -> torch.Tensor:
    """CPU routed-expert math of ``streamed_moe_forward`` (moe_safetensors.py:603-627) in
    bf16 over int8 experts dequantised per active expert (the reference's CPU MoE path pulls
    each routed expert's weights, then runs the fused gate/up GEMM, SwiGLU and down GEMM).
    ``experts`` restricts the loop to a subset (a bounded timing sample)."""
    y = source.to(torch.bfloat16)
    moe = torch.zeros_like(y)
    I = gu_q.shape[1] // 2
    routed = torch.unique(top_idx).tolist() if experts is None else experts
    for e in routed:
        sel = top_idx == e
        tok = sel.any(-1)
        w_e = (top_w * sel.to(top_w.dtype)).sum(-1)[tok]
        Wgu = dequant_qrow(gu_q[e], gu_s[e]).to(torch.bfloat16)
        Wd = dequant_qrow(dn_q[e], dn_s[e]).to(torch.bfloat16)
        gu = y[tok] @ Wgu.T
        g, u = gu[:, :I], gu[:, I:]
        act = torch.nn.functional.silu(g) * u
        moe[tok] += w_e[:, None] * (act @ Wd.T)
    return moe
