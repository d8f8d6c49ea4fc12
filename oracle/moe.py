"""Oracle: routed MoE with int8 experts (numpy, CPU).

Restates (reference paths relative to /root/reference):
* ``router``            -- qwen3_moe_cuda.py:3702-3707 (softmax fp32, top-k, renormalise,
                           cast to the model dtype)
* ``route_stable``      -- CPU branch of ``_grouped_route_tensors_impl`` olmoe_cuda.py:1063-1090
                           (stable argsort, bincount, exclusive prefix, inverse)
* ``quantize_rows``     -- per-row absmax/127 int8 codec (w8a8.py:118-121 recipe; the int8
                           analogue of ``quantize_fp8_activation`` olmoe_cuda.py:1173-1176)
* ``grouped_int8_mm``   -- per-group exact int GEMM with the epilogue
                           ``(acc * a_scale[m]) * w_scale[n]`` (olmoe_cuda.py:185-238)
* ``grouped_w8a16_mm``  -- ``_grouped_bf16_kernel`` (qwen3_moe_cuda.py:2117-2157) over
                           weights ``bf16(float(code) * scale)``: fp32 result of the bf16
                           GEMM, bf16 SwiGLU halves as PackedBF16ExpertBackend.moe
                           (:3020-3033)
* ``stable_route_reduce`` -- CPU branch qwen3_moe_cuda.py:2655-2664
* ``moe_forward``       -- the W8A8-shaped expert flow of FP8ExpertBackend.moe
                           (olmoe_cuda.py:1308-1420) with the stable reducer
                           (qwen3_moe_cuda.py:2911-2920) and bf16 boundaries
* ``moe_forward_w8a16`` -- the weight-only flow of PackedBF16ExpertBackend.moe
                           (qwen3_moe_cuda.py:2978-3046) on int8 pages, stable reducer
* ``moe_dense_reference`` -- per-expert float math of streamed_moe_forward
                           (moe_safetensors.py:603-627), weights dequantized to fp32, in float64
* ``moe_streamed_reference`` -- the same in the model dtype (bf16 / fp32 roundings)

Pinned by (tests/test_oracle_moe.py): the reference KATs test_olmoe_cuda.py:73-112 and
test_qwen3_moe_cuda.py:1140-1241 (counts/starts/token ids/coefficients, inverse bijection,
reduce == index_add and invariance under within-group permutation); numpy/torch library
routines for the router; exact integer brute force for the grouped GEMM; the dense fp32
per-expert formulation for the whole layer (tolerance).  ``moe_dense_reference`` and
``moe_streamed_reference`` are pinned by tests/golden/moe_forward.npz, written by the
reference's own streamed_moe_forward on a tiny Qwen3-MoE layer: fp32 within 1e-6, and the
bf16 restatement reproduces the reference's residual bit for bit.  ``grouped_w8a16_mm``
is pinned by the same golden: its per-expert outputs, accumulated in the reference's
expert order, give the reference's bf16 residual bit for bit.
"""

from __future__ import annotations

import numpy as np

from .qrow import round_bf16, silu_f32
from .w8a8 import act_quant, int8_gemm


def router(logits: np.ndarray, k: int, norm_topk: bool = True, bf16: bool = True):
    p = np.asarray(logits, dtype=np.float32)
    p = p - p.max(axis=-1, keepdims=True)
    e = np.exp(p).astype(np.float32)
    prob = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    order = np.argsort(-prob, axis=-1, kind="stable")[:, :k]
    w = np.take_along_axis(prob, order, axis=-1).astype(np.float32)
    if norm_topk:
        w = (w / w.sum(axis=-1, keepdims=True)).astype(np.float32)
    if bf16:
        w = round_bf16(w)
    return w, order.astype(np.int64)


def route_stable(top_indices: np.ndarray, top_weights: np.ndarray, num_experts: int):
    ti = np.asarray(top_indices).reshape(-1).astype(np.int64)
    tw = np.asarray(top_weights, dtype=np.float32).reshape(-1)
    rows, k = np.asarray(top_indices).shape
    order = np.argsort(ti, kind="stable")
    token_ids = (np.arange(rows * k) // k)[order].astype(np.int64)
    coef = tw[order]
    counts = np.bincount(ti, minlength=num_experts).astype(np.int32)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int32)
    inverse = np.empty(rows * k, dtype=np.int64)
    inverse[order] = np.arange(rows * k)
    return token_ids, coef, starts, counts, inverse


def quantize_rows(x: np.ndarray):
    return act_quant(np.asarray(x, dtype=np.float32))


def grouped_int8_mm(rows_q, row_scales, weights, weight_scales, starts, counts, *, slots=None,
                    swiglu: bool = False, out_bf16: bool = True, acc_out: list | None = None):
    rows_q = np.asarray(rows_q)
    G = len(starts)
    n_w = weights.shape[1]
    n_out = n_w // 2 if swiglu else n_w
    out = np.zeros((rows_q.shape[0], n_out), dtype=np.float32)
    for g in range(G):
        s0, c = int(starts[g]), int(counts[g])
        if c == 0:
            continue
        slot = g if slots is None else int(slots[g])
        acc = int8_gemm(rows_q[s0 : s0 + c], weights[slot])
        if acc_out is not None:
            acc_out.append((g, acc))
        v = (acc.astype(np.float32) * row_scales[s0 : s0 + c, None]).astype(np.float32) * weight_scales[slot][None, :]
        v = v.astype(np.float32)
        if swiglu:
            gt = round_bf16(v[:, :n_out])
            ut = round_bf16(v[:, n_out:])
            out[s0 : s0 + c] = round_bf16(round_bf16(silu_f32(gt)) * ut)
        else:
            out[s0 : s0 + c] = round_bf16(v) if out_bf16 else v
    return out


def grouped_w8a16_mm(rows, weights, weight_scales, starts, counts, *, slots=None, swiglu: bool = False,
                     out_bf16: bool = True):
    """Per group: ``rows @ bf16(code * scale)^T``, summed in float64 and rounded once to
    fp32 (the kernel's fp32 accumulation order is not fixed); SwiGLU takes gate rows
    ``[0, N)`` and up rows ``[N, 2N)`` with the bf16 roundings of the reference's eager
    ``F.silu(gate) * up`` on bf16 halves."""
    rows = np.asarray(rows, dtype=np.float32)
    n_w = weights.shape[1]
    n_out = n_w // 2 if swiglu else n_w
    out = np.zeros((rows.shape[0], n_out), dtype=np.float32)
    for g in range(len(starts)):
        s0, c = int(starts[g]), int(counts[g])
        if c == 0:
            continue
        slot = g if slots is None else int(slots[g])
        w = round_bf16(weights[slot].astype(np.float32) * weight_scales[slot][:, None]).astype(np.float64)
        v = (rows[s0 : s0 + c].astype(np.float64) @ w.T).astype(np.float32)
        if swiglu:
            gt = round_bf16(v[:, :n_out])
            ut = round_bf16(v[:, n_out:])
            out[s0 : s0 + c] = round_bf16(round_bf16(silu_f32(gt)) * ut)
        else:
            out[s0 : s0 + c] = round_bf16(v) if out_bf16 else v
    return out


def stable_route_reduce(expert_output, coefficients, inverse, rows: int, k: int):
    eo = np.asarray(expert_output, dtype=np.float32)
    cf = np.asarray(coefficients, dtype=np.float32)
    inv = np.asarray(inverse).reshape(rows, k)
    contrib = (eo[inv] * cf[inv][..., None]).astype(np.float32)
    out = contrib[:, 0].copy()
    for r in range(1, k):
        out = (out + contrib[:, r]).astype(np.float32)
    return out


def moe_forward(source, top_indices, top_weights, gate_up, gate_up_scales, down, down_scales):
    """int8 expert layer, returns bf16-rounded fp32 [T, H]."""
    E = gate_up.shape[0]
    rows, k = top_indices.shape
    token_ids, coef, starts, counts, inverse = route_stable(top_indices, top_weights, E)
    q, s = quantize_rows(np.asarray(source, dtype=np.float32)[token_ids])
    act = grouped_int8_mm(q, s, gate_up, gate_up_scales, starts, counts, swiglu=True)
    q2, s2 = quantize_rows(act)
    y = grouped_int8_mm(q2, s2, down, down_scales, starts, counts)
    return round_bf16(stable_route_reduce(y, coef, inverse, rows, k))


def moe_forward_w8a16(source, top_indices, top_weights, gate_up, gate_up_scales, down, down_scales):
    """Weight-only int8 expert layer (bf16 activations), returns bf16-rounded fp32 [T, H]."""
    E = gate_up.shape[0]
    rows, k = top_indices.shape
    token_ids, coef, starts, counts, inverse = route_stable(top_indices, top_weights, E)
    x = round_bf16(np.asarray(source, dtype=np.float32))[token_ids]
    act = grouped_w8a16_mm(x, gate_up, gate_up_scales, starts, counts, swiglu=True)
    y = grouped_w8a16_mm(act, down, down_scales, starts, counts)
    return round_bf16(stable_route_reduce(y, coef, inverse, rows, k))


def moe_streamed_reference(y, top_indices, top_weights, gate_up, gate_up_scales, down, down_scales,
                           dtype: str = "bf16", round_act: bool = True):
    """Per-expert math of streamed_moe_forward (moe_safetensors.py:603-627) in the model dtype.

    Weights are ``dtype(float(code) * scale)``; every torch op's result is rounded to
    ``dtype`` as the reference's eager ops round it: the fused gate/up GEMM, silu, the
    product, the down GEMM, ``w_e * ye`` and the running ``moe[tok] += ...``.  GEMMs sum in
    float64 and round once (the reference's BLAS order is not fixed).  ``round_act=False``
    drops the rounding of ``silu(g) * u`` (a planted mistake for the tests).  Returns the
    ``moe`` tensor as fp32 values."""
    rnd = round_bf16 if dtype == "bf16" else (lambda a: np.asarray(a, dtype=np.float32))
    y = rnd(np.asarray(y, dtype=np.float32))
    T, H = y.shape
    out = np.zeros((T, H), dtype=np.float32)
    I = gate_up.shape[1] // 2
    w_all = rnd(np.asarray(top_weights, dtype=np.float32))
    for e in np.unique(top_indices):
        sel = top_indices == e
        tok = sel.any(-1)
        w_e = rnd((w_all * sel).sum(-1))[tok]
        Wgu = rnd(gate_up[e].astype(np.float32) * gate_up_scales[e][:, None]).astype(np.float64)
        Wd = rnd(down[e].astype(np.float32) * down_scales[e][:, None]).astype(np.float64)
        gu = rnd(y[tok].astype(np.float64) @ Wgu.T)
        g, u = gu[:, :I], gu[:, I:]
        act = rnd(silu_f32(g)) * u
        act = rnd(act) if round_act else act.astype(np.float32)
        ye = rnd(act.astype(np.float64) @ Wd.T)
        out[tok] = rnd(out[tok] + rnd(w_e[:, None] * ye))
    return out


def moe_dense_reference(source, top_indices, top_weights, gate_up, gate_up_scales, down, down_scales):
    """Float per-expert math (moe_safetensors.py:603-627) on fp32-dequantized weights."""
    x = np.asarray(source, dtype=np.float64)
    T, H = x.shape
    out = np.zeros((T, H), dtype=np.float64)
    I = gate_up.shape[1] // 2
    for e in np.unique(top_indices):
        sel = top_indices == e
        tok = sel.any(-1)
        w_e = (np.asarray(top_weights, np.float64) * sel).sum(-1)[tok]
        Wgu = gate_up[e].astype(np.float64) * gate_up_scales[e][:, None]
        Wd = down[e].astype(np.float64) * down_scales[e][:, None]
        gu = x[tok] @ Wgu.T
        g, u = gu[:, :I], gu[:, I:]
        act = g / (1 + np.exp(-g)) * u
        out[tok] += w_e[:, None] * (act @ Wd.T)
    return out
