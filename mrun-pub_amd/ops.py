"""The QStore hot path as PyTorch custom operators (namespace ``qstore_hip``).

Importing this module registers every operator below with ``torch.library``, each with a
fake (meta) implementation, so that callers that go through the dispatcher -- graph
capture through torch, ``torch.compile``, ``torch.export``, FakeTensor tracing -- see
real operators with known output shapes instead of opaque Python.  Each operator calls
the same C ABI as the module-level wrappers (``qrow``, ``w8a8``, ``moe``, ``lowbit``), on
torch's current stream, and allocates its outputs fresh; no operator mutates an input.

| operator | replaces (reference, src/mrun/engine/...) |
|---|---|
| ``qrow_dequant(codes, scales, dtype)`` | ``_dequant_qrow`` kernels/qstore.py:385-399 |
| ``qrow_matmul(codes, scales, x, row_stable)`` | ``QStore.matmul`` / ``matmul_row_stable`` qstore.py:1082-1097, ``fused_qrow_matmul`` kernels/dense_qstore_cuda.py:1105-1153 |
| ``qrow_swiglu(gate_codes, gate_scales, up_codes, up_scales, x)`` | ``fused_qrow_swiglu`` dense_qstore_cuda.py:1053-1102 |
| ``qrow_top2(codes, scales, x, start_row, row_count)`` | ``fused_qrow_top2`` dense_qstore_cuda.py:1239-1317 |
| ``act_quant(x, keep)`` | activation quantiser kernels/w8a8.py:118-121 |
| ``int8_gemm(q_x, q_w)`` | ``_int8_gemm`` w8a8.py:33-64 |
| ``w8a8_matmul(q_w, sc_w, x, protect_idx, protect_k, out_dtype)`` | ``w8a8_matmul`` w8a8.py:67-125 |
| ``moe_router(logits, top_k, norm_topk, out_dtype)`` | router qwen3_moe_cuda.py:3702-3707 |
| ``moe_route(top_indices, top_weights, num_experts)`` | ``grouped_route_tensors_with_inverse`` olmoe_cuda.py:1108-1135 |
| ``grouped_int8_mm(rows_q, row_scales, weights, weight_scales, starts, counts, group_slots, max_rows, swiglu, out_dtype)`` | ``grouped_fp8_mm(_strided)`` olmoe_cuda.py:1197-1252, qwen3_moe_cuda.py:2257-2310 |
| ``grouped_w8a16_mm(rows, weights, weight_scales, starts, counts, row_ids, group_slots, max_rows, swiglu, out_dtype)`` | ``grouped_bf16_mm`` qwen3_moe_cuda.py:2473-2510 (weight-only, int8 pages) |
| ``route_reduce(expert_output, coefficients, inverse, rows, top_k)`` | ``stable_route_reduce`` qwen3_moe_cuda.py:2561-2664 |
| ``lowbit_matmul(packed, scales, zeros, x, bits, group_size, in_features)`` | ``QStoreInt3/Int2.matmul`` qstore.py:1318-1341, 1451-1474 |
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _native as nat
from . import lowbit as _lowbit
from . import moe as _moe
from . import qrow as _qrow
from . import w8a8 as _w8a8

NS = "qstore_hip"


def _op(name: str):
    return torch.library.custom_op(f"{NS}::{name}", mutates_args=(), device_types="cuda")


# ---- int8 qrow ------------------------------------------------------------------------------


@_op("qrow_dequant")
def qrow_dequant(codes: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return _qrow.qrow_dequant(codes, scales, dtype)


@qrow_dequant.register_fake
def _(codes, scales, dtype):
    return codes.new_empty(codes.shape, dtype=dtype)


@_op("qrow_matmul")
def qrow_matmul(codes: torch.Tensor, scales: torch.Tensor, x: torch.Tensor, row_stable: bool = False) -> torch.Tensor:
    return _qrow.qrow_matmul(codes, scales, x, row_stable=row_stable)


@qrow_matmul.register_fake
def _(codes, scales, x, row_stable=False):
    return x.new_empty((*x.shape[:-1], codes.shape[0]))


@_op("qrow_swiglu")
def qrow_swiglu(gate_codes: torch.Tensor, gate_scales: torch.Tensor, up_codes: torch.Tensor,
                up_scales: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    g = _qrow.CompactQRowPage("gate", 0, int(gate_codes.shape[0]), int(gate_codes.shape[1]), gate_codes, gate_scales)
    u = _qrow.CompactQRowPage("up", 0, int(up_codes.shape[0]), int(up_codes.shape[1]), up_codes, up_scales)
    return _qrow.fused_qrow_swiglu(g, u, x)[0]


@qrow_swiglu.register_fake
def _(gate_codes, gate_scales, up_codes, up_scales, x):
    return x.new_empty((*x.shape[:-1], gate_codes.shape[0]), dtype=torch.bfloat16)


@_op("qrow_top2")
def qrow_top2(codes: torch.Tensor, scales: torch.Tensor, x: torch.Tensor, start_row: int,
              row_count: int) -> tuple[torch.Tensor, torch.Tensor]:
    page = _qrow.CompactQRowPage("head", start_row, start_row + int(codes.shape[0]), int(codes.shape[1]),
                                 codes, scales)
    idx, val, _tag, _bytes = _qrow.fused_qrow_top2(page, x, semantic_row_count=row_count)
    return idx, val


@qrow_top2.register_fake
def _(codes, scales, x, start_row, row_count):
    shape = (*x.shape[:-1], 2)
    return x.new_empty(shape, dtype=torch.int32), x.new_empty(shape, dtype=torch.float32)


# ---- W8A8 -----------------------------------------------------------------------------------


@_op("act_quant")
def act_quant(x: torch.Tensor, keep: Optional[torch.Tensor] = None) -> tuple[torch.Tensor, torch.Tensor]:
    return _w8a8.quantize_activation(x, keep)


@act_quant.register_fake
def _(x, keep=None):
    K = x.shape[-1]
    T = x.numel() // K if K else 0
    return x.new_empty((T, K), dtype=torch.int8), x.new_empty((T,), dtype=torch.float32)


@_op("int8_gemm")
def int8_gemm(q_x: torch.Tensor, q_w: torch.Tensor) -> torch.Tensor:
    return _w8a8._int8_gemm(q_x, q_w)


@int8_gemm.register_fake
def _(q_x, q_w):
    return q_x.new_empty((q_x.shape[0], q_w.shape[0]), dtype=torch.int32)


@_op("w8a8_matmul")
def w8a8_matmul(q_w: torch.Tensor, sc_w: torch.Tensor, x: torch.Tensor, protect_idx: Optional[torch.Tensor] = None,
                protect_k: int = 0, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    return _w8a8.w8a8_matmul(q_w, sc_w, x, protect_idx=protect_idx, protect_k=protect_k, out_dtype=out_dtype)


@w8a8_matmul.register_fake
def _(q_w, sc_w, x, protect_idx=None, protect_k=0, out_dtype=torch.float32):
    return x.new_empty((*x.shape[:-1], q_w.shape[0]), dtype=out_dtype)


# ---- routed MoE -----------------------------------------------------------------------------


@_op("moe_router")
def moe_router(logits: torch.Tensor, top_k: int, norm_topk: bool = True,
               out_dtype: torch.dtype = torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor]:
    return _moe.route_topk(logits, top_k, norm_topk=norm_topk, out_dtype=out_dtype)


@moe_router.register_fake
def _(logits, top_k, norm_topk=True, out_dtype=torch.bfloat16):
    T = logits.shape[0]
    return logits.new_empty((T, top_k), dtype=out_dtype), logits.new_empty((T, top_k), dtype=torch.int64)


@_op("moe_route")
def moe_route(top_indices: torch.Tensor, top_weights: torch.Tensor,
              num_experts: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    tok, coef, starts, counts, inv, _ = _moe.grouped_route_tensors_with_inverse(
        top_indices, top_weights, num_experts=num_experts)
    return tok, coef, starts, counts, inv


@moe_route.register_fake
def _(top_indices, top_weights, num_experts):
    A = top_indices.numel()
    return (top_indices.new_empty((A,), dtype=torch.int64), top_weights.new_empty((A,)),
            top_indices.new_empty((num_experts,), dtype=torch.int32),
            top_indices.new_empty((num_experts,), dtype=torch.int32),
            top_indices.new_empty((A,), dtype=torch.int64))


@_op("grouped_int8_mm")
def grouped_int8_mm(rows_q: torch.Tensor, row_scales: torch.Tensor, weights: torch.Tensor,
                    weight_scales: torch.Tensor, starts: torch.Tensor, counts: torch.Tensor,
                    group_slots: Optional[torch.Tensor] = None, max_rows: int = 0, swiglu: bool = False,
                    out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    y, _tag = _moe.grouped_int8_mm(rows_q, row_scales, weights, weight_scales, starts, counts,
                                   group_slots=group_slots, max_rows=max_rows or None, swiglu=swiglu,
                                   out_dtype=out_dtype)
    return y


@grouped_int8_mm.register_fake
def _(rows_q, row_scales, weights, weight_scales, starts, counts, group_slots=None, max_rows=0, swiglu=False,
      out_dtype=torch.bfloat16):
    n = weights.shape[1] // 2 if swiglu else weights.shape[1]
    return rows_q.new_empty((rows_q.shape[0], n), dtype=out_dtype)


@_op("grouped_w8a16_mm")
def grouped_w8a16_mm(rows: torch.Tensor, weights: torch.Tensor, weight_scales: torch.Tensor, starts: torch.Tensor,
                     counts: torch.Tensor, row_ids: Optional[torch.Tensor] = None,
                     group_slots: Optional[torch.Tensor] = None, max_rows: int = 0, swiglu: bool = False,
                     out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    y, _tag = _moe.grouped_w8a16_mm(rows, weights, weight_scales, starts, counts, row_ids=row_ids,
                                    group_slots=group_slots, max_rows=max_rows or None, swiglu=swiglu,
                                    out_dtype=out_dtype)
    return y


@grouped_w8a16_mm.register_fake
def _(rows, weights, weight_scales, starts, counts, row_ids=None, group_slots=None, max_rows=0, swiglu=False,
      out_dtype=torch.bfloat16):
    n = weights.shape[1] // 2 if swiglu else weights.shape[1]
    A = rows.shape[0] if row_ids is None else row_ids.shape[0]
    return rows.new_empty((A, n), dtype=out_dtype)


@_op("route_reduce")
def route_reduce(expert_output: torch.Tensor, coefficients: torch.Tensor, inverse: torch.Tensor, rows: int,
                 top_k: int) -> torch.Tensor:
    A = rows * top_k
    if expert_output.ndim != 2 or int(expert_output.shape[0]) != A:
        raise ValueError("expert output rows must equal rows * top_k")
    if coefficients.dtype != torch.float32 or coefficients.numel() != A or inverse.numel() != A:
        raise ValueError("coefficients (float32) and inverse must cover every assignment")
    if expert_output.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("expert output must be float32 or bfloat16")
    device = nat.require_device(expert_output, coefficients, inverse)
    y = expert_output.contiguous()
    inv = inverse.to(torch.int64).contiguous()
    H = int(y.shape[1])
    out = torch.empty((rows, H), dtype=torch.float32, device=device)
    if rows:
        nat.call("qs_moe_route_reduce", nat.ptr(y), nat.dtype_code(y.dtype), nat.ptr(coefficients.contiguous()),
                 nat.ptr(inv), rows, top_k, H, nat.ptr(out), nat.stream_of(device))
    return out


@route_reduce.register_fake
def _(expert_output, coefficients, inverse, rows, top_k):
    return expert_output.new_empty((rows, expert_output.shape[1]), dtype=torch.float32)


# ---- packed low-bit -------------------------------------------------------------------------


@_op("lowbit_matmul")
def lowbit_matmul(packed: torch.Tensor, scales: torch.Tensor, zeros: Optional[torch.Tensor], x: torch.Tensor,
                  bits: int, group_size: int, in_features: int) -> torch.Tensor:
    page = _lowbit.LowbitPage("w", bits, group_size, in_features, packed, scales, zeros)
    return _lowbit.lowbit_matmul(page, x)


@lowbit_matmul.register_fake
def _(packed, scales, zeros, x, bits, group_size, in_features):
    return x.new_empty((*x.shape[:-1], packed.shape[0]), dtype=torch.float32)


OPS = ("qrow_dequant", "qrow_matmul", "qrow_swiglu", "qrow_top2", "act_quant", "int8_gemm", "w8a8_matmul",
       "moe_router", "moe_route", "grouped_int8_mm", "grouped_w8a16_mm", "route_reduce", "lowbit_matmul")
