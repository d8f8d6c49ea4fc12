"""Routed MoE with int8 experts on gfx950 -- the reference's MoE operator surface.

Mirrors (reference paths relative to /root/reference):
* router: softmax(fp32) -> top-k -> renormalise -> model dtype
  (src/mrun/engine/qwen3_moe_cuda.py:3702-3707)                      -> ``route_topk``
* ``grouped_route_tensors(_with_inverse)`` (src/mrun/engine/olmoe_cuda.py:989-1135)
* ``_compact_route(_with_inverse)`` (qwen3_moe_cuda.py:2530-2558)
* ``stable_route_reduce`` (qwen3_moe_cuda.py:2561-2664)
* the grouped GEMM ABI of ``grouped_fp8_mm(_strided)`` (olmoe_cuda.py:1197-1252,
  qwen3_moe_cuda.py:2191-2310) for int8 codes + per-row fp32 scales  -> ``grouped_int8_mm``
* the W8A8-shaped expert flow of ``FP8ExpertBackend.moe`` (olmoe_cuda.py:1308-1420) with
  the int8 qrow codec instead of FP8, and the stable reducer of
  ``PagedInt4ExpertBackend.moe`` (qwen3_moe_cuda.py:2840-2936)    -> ``Int8ExpertBackend``
* expert page layout ``ExpertPageLayout`` (qwen3_moe_cuda.py:187-233)  -> ``ExpertPageLayout``

Differences by design: the device route compiler is stable (queue order = the CPU stable
argsort), so the reference's "atomic cursor" nondeterminism does not exist here; the
reducer is still rank ordered.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import torch

from . import _native as nat

IMPL_ROUTE = "hip-gfx950-stable-route-v1"
IMPL_GROUPED = "hip-gfx950-grouped-w8a8-mfma-i8-v1"
IMPL_GROUPED_W8A16 = "hip-gfx950-grouped-w8a16-mfma-bf16-v1"


def _align(n: int, a: int = 4096) -> int:
    return (n + a - 1) // a * a


# ---- router ------------------------------------------------------------------------------


@torch.inference_mode()
def route_topk(
    logits: torch.Tensor, top_k: int, *, norm_topk: bool = True, out_dtype: torch.dtype = torch.bfloat16
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(top_weights [T,k] out_dtype, top_indices [T,k] int64)`` of softmax(fp32) routing."""
    if logits.ndim != 2:
        raise ValueError("router logits must have shape [tokens, experts]")
    if logits.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("router logits must be float32 or bfloat16")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("router weights are float32 or bfloat16")
    device = nat.require_device(logits)
    lg = logits.contiguous()
    T, E = map(int, lg.shape)
    idx = torch.empty((T, top_k), dtype=torch.int64, device=device)
    w = torch.empty((T, top_k), dtype=out_dtype, device=device)
    nat.call(
        "qs_moe_router", nat.ptr(lg), nat.dtype_code(lg.dtype), T, E, int(top_k), int(bool(norm_topk)),
        nat.ptr(idx), nat.ptr(w), nat.dtype_code(out_dtype), nat.stream_of(device),
    )
    return w, idx


# ---- route compiler ----------------------------------------------------------------------


def _route_impl(top_indices, top_weights, num_experts: int, include_inverse: bool, coef_f32: bool = False,
                quant_source: torch.Tensor | None = None):
    """The route plan; with ``quant_source`` ([T, H] bf16/fp32) also the per-token int8
    codes and scales of its T rows (unpermuted), in the same launch where possible
    (qs_moe_route_quant) -- appended to the returned tuple as ``(q, scale)``."""
    started = time.perf_counter()
    if top_indices.ndim != 2 or top_weights.shape != top_indices.shape:
        raise ValueError("route tensors must both have shape [rows, top_k]")
    if top_indices.dtype not in (torch.int32, torch.int64):
        raise ValueError("top_indices must be int32 or int64")
    if top_weights.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("top_weights must be float32 or bfloat16")
    if top_indices.device.type == "cpu" and top_indices.numel():
        # host tensors are checked here; on the device the route kernel drops such
        # assignments instead (no sync in the hot path), see qs_moe_route
        lo, hi = int(top_indices.min()), int(top_indices.max())
        if lo < 0 or hi >= num_experts:
            raise ValueError(f"top_indices must lie in [0, {num_experts}); found [{lo}, {hi}]")
    device = nat.require_device(top_indices, top_weights)
    rows, top_k = map(int, top_indices.shape)
    A = rows * top_k
    ti = top_indices.contiguous()
    tw = top_weights.contiguous()
    token_ids = torch.empty(A, dtype=torch.long, device=device)
    coef = torch.empty(A, dtype=torch.float32, device=device)
    starts = torch.empty(num_experts, dtype=torch.int32, device=device)
    counts = torch.empty(num_experts, dtype=torch.int32, device=device)
    inverse = torch.empty(A, dtype=torch.long, device=device) if include_inverse else None
    if quant_source is None:
        nat.call(
            "qs_moe_route", nat.ptr(ti), nat.dtype_code(ti.dtype), nat.ptr(tw), nat.dtype_code(tw.dtype),
            rows, top_k, int(num_experts), nat.ptr(token_ids), nat.ptr(coef), nat.ptr(starts),
            nat.ptr(counts), nat.ptr(inverse), nat.stream_of(device),
        )
        quant = ()
    else:
        src = quant_source.contiguous()
        if src.ndim != 2 or int(src.shape[0]) != rows:
            raise ValueError("quant_source must have one row per routed token")
        nat.require_device(src)
        H = int(src.shape[1])
        q = torch.empty((rows, H), dtype=torch.int8, device=device)
        sc = torch.empty(rows, dtype=torch.float32, device=device)
        nat.call(
            "qs_moe_route_quant", nat.ptr(ti), nat.dtype_code(ti.dtype), nat.ptr(tw), nat.dtype_code(tw.dtype),
            rows, top_k, int(num_experts), nat.ptr(token_ids), nat.ptr(coef), nat.ptr(starts),
            nat.ptr(counts), nat.ptr(inverse), nat.ptr(src), nat.dtype_code(src.dtype), H, H, nat.ptr(q),
            nat.ptr(sc), nat.stream_of(device),
        )
        quant = (q, sc)
    # coefficients keep the routing-weight dtype, as the reference's index_select does
    # (the kernel's fp32 copy of a bf16 weight is exact, so coef_f32 loses nothing)
    coef = coef if (tw.dtype == torch.float32 or coef_f32) else coef.to(tw.dtype)
    return (token_ids, coef, starts, counts, inverse, time.perf_counter() - started) + quant


def grouped_route_tensors(top_indices, top_weights, *, num_experts: int):
    """Expert-major route plan ``(token_ids, coefficients, starts, counts, metadata_s)``."""
    t, c, s, n, _inv, dt = _route_impl(top_indices, top_weights, num_experts, False)
    return t, c, s, n, dt


def grouped_route_tensors_with_inverse(top_indices, top_weights, *, num_experts: int):
    """Route plan plus ``inverse[t*k + rank] = queue row`` (olmoe_cuda.py:1108-1135)."""
    return _route_impl(top_indices, top_weights, num_experts, True)


def _compact_route(top_indices, top_weights, selected_experts):
    compact = torch.searchsorted(selected_experts, top_indices)
    t, c, s, n, _ = grouped_route_tensors(compact, top_weights, num_experts=int(selected_experts.numel()))
    return t, c, s, n


def _compact_route_with_inverse(top_indices, top_weights, selected_experts):
    compact = torch.searchsorted(selected_experts, top_indices)
    t, c, s, n, inv, _ = grouped_route_tensors_with_inverse(
        compact, top_weights, num_experts=int(selected_experts.numel())
    )
    return t, c, s, n, inv


# ---- reducer -------------------------------------------------------------------------------


@torch.inference_mode()
def stable_route_reduce(
    expert_output: torch.Tensor,
    coefficients: torch.Tensor,
    token_ids: torch.Tensor,
    counts: torch.Tensor,
    top_indices: torch.Tensor,
    selected_experts: torch.Tensor,
    *,
    inverse_assignments: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """``out[t] = sum_rank float(expert_out[inv[t*k+rank]]) * float(coef[...])`` in fixed rank
    order, fp32 ``[T, H]`` (qwen3_moe_cuda.py:2561-2664).  ``out_dtype=torch.bfloat16``
    returns the fp32 sums rounded once, what the caller's ``output.to(self.dtype)``
    (qwen3_moe_cuda.py:2936) makes of them, from the same kernel."""
    if top_indices.ndim != 2:
        raise ValueError("stable route reduction requires [rows, top_k] indices")
    rows, top_k = map(int, top_indices.shape)
    A = rows * top_k
    if expert_output.ndim != 2 or int(expert_output.shape[0]) != A:
        raise ValueError("expert output rows must equal rows * top_k")
    if token_ids.ndim != 1 or int(token_ids.numel()) != A:
        raise ValueError("stable route token IDs must cover every assignment")
    if coefficients.ndim != 1 or int(coefficients.numel()) != A:
        raise ValueError("stable route coefficients must cover every assignment")
    if counts.ndim != 1 or int(counts.numel()) != int(selected_experts.numel()):
        raise ValueError("stable route counts must match selected experts")
    device = nat.require_device(expert_output, coefficients, token_ids, counts, top_indices, selected_experts)
    inverse = inverse_assignments
    if inverse is not None:
        if inverse.ndim != 1 or int(inverse.numel()) != A:
            raise ValueError("stable route inverse must cover every assignment")
        if inverse.dtype not in (torch.int32, torch.int64):
            raise ValueError("stable route inverse must use int32 or int64")
        inverse = inverse.to(torch.long)
    else:
        # rebuild the [token, rank] -> queue-row bijection from the plan itself
        compact = torch.searchsorted(selected_experts, top_indices)
        group_ids = torch.repeat_interleave(
            torch.arange(int(selected_experts.numel()), device=device, dtype=torch.long),
            counts.to(torch.long), output_size=A,
        )
        matches = compact.index_select(0, token_ids) == group_ids[:, None]
        ranks = matches.to(torch.int64).argmax(dim=1)
        inverse = torch.empty(A, device=device, dtype=torch.long)
        inverse.index_copy_(0, token_ids * top_k + ranks, torch.arange(A, device=device, dtype=torch.long))
    H = int(expert_output.shape[1])
    y = expert_output.contiguous()
    if y.dtype not in (torch.float32, torch.bfloat16):
        y = y.float()
    coef = coefficients.float().contiguous()
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("stable route reduction output must be float32 or bfloat16")
    out = torch.empty((rows, H), dtype=out_dtype, device=device)
    nat.call(
        "qs_moe_route_reduce_to", nat.ptr(y), nat.dtype_code(y.dtype), nat.ptr(coef), nat.ptr(inverse.contiguous()),
        rows, top_k, H, nat.ptr(out), nat.dtype_code(out_dtype), nat.stream_of(device),
    )
    return out


# ---- grouped GEMM --------------------------------------------------------------------------


@torch.inference_mode()
def quantize_rows(source: torch.Tensor, rows: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """int8 codes and fp32 scales of ``source[rows]`` (per-row absmax/127, W8A8 recipe)."""
    device = nat.require_device(source, rows)
    src = source.contiguous()
    H = int(src.shape[1])
    A = int(rows.numel()) if rows is not None else int(src.shape[0])
    q = torch.empty((A, H), dtype=torch.int8, device=device)
    s = torch.empty(A, dtype=torch.float32, device=device)
    if A:
        nat.call(
            "qs_moe_gather_quant", nat.ptr(src), nat.dtype_code(src.dtype), H,
            nat.ptr(None if rows is None else rows.contiguous()), A, H, nat.ptr(q), nat.ptr(s), nat.stream_of(device),
        )
    return q, s


def _grouped_contract(rows_q, weights, weight_scales, starts, counts, group_slots):
    """Geometry checks of _grouped_fp8_shape_contract (qwen3_moe_cuda.py:2191-2255)."""
    if rows_q.ndim != 2:
        raise ValueError("grouped int8 source must have shape [rows, contraction]")
    if weights.ndim != 3:
        raise ValueError("grouped int8 weights must have shape [groups, output, contraction]")
    if starts.ndim != 1 or counts.ndim != 1 or starts.numel() != counts.numel():
        raise ValueError("grouped int8 starts and counts must be equal-length vectors")
    logical = int(starts.numel())
    physical, n_out, contraction = map(int, weights.shape)
    if logical < 1:
        raise ValueError("grouped int8 execution requires at least one logical group")
    if int(rows_q.shape[1]) != contraction:
        raise ValueError("grouped int8 source contraction differs from weight contraction")
    if tuple(weight_scales.shape) != (physical, n_out):
        raise ValueError("grouped int8 scales must have shape [physical_groups, output_features]")
    if weights.stride(2) != 1 or weights.stride(1) != contraction or weight_scales.stride(1) != 1:
        raise ValueError("grouped int8 weights and scales require contiguous rows")
    if group_slots is None:
        if physical != logical:
            raise ValueError("compact grouped int8 weights require one physical group per logical group")
    elif group_slots.ndim != 1 or int(group_slots.numel()) != logical:
        raise ValueError("grouped int8 slot binding must have one index per logical group")
    return logical, n_out, contraction


@torch.inference_mode()
def grouped_int8_mm(
    rows_q: torch.Tensor,
    row_scales: torch.Tensor,
    weights: torch.Tensor,
    weight_scales: torch.Tensor,
    starts: torch.Tensor,
    counts: torch.Tensor,
    *,
    group_slots: torch.Tensor | None = None,
    max_rows: int | None = None,
    swiglu: bool = False,
    out_dtype: torch.dtype = torch.bfloat16,
    row_ids: torch.Tensor | None = None,
) -> tuple[torch.Tensor, str]:
    """Ragged grouped ``out[start_g + m] = (acc * a_scale) * w_scale`` for each group g.

    With ``row_ids``, queue row ``r`` reads ``rows_q[row_ids[r]]`` and its scale (the
    gather ``index_select(0, token_ids)`` folded into the kernel; ``rows_q`` are then the
    T quantized source rows).

    ``weights[slot(g)]`` is ``[N, K]`` int8 (``weights`` may be a strided view into an
    expert-page arena); ``swiglu=True`` treats rows ``[0, N/2)`` as gate and ``[N/2, N)``
    as up and returns ``bf16(silu(gate) * up)`` of width ``N/2``.  ``max_rows`` bounds
    every group's row count as in the reference's grouped kernels
    (qwen3_moe_cuda.py:2257-2310); it defaults to the routed row count, as its callers
    pass (:2747), and only sizes the kernel's row tile.
    """
    G, n_w, K = _grouped_contract(rows_q, weights, weight_scales, starts, counts, group_slots)
    device = nat.require_device(rows_q, row_scales, weights, weight_scales, starts, counts, group_slots, row_ids)
    n_out = n_w // 2 if swiglu else n_w
    if swiglu and n_w % 2:
        raise ValueError("SwiGLU weights need an even number of rows")
    if row_ids is not None and row_ids.ndim != 1:
        raise ValueError("row_ids must be a vector")
    A = int(rows_q.shape[0]) if row_ids is None else int(row_ids.numel())
    out = torch.empty((A, n_out), dtype=out_dtype, device=device)
    st = starts.to(torch.int32).contiguous()
    ct = counts.to(torch.int32).contiguous()
    sl = None if group_slots is None else group_slots.to(torch.int32).contiguous()
    rows_bound = A if max_rows is None else int(max_rows)
    if rows_bound < 0:
        raise ValueError("max_rows must be non-negative")
    tail = (nat.ptr(weights), int(weights.stride(0)), nat.ptr(weight_scales), int(weight_scales.stride(0)), nat.ptr(st),
            nat.ptr(ct), nat.ptr(sl), G, n_out, K, rows_bound, int(bool(swiglu)), nat.ptr(out),
            nat.dtype_code(out_dtype), nat.stream_of(device))
    if row_ids is None:
        nat.call("qs_moe_grouped_gemm_i8", nat.ptr(rows_q), nat.ptr(row_scales), *tail)
    else:
        ids = row_ids.to(torch.int64).contiguous()
        nat.call("qs_moe_grouped_gemm_i8_rows", nat.ptr(rows_q), nat.ptr(row_scales), nat.ptr(ids),
                 int(rows_q.shape[0]), *tail)
    return out, IMPL_GROUPED


@torch.inference_mode()
def grouped_w8a16_mm(
    rows: torch.Tensor,
    weights: torch.Tensor,
    weight_scales: torch.Tensor,
    starts: torch.Tensor,
    counts: torch.Tensor,
    *,
    row_ids: torch.Tensor | None = None,
    group_slots: torch.Tensor | None = None,
    max_rows: int | None = None,
    swiglu: bool = False,
    out_dtype: torch.dtype = torch.bfloat16,
) -> tuple[torch.Tensor, str]:
    """Weight-only ragged grouped GEMM over int8 expert pages:
    ``out[start_g + m] = rows[start_g + m] @ bf16(weights[slot(g)] * scales)^T``.

    The counterpart of the reference's ``grouped_bf16_mm`` (qwen3_moe_cuda.py:2473-2510)
    with the experts' bf16 weights given as int8 codes and per-row scales, dequantized in
    registers to ``bf16(float(code) * scale)`` (the W8A16 weight contract); ``rows`` stay
    bf16, so no activation is quantized.  ``row_ids`` folds the gather
    ``source.index_select(0, token_ids)`` (qwen3_moe_cuda.py:3020) into the kernel:
    ``rows`` is then the unpermuted source and queue row ``r`` reads ``rows[row_ids[r]]``.
    ``swiglu=True`` returns ``bf16(silu(gate) * up)`` of width ``N/2`` as
    ``grouped_int8_mm`` does.
    """
    if rows.dtype != torch.bfloat16:
        raise ValueError("grouped W8A16 rows must be bfloat16")
    G, n_w, K = _grouped_contract(rows, weights, weight_scales, starts, counts, group_slots)
    device = nat.require_device(rows, weights, weight_scales, starts, counts, group_slots, row_ids)
    n_out = n_w // 2 if swiglu else n_w
    if swiglu and n_w % 2:
        raise ValueError("SwiGLU weights need an even number of rows")
    src = rows.contiguous()
    if row_ids is not None:
        if row_ids.ndim != 1:
            raise ValueError("row_ids must be a vector")
        ids = row_ids.to(torch.int64).contiguous()
        A = int(ids.numel())
    else:
        ids = None
        A = int(src.shape[0])
    out = torch.empty((A, n_out), dtype=out_dtype, device=device)
    st = starts.to(torch.int32).contiguous()
    ct = counts.to(torch.int32).contiguous()
    sl = None if group_slots is None else group_slots.to(torch.int32).contiguous()
    rows_bound = A if max_rows is None else int(max_rows)
    if rows_bound < 0:
        raise ValueError("max_rows must be non-negative")
    nat.call(
        "qs_moe_grouped_gemm_w8a16", nat.ptr(src), nat.ptr(ids), int(src.shape[0]), nat.ptr(weights),
        int(weights.stride(0)), nat.ptr(weight_scales), int(weight_scales.stride(0)), nat.ptr(st), nat.ptr(ct),
        nat.ptr(sl), G, n_out, K, rows_bound, int(bool(swiglu)), nat.ptr(out), nat.dtype_code(out_dtype),
        nat.stream_of(device),
    )
    return out, IMPL_GROUPED_W8A16


# ---- expert pages and backend ------------------------------------------------------------------


@dataclass(frozen=True)
class ExpertPageLayout:
    """One page per (layer, expert): gate_up codes [2I,H] | gate_up scales [2I] f32 |
    down codes [H,I] | down scales [H] f32, padded to 4096 B (qwen3_moe_cuda.py:187-224)."""

    hidden_size: int
    intermediate_size: int
    gate_up_codes_offset: int
    gate_up_codes_bytes: int
    gate_up_scales_offset: int
    gate_up_scales_bytes: int
    down_codes_offset: int
    down_codes_bytes: int
    down_scales_offset: int
    down_scales_bytes: int
    page_stride: int

    @classmethod
    def create(cls, hidden_size: int, intermediate_size: int) -> "ExpertPageLayout":
        gu_rows = 2 * intermediate_size
        gu_c = gu_rows * hidden_size
        gu_s_off = gu_c
        d_c_off = gu_s_off + gu_rows * 4
        d_c = hidden_size * intermediate_size
        d_s_off = d_c_off + d_c
        stride = _align(d_s_off + hidden_size * 4)
        return cls(hidden_size, intermediate_size, 0, gu_c, gu_s_off, gu_rows * 4, d_c_off, d_c, d_s_off,
                   hidden_size * 4, stride)

    @classmethod
    def from_dict(cls, payload: dict) -> "ExpertPageLayout":
        return cls(**{name: int(payload[name]) for name in cls.__dataclass_fields__})

    def as_dict(self) -> dict[str, int]:
        return {name: int(getattr(self, name)) for name in self.__dataclass_fields__}


class Int8ExpertLayer:
    """All experts of one layer in one HBM arena laid out as ``ExpertPageLayout`` pages."""

    def __init__(self, arena: torch.Tensor, layout: ExpertPageLayout, num_experts: int):
        if arena.dtype != torch.uint8 or arena.numel() < layout.page_stride * num_experts:
            raise ValueError("expert arena too small for the page layout")
        self.arena = arena
        self.layout = layout
        self.num_experts = num_experts
        L, E = layout, num_experts
        H, I = L.hidden_size, L.intermediate_size
        ps = L.page_stride
        base = arena.view(torch.int8)
        # strided [E, N, K] views into the pages (no copies); as_strided offsets count from
        # the start of the storage, so the arena's own offset (a slab inside a larger
        # allocation) is added
        o8 = base.storage_offset()
        self.gate_up = base.as_strided((E, 2 * I, H), (ps, H, 1), o8 + L.gate_up_codes_offset)
        self.down = base.as_strided((E, H, I), (ps, I, 1), o8 + L.down_codes_offset)
        fl = arena.view(torch.float32)
        o32 = fl.storage_offset()
        self.gate_up_scales = fl.as_strided((E, 2 * I), (ps // 4, 1), o32 + L.gate_up_scales_offset // 4)
        self.down_scales = fl.as_strided((E, H), (ps // 4, 1), o32 + L.down_scales_offset // 4)

    @classmethod
    def from_arrays(cls, gate_up, gate_up_scales, down, down_scales, device) -> "Int8ExpertLayer":
        """Pack ``[E,2I,H]`` / ``[E,2I]`` / ``[E,H,I]`` / ``[E,H]`` tensors into one page arena."""
        E, two_i, H = map(int, gate_up.shape)
        layout = ExpertPageLayout.create(H, two_i // 2)
        arena = torch.zeros(layout.page_stride * E, dtype=torch.uint8, device=device)
        layer = cls(arena, layout, E)
        layer.gate_up.copy_(gate_up.to(device))
        layer.gate_up_scales.copy_(gate_up_scales.to(device))
        layer.down.copy_(down.to(device))
        layer.down_scales.copy_(down_scales.to(device))
        return layer


class Int8ExpertBackend:
    """``backend.moe(layer, source, top_indices, top_weights)`` with int8 experts.

    Flow per layer (W8A8, the default): stable route compile and per-row int8
    quantization of the T source rows (one launch) -> grouped gate_up GEMM gathering the
    routed rows' codes, with the fused BF16 SwiGLU epilogue -> per-row requantization ->
    grouped down GEMM -> fixed rank-order reduce -> model dtype.  (Unaligned sources, or H
    not a multiple of 8 or above 8192, gather and quantize the A routed rows instead: the
    same codes.)

    ``w8a16=True`` is the weight-only flow of the reference's PackedBF16ExpertBackend.moe
    (qwen3_moe_cuda.py:2978-3046) over the same int8 pages: the routed bf16 rows are
    gathered inside the gate_up kernel, both grouped GEMMs multiply bf16 activations by
    weights dequantized to ``bf16(code * scale)``, and nothing is quantized per token.
    """

    def __init__(self, layers: list[Int8ExpertLayer] | None = None, *, dtype: torch.dtype = torch.bfloat16,
                 page_cache=None, w8a16: bool = False):
        """``layers``: resident expert layers; ``page_cache``: an ``expert_cache.ExpertPageCache``
        serving the layers' pages from host memory instead (slot-indirect binding);
        ``w8a16``: weight-only expert math (bf16 activations)."""
        if not layers and page_cache is None:
            raise ValueError("Int8ExpertBackend needs resident layers or a page cache")
        self.layers = layers or []
        self.page_cache = page_cache
        self.dtype = dtype
        self.w8a16 = bool(w8a16)
        self.stats = {"grouped_kernel_calls": 0, "route_compiler_calls": 0, "expert_assignments": 0}
        self._experts: dict[tuple[torch.device, int], torch.Tensor] = {}

    def _reduce_dtype(self) -> torch.dtype:
        # the reduce kernel rounds its fp32 sums to bf16 itself; other model dtypes are
        # cast from the fp32 result
        return self.dtype if self.dtype in (torch.float32, torch.bfloat16) else torch.float32

    def _expert_ids(self, device: torch.device, E: int) -> torch.Tensor:
        key = (device, E)
        ids = self._experts.get(key)
        if ids is None:
            ids = self._experts[key] = torch.arange(E, device=device)
        return ids

    @torch.inference_mode()
    def moe(
        self,
        layer: int,
        source: torch.Tensor,
        top_indices: torch.Tensor,
        top_weights: torch.Tensor,
        *,
        prefill: bool = False,
    ) -> torch.Tensor:
        if self.page_cache is not None:
            return self._moe_paged(layer, source, top_indices, top_weights, prefill=prefill)
        del prefill
        page = self.layers[layer]
        E = page.num_experts
        src_q = None
        # fp32 coefficients: the reduce widens them to fp32 anyway
        if self._fused_route_ok(source):
            token_ids, coef, starts, counts, inverse, _, q, s = _route_impl(
                top_indices, top_weights, E, True, coef_f32=True, quant_source=source
            )
            src_q = (q, s)
        else:
            token_ids, coef, starts, counts, inverse, _ = _route_impl(top_indices, top_weights, E, True, coef_f32=True)
        expert_output = self._experts_math(page, source, token_ids, starts, counts, None, src_q)
        out = stable_route_reduce(
            expert_output, coef, token_ids, counts, top_indices,
            self._expert_ids(source.device, E), inverse_assignments=inverse, out_dtype=self._reduce_dtype(),
        )
        self.stats["grouped_kernel_calls"] += 2
        self.stats["route_compiler_calls"] += 1
        self.stats["expert_assignments"] += int(top_indices.numel())
        return out.to(self.dtype)

    def _fused_route_ok(self, source) -> bool:
        """The W8A8 flow quantizes the T source rows in the route's launch and gathers them
        in the gate/up kernel when the rows are 16-byte aligned with H % 8 == 0."""
        H = int(source.shape[-1])
        return (not self.w8a16 and source.dtype in (torch.bfloat16, torch.float32) and H % 8 == 0 and H <= 8192
                and source.is_contiguous() and source.data_ptr() % 16 == 0)

    def _experts_math(self, page, source, token_ids, starts, counts, slots, src_q=None) -> torch.Tensor:
        """gate_up + SwiGLU and down over the routed queue; [A, H] in the model dtype.
        ``src_q``: the per-token codes and scales of the T source rows (route_quant), read
        through ``token_ids`` by the gate/up kernel."""
        if self.w8a16:
            src = source if source.dtype == torch.bfloat16 else source.to(torch.bfloat16)
            activated, _ = grouped_w8a16_mm(
                src, page.gate_up, page.gate_up_scales, starts, counts, row_ids=token_ids, group_slots=slots,
                swiglu=True,
            )
            expert_output, _ = grouped_w8a16_mm(
                activated, page.down, page.down_scales, starts, counts, group_slots=slots, out_dtype=self.dtype
            )
            return expert_output
        if src_q is not None:
            activated, _ = grouped_int8_mm(
                src_q[0], src_q[1], page.gate_up, page.gate_up_scales, starts, counts, group_slots=slots,
                swiglu=True, row_ids=token_ids,
            )
        else:
            rows_q, rows_s = quantize_rows(source, token_ids)
            activated, _ = grouped_int8_mm(
                rows_q, rows_s, page.gate_up, page.gate_up_scales, starts, counts, group_slots=slots, swiglu=True
            )
        act_q, act_s = quantize_rows(activated)
        expert_output, _ = grouped_int8_mm(
            act_q, act_s, page.down, page.down_scales, starts, counts, group_slots=slots, out_dtype=self.dtype
        )
        return expert_output

    def _moe_paged(self, layer, source, top_indices, top_weights, *, prefill: bool) -> torch.Tensor:
        """Same flow over the experts of this step only: the page cache binds each routed
        expert (a compact group id) to its cache slot, and the grouped GEMMs read the pages
        in place through ``group_slots``."""
        cache = self.page_cache
        transient = prefill and getattr(cache, "prefill_page_policy", None) == "transient-frequency-v1"
        table = None if transient else cache.acquire_layer_table(layer, top_indices, protect=not prefill)
        if transient:
            # the layer runs from the cache's transient slab (qwen3_moe_cuda.py:2850-2854)
            selected, page, slots = cache.acquire_transient_prefill(layer, top_indices)
            route_idx = torch.searchsorted(selected, top_indices)
            E = int(selected.numel())
        elif table is not None:
            # every page of the layer is resident: groups are the expert ids themselves and
            # the device slot table binds them, with no host synchronisation
            page, slots = table
            E = int(slots.numel())
            selected = self._expert_ids(source.device, E)
            route_idx = top_indices
        else:
            selected, page, slots = cache.acquire_slot_binding(layer, top_indices, protect=not prefill)
            route_idx = torch.searchsorted(selected, top_indices)
            E = int(selected.numel())
        src_q = None
        if self._fused_route_ok(source):
            token_ids, coef, starts, counts, inverse, _, q, s = _route_impl(
                route_idx, top_weights, E, True, coef_f32=True, quant_source=source
            )
            src_q = (q, s)
        else:
            token_ids, coef, starts, counts, inverse, _ = _route_impl(route_idx, top_weights, E, True, coef_f32=True)
        expert_output = self._experts_math(page, source, token_ids, starts, counts, slots, src_q)
        out = stable_route_reduce(
            expert_output, coef, token_ids, counts, top_indices, selected, inverse_assignments=inverse,
            out_dtype=self._reduce_dtype(),
        )
        cache.release()
        self.stats["grouped_kernel_calls"] += 2
        self.stats["route_compiler_calls"] += 1
        self.stats["expert_assignments"] += int(top_indices.numel())
        return out.to(self.dtype)
