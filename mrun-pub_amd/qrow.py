"""int8 row-scaled (qrow) linears on gfx950: the fused dequant+matmul operator surface.

Mirrors the reference kernel-level API
(src/mrun/engine/kernels/dense_qstore_cuda.py:78-101, 1003-1153) with the HIP kernels of
``csrc/qs_qrow.hip`` underneath:

* ``CompactQRowPage``        -- device-resident ``(codes int8[rows, K], scales f32[rows])``.
* ``fused_qrow_matmul``       -- ``y = x @ (bf16|fp16|fp32)(codes * scales)^T``.
* ``fused_qrow_swiglu``       -- paired gate/up projections with the BF16 SwiGLU epilogue.
* ``qrow_dequant``            -- the materialized weight (``_dequant_qrow``, qstore.py:385).

There is no CPU or "reference-materialized" branch: CPU tensors raise ``ValueError`` and a
missing native library raises ``RuntimeError`` (the reference's ``require_triton`` fail-closed
behaviour, dense_qstore_cuda.py:1125-1128, is therefore always in force).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native as nat

IMPL_W8A16 = "hip-gfx950-w8a16-qrow-v1"
IMPL_FP32 = "hip-gfx950-qrow-fp32-v1"
IMPL_SWIGLU = "hip-gfx950-paired-w8a16-swiglu-bf16-v1"
IMPL_TOP2 = "hip-gfx950-w8a16-qrow-block-top2-v1"
IMPL_TOP2_FP32 = "hip-gfx950-qrow-fp32-block-top2-v1"
IMPL_RERANK_SUFFIX = "+fp32-candidate-rerank-v1"

_ACT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _tensor_bytes(tensor: torch.Tensor) -> int:
    return int(tensor.numel() * tensor.element_size())


@dataclass(frozen=True)
class CompactQRowPage:
    """Row range ``[start_row, end_row)`` of one qrow block, codes and scales in HBM.

    Same fields and byte accounting as the reference ``CompactQRowPage``
    (dense_qstore_cuda.py:78-101).
    """

    name: str
    start_row: int
    end_row: int
    in_features: int
    codes: torch.Tensor
    scales: torch.Tensor

    @property
    def out_features(self) -> int:
        return self.end_row - self.start_row

    @property
    def compact_bytes(self) -> int:
        return _tensor_bytes(self.codes) + _tensor_bytes(self.scales)

    @property
    def expanded_fp32_bytes(self) -> int:
        return self.out_features * self.in_features * 4

    def expanded_compute_bytes(self, dtype: torch.dtype) -> int:
        return self.out_features * self.in_features * torch.empty((), dtype=dtype).element_size()


def _check_codes(codes: torch.Tensor, scales: torch.Tensor) -> tuple[int, int]:
    if codes.dtype != torch.int8 or codes.ndim != 2:
        raise ValueError("qrow codes must be int8 [out, in]")
    if scales.dtype != torch.float32 or scales.ndim != 1 or scales.numel() != codes.shape[0]:
        raise ValueError("qrow scales must be float32 [out]")
    if not codes.is_contiguous() or not scales.is_contiguous():
        raise ValueError("qrow codes and scales must be contiguous")
    return int(codes.shape[0]), int(codes.shape[1])


@torch.inference_mode()
def qrow_dequant(
    codes: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype = torch.float32
) -> torch.Tensor:
    """``dtype(float32(codes) * scales[:, None])`` on the device (bit-exact widen+scale)."""
    n, k = _check_codes(codes, scales)
    device = nat.require_device(codes, scales)
    out = torch.empty((n, k), dtype=dtype, device=device)
    nat.call(
        "qs_qrow_dequant",
        nat.ptr(codes),
        nat.ptr(scales),
        nat.ptr(out),
        nat.dtype_code(dtype),
        n,
        k,
        k,
        nat.stream_of(device),
    )
    return out


def normalize_row_ids(ids, n_rows: int):
    """Host row indices of an embedding lookup: any integer array, negative values count
    from the end as numpy indexing does; IndexError outside ``[-n_rows, n_rows)``."""
    import numpy as np

    idx = np.asarray(ids)
    if idx.dtype.kind not in "iu":
        raise TypeError("embedding row ids must be integers")
    idx = idx.astype(np.int64)
    if idx.size and (int(idx.min()) < -n_rows or int(idx.max()) >= n_rows):
        raise IndexError(f"embedding row id out of range for {n_rows} rows")
    return np.where(idx < 0, idx + n_rows, idx), idx.shape


@torch.inference_mode()
def qrow_embed_rows(codes: torch.Tensor, scales: torch.Tensor, ids) -> torch.Tensor:
    """fp32 rows ``float(codes[ids]) * scales[ids]`` with shape ``[*ids.shape, in]``
    (the qrow branch of ``QStore.embed_rows``, qstore.py:1099-1128)."""
    n, k = _check_codes(codes, scales)
    flat, shape = normalize_row_ids(ids, n)
    device = nat.require_device(codes, scales)
    rows = torch.from_numpy(flat.reshape(-1)).to(device)
    out = torch.empty((rows.numel(), k), dtype=torch.float32, device=device)
    if rows.numel():
        nat.call("qs_qrow_dequant_rows", nat.ptr(codes), nat.ptr(scales), n, k, nat.ptr(rows),
                 int(rows.numel()), nat.ptr(out), nat.stream_of(device))
    return out.reshape(*shape, k)


def _out_buffer(out: torch.Tensor | None, m: int, n: int, dtype: torch.dtype, device) -> torch.Tensor:
    """A caller's output buffer (contiguous ``[m, n]`` of ``dtype`` on ``device``, any leading
    shape) or a fresh one."""
    if out is None:
        return torch.empty((m, n), dtype=dtype, device=device)
    if out.dtype != dtype or out.device != device or not out.is_contiguous() or out.numel() != m * n:
        raise ValueError(f"out must be a contiguous {dtype} tensor of {m}x{n} elements on {device}")
    return out.view(m, n)


# The batched kernels (k_bd2: an LDS activation slice shared by a workgroup's weight rows,
# weights streamed into VGPRs, K split only for rows longer than 2048) serve every
# bf16/f16 call with at least 16 activation rows: in same-box A/B timings of the config-2
# shapes they match or beat the 16-row-tile kernels at M = 16 and beat them at M = 32
# (1536 x 8960: 25.4 -> 11.5 us, paired SwiGLU 8960 x 1536: 18.5 -> 14.3 us).
# Fewer rows take them where they measured faster than the 16-row-tile kernels that serve
# M 5..15 (same box, config-2 shapes): the paired SwiGLU from 5 rows (11.7 -> 10.7 us at
# M = 8, 13.4 -> 10.8 at M = 12), rows longer than 2048 from 8 (1536 x 8960: 10.6 ->
# 9.9 us at M = 8, 15.2 -> 10.1 at M = 12); short rows keep the tiles below 16 (1536 x 1536
# at M = 12: 4.89 against 5.03 us).  M <= 4 stays on the register-activation GEMV, whose
# rows equal single-row results bit for bit (and whose chained M = 4 pass is faster).
BATCHED_MIN_M = 16
BATCHED_MIN_M_SWIGLU = 5
BATCHED_MIN_M_LONG = 8
BATCHED_MAX_K = 16384


def _batched_eligible(x2: torch.Tensor, codes: list[torch.Tensor], swiglu: bool = False) -> bool:
    m, k = int(x2.shape[0]), int(x2.shape[1])
    ns = [int(c.shape[0]) for c in codes]
    min_m = BATCHED_MIN_M_SWIGLU if swiglu else (BATCHED_MIN_M_LONG if k > 2048 else BATCHED_MIN_M)
    return (x2.dtype in (torch.bfloat16, torch.float16) and (not swiglu or x2.dtype == torch.bfloat16)
            and m >= min_m and k % 128 == 0 and k <= BATCHED_MAX_K
            and (k <= 2048 or all(n % 4 == 0 for n in ns))
            and x2.stride(0) == k and x2.data_ptr() % 16 == 0 and all(c.data_ptr() % 16 == 0 for c in codes))


def _run_batched(x2: torch.Tensor, pages: list[tuple[torch.Tensor, torch.Tensor]], outs: list[torch.Tensor],
                 swiglu: bool) -> None:
    """``qs_qrow_matmul_batched`` / ``qs_qrow_swiglu_batched`` over row batches of <= 32,
    with a workspace for the K-slice partial sums (the split depends on N and K only)."""
    device = x2.device
    m_all, k = int(x2.shape[0]), int(x2.shape[1])
    ns = [int(c.shape[0]) for c, _ in pages[:1 if swiglu else len(pages)]]
    stream = nat.stream_of(device)
    n_arr = nat.int64_array(ns)
    lib = nat.load()
    ws_bytes = int(lib.qs_qrow_batched_workspace_bytes(min(32, m_all), len(ns), n_arr, k, int(swiglu)))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=device)
    for m0 in range(0, m_all, 32):
        mm = min(32, m_all - m0)
        xb = x2[m0:m0 + mm]
        if swiglu:
            (gc, gs), (uc, us) = pages
            nat.call("qs_qrow_swiglu_batched", nat.ptr(xb), k, nat.ptr(gc), nat.ptr(gs), nat.ptr(uc), nat.ptr(us),
                     nat.ptr(outs[0][m0:]), ns[0], mm, ns[0], k, nat.ptr(ws), ws_bytes, stream)
        else:
            nat.call("qs_qrow_matmul_batched", nat.ptr(xb), nat.dtype_code(x2.dtype), k, len(pages),
                     nat.pointer_array([nat.ptr(c) for c, _ in pages]), nat.pointer_array([nat.ptr(sc) for _, sc in pages]),
                     nat.pointer_array([nat.ptr(o[m0:]) for o in outs]), n_arr, n_arr, mm, k, nat.ptr(ws), ws_bytes,
                     stream)


@torch.inference_mode()
def qrow_matmul(
    codes: torch.Tensor, scales: torch.Tensor, x: torch.Tensor, *, row_stable: bool = False,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``x[..., K] @ W^T`` with the dtype contract of ``qs_qrow_matmul``.

    fp32 activations: fp32 weights and output (QStore compute contract, qstore.py:1082-1092).
    bf16 / fp16 activations: weights rounded per element to the activation dtype, fp32
    accumulation, output in the activation dtype (W8A16, dense_qstore_cuda.py:467-512).
    ``row_stable=True`` selects the batch-invariant lane (``matmul_row_stable``,
    qstore.py:49-76): every row equals its own ``M = 1`` result bit for bit.  ``out``: an
    optional preallocated output (it must not overlap ``x``).
    """
    n, k = _check_codes(codes, scales)
    if x.dtype not in _ACT_DTYPES:
        raise ValueError(f"activation dtype {x.dtype} not supported")
    if x.ndim < 1 or int(x.shape[-1]) != k:
        raise ValueError("activation width does not match compact qrow page")
    device = nat.require_device(codes, scales, x)
    flat = x.reshape(-1, k)
    if not flat.is_contiguous():
        flat = flat.contiguous()
    m = int(flat.shape[0])
    y = _out_buffer(out, m, n, x.dtype, device)
    if m and not row_stable and _batched_eligible(flat, [codes]):
        _run_batched(flat, [(codes, scales)], [y], swiglu=False)
    elif m:
        nat.call(
            "qs_qrow_matmul_row_stable" if row_stable else "qs_qrow_matmul",
            nat.ptr(flat),
            nat.dtype_code(x.dtype),
            k,
            nat.ptr(codes),
            nat.ptr(scales),
            nat.ptr(y),
            n,
            m,
            n,
            k,
            nat.stream_of(device),
        )
    return y.reshape(*x.shape[:-1], n)


@torch.inference_mode()
def qrow_matmul_multi(
    pages: list[tuple[torch.Tensor, torch.Tensor]], x: torch.Tensor,
    out: list[torch.Tensor] | None = None,
) -> list[torch.Tensor]:
    """Several linears over one activation in a single launch (q/k/v); ``out``: optional
    preallocated outputs, one per linear."""
    if not 1 <= len(pages) <= 4:
        raise ValueError("qrow_matmul_multi takes 1..4 linears")
    k = int(x.shape[-1])
    shapes = [_check_codes(c, s) for c, s in pages]
    if any(kk != k for _, kk in shapes):
        raise ValueError("all linears must share the activation width")
    if x.dtype not in _ACT_DTYPES:
        raise ValueError(f"activation dtype {x.dtype} not supported")
    device = nat.require_device(x, *[t for p in pages for t in p])
    flat = x.reshape(-1, k).contiguous()
    m = int(flat.shape[0])
    if out is not None and len(out) != len(pages):
        raise ValueError("one output buffer per linear")
    outs = [_out_buffer(None if out is None else out[i], m, n, x.dtype, device) for i, (n, _) in enumerate(shapes)]
    if m and _batched_eligible(flat, [c for c, _ in pages]):
        _run_batched(flat, pages, outs, swiglu=False)
    elif m:
        nat.call(
            "qs_qrow_matmul_multi",
            nat.ptr(flat),
            nat.dtype_code(x.dtype),
            k,
            len(pages),
            nat.pointer_array([nat.ptr(c) for c, _ in pages]),
            nat.pointer_array([nat.ptr(s) for _, s in pages]),
            nat.pointer_array([nat.ptr(o) for o in outs]),
            nat.int64_array([n for n, _ in shapes]),
            nat.int64_array([n for n, _ in shapes]),
            m,
            k,
            nat.stream_of(device),
        )
    return [o.reshape(*x.shape[:-1], o.shape[1]) for o in outs]


def _validate_block_m(block_m: int) -> None:
    # Same accepted values as the reference; the HIP kernels choose their own tiles.
    if block_m not in {16, 32, 64}:
        raise ValueError("block_m must be one of 16, 32, or 64")


@torch.inference_mode()
def fused_qrow_matmul(
    page: CompactQRowPage,
    activations: torch.Tensor,
    *,
    require_triton: bool = False,
    block_m: int = 16,
) -> tuple[torch.Tensor, str]:
    """Drop-in for ``fused_qrow_matmul`` (dense_qstore_cuda.py:1105-1153).

    Returns ``(y, implementation_tag)``.  ``require_triton`` is accepted for signature
    compatibility; the native path is the only path.
    """
    del require_triton
    if activations.shape[-1] != page.in_features:
        raise ValueError("activation width does not match compact qrow page")
    if page.codes.device != activations.device or page.scales.device != activations.device:
        raise ValueError("compact qrow page and activations must use one device")
    _validate_block_m(block_m)
    y = qrow_matmul(page.codes, page.scales, activations)
    return y, (IMPL_FP32 if activations.dtype == torch.float32 else IMPL_W8A16)


def _validate_paired_qrow_pages(
    gate_page: CompactQRowPage, up_page: CompactQRowPage, activations: torch.Tensor
) -> None:
    """Same checks and messages as dense_qstore_cuda.py:1016-1034."""
    if activations.ndim < 2 or activations.dtype is not torch.bfloat16:
        raise ValueError("paired SwiGLU requires BF16 activation rows")
    if gate_page.in_features != activations.shape[-1]:
        raise ValueError("activation width does not match paired compact qrow pages")
    if (
        gate_page.in_features != up_page.in_features
        or gate_page.out_features != up_page.out_features
        or gate_page.start_row != up_page.start_row
        or gate_page.end_row != up_page.end_row
    ):
        raise ValueError("gate/up compact qrow pages must have identical geometry")
    tensors = (gate_page.codes, gate_page.scales, up_page.codes, up_page.scales)
    if any(tensor.device != activations.device for tensor in tensors):
        raise ValueError("paired compact qrow pages and activations must use one device")


@torch.inference_mode()
def fused_qrow_swiglu(
    gate_page: CompactQRowPage,
    up_page: CompactQRowPage,
    activations: torch.Tensor,
    *,
    require_triton: bool = False,
    block_m: int = 16,
) -> tuple[torch.Tensor, str]:
    """Drop-in for ``fused_qrow_swiglu`` (dense_qstore_cuda.py:1053-1102)."""
    del require_triton
    _validate_block_m(block_m)
    return qrow_swiglu_into(gate_page, up_page, activations), IMPL_SWIGLU


@torch.inference_mode()
def qrow_swiglu_into(gate_page: CompactQRowPage, up_page: CompactQRowPage, activations: torch.Tensor,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """The paired SwiGLU of :func:`fused_qrow_swiglu`, optionally into a preallocated bf16
    ``out`` (which must not overlap the activations)."""
    _validate_paired_qrow_pages(gate_page, up_page, activations)
    n, k = _check_codes(gate_page.codes, gate_page.scales)
    _check_codes(up_page.codes, up_page.scales)
    device = nat.require_device(activations, gate_page.codes)
    flat = activations.reshape(-1, k).contiguous()
    m = int(flat.shape[0])
    y = _out_buffer(out, m, n, torch.bfloat16, device)
    if m and _batched_eligible(flat, [gate_page.codes, up_page.codes], swiglu=True):
        _run_batched(flat, [(gate_page.codes, gate_page.scales), (up_page.codes, up_page.scales)], [y], swiglu=True)
    elif m:
        nat.call(
            "qs_qrow_swiglu",
            nat.ptr(flat),
            k,
            nat.ptr(gate_page.codes),
            nat.ptr(gate_page.scales),
            nat.ptr(up_page.codes),
            nat.ptr(up_page.scales),
            nat.ptr(y),
            n,
            m,
            n,
            k,
            nat.stream_of(device),
        )
    return y.reshape(*activations.shape[:-1], n)


# ---- head: fused top-2 and fp32 candidate rerank ----------------------------------------------


def _semantic_row_count(page: CompactQRowPage, value: int | None) -> int:
    """Same checks and messages as dense_qstore_cuda.py:67-76."""
    if value is None:
        return page.out_features
    if isinstance(value, bool) or not isinstance(value, int):
        raise TypeError("semantic_row_count must be an integer or None")
    row_count = int(value)
    if row_count < 2 or row_count > page.out_features:
        raise ValueError("semantic_row_count must select at least two rows inside the compact page")
    return row_count


def _check_head(page: CompactQRowPage, activations: torch.Tensor) -> None:
    if activations.ndim < 2 or activations.shape[-1] != page.in_features:
        raise ValueError("activation shape does not match compact head page")
    if page.codes.device != activations.device or page.scales.device != activations.device:
        raise ValueError("head page and activations must use one device")


@torch.inference_mode()
def fused_qrow_top2(
    page: CompactQRowPage,
    activations: torch.Tensor,
    *,
    semantic_row_count: int | None = None,
    require_triton: bool = False,
    block_m: int = 16,
    block_n: int = 64,
) -> tuple[torch.Tensor, torch.Tensor, str, int]:
    """Drop-in for ``fused_qrow_top2`` (dense_qstore_cuda.py:1239-1317).

    Returns ``(indices, values, implementation, working_bytes)``: the two best rows of the
    semantic prefix of the page per activation row (int32 global row indices, fp32
    logits), without materializing logits.  ``require_triton`` and the tile arguments
    keep the reference's signature and checks; the native kernel picks its own tiles.
    """
    del require_triton
    _check_head(page, activations)
    if block_m not in {16, 32, 64} or block_n != 64:
        raise ValueError("supported head tiles are block_m in {16,32,64}, block_n=64")
    row_count = _semantic_row_count(page, semantic_row_count)
    if activations.dtype not in _ACT_DTYPES:
        raise ValueError(f"activation dtype {activations.dtype} not supported")
    n, k = _check_codes(page.codes, page.scales)
    device = nat.require_device(activations, page.codes)
    flat = activations.reshape(-1, k)
    if not flat.is_contiguous():
        flat = flat.contiguous()
    m = int(flat.shape[0])
    out_i = torch.empty((m, 2), dtype=torch.int32, device=device)
    out_v = torch.empty((m, 2), dtype=torch.float32, device=device)
    ws_bytes = int(nat.load().qs_qrow_top2_workspace_bytes(m, row_count))
    if m:
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
        nat.call(
            "qs_qrow_top2", nat.ptr(flat), nat.dtype_code(flat.dtype), k, nat.ptr(page.codes),
            nat.ptr(page.scales), m, row_count, k, int(page.start_row), nat.ptr(ws), ws_bytes,
            nat.ptr(out_i), nat.ptr(out_v), nat.stream_of(device),
        )
    shape = (*activations.shape[:-1], 2)
    tag = IMPL_TOP2_FP32 if activations.dtype == torch.float32 else IMPL_TOP2
    working = ws_bytes + m * 2 * (4 + 4)
    return out_i.reshape(shape), out_v.reshape(shape), tag, int(working)


def _rerank(page: CompactQRowPage, activations: torch.Tensor, candidate_indices: torch.Tensor,
            *, validate_candidate_bounds: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """Checks and messages of dense_qstore_cuda.py:1189-1210; scoring on the device."""
    if activations.ndim < 2 or activations.shape[-1] != page.in_features:
        raise ValueError("activation shape does not match compact head page")
    if candidate_indices.shape[:-1] != activations.shape[:-1]:
        raise ValueError("candidate rows must match the activation prefix shape")
    if candidate_indices.shape[-1] < 1:
        raise ValueError("at least one candidate is required")
    if candidate_indices.device != activations.device:
        raise ValueError("candidate indices and activations must use one device")
    if page.codes.device != activations.device or page.scales.device != activations.device:
        raise ValueError("head page and activations must use one device")
    if activations.dtype not in _ACT_DTYPES:
        raise ValueError(f"activation dtype {activations.dtype} not supported")
    n, k = _check_codes(page.codes, page.scales)
    device = nat.require_device(activations, page.codes)
    flat = activations.reshape(-1, k)
    if not flat.is_contiguous():
        flat = flat.contiguous()
    m = int(flat.shape[0])
    cand = candidate_indices.reshape(m, -1).to(torch.long).contiguous()
    c = int(cand.shape[1])
    if validate_candidate_bounds:
        local = cand - int(page.start_row)
        if bool(((local < 0) | (local >= page.out_features)).any().item()):
            raise ValueError("candidate index falls outside the compact head page")
    out_i = torch.empty(m, dtype=torch.long, device=device)
    out_v = torch.empty(m, dtype=torch.float32, device=device)
    if m:
        nat.call(
            "qs_qrow_rerank_fp32", nat.ptr(flat), nat.dtype_code(flat.dtype), k, nat.ptr(page.codes),
            nat.ptr(page.scales), n, k, int(page.start_row), nat.ptr(cand), c, m, nat.ptr(out_i),
            nat.ptr(out_v), nat.stream_of(device),
        )
    shape = activations.shape[:-1]
    return out_i.reshape(shape), out_v.reshape(shape)


@torch.inference_mode()
def rerank_qrow_candidates_fp32(
    page: CompactQRowPage, activations: torch.Tensor, candidate_indices: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """Drop-in for ``rerank_qrow_candidates_fp32`` (dense_qstore_cuda.py:1174-1186): score a
    shortlist in fp32 with exact dequant; returns ``(best_indices, best_values)``."""
    return _rerank(page, activations, candidate_indices, validate_candidate_bounds=True)


@torch.inference_mode()
def fused_qrow_reranked_argmax(
    page: CompactQRowPage,
    activations: torch.Tensor,
    *,
    semantic_row_count: int | None = None,
    require_triton: bool = False,
    block_m: int = 16,
    block_n: int = 64,
) -> tuple[torch.Tensor, torch.Tensor, str, int]:
    """Drop-in for ``fused_qrow_reranked_argmax`` (dense_qstore_cuda.py:1332-1374): fused
    top-two search, then fp32 reranking of the two candidates."""
    candidates, _, implementation, working = fused_qrow_top2(
        page, activations, semantic_row_count=semantic_row_count, require_triton=require_triton,
        block_m=block_m, block_n=block_n,
    )
    # the candidates come from the masked kernel above: no bounds revalidation (no sync)
    indices, values = _rerank(page, activations, candidates, validate_candidate_bounds=False)
    rows = activations.numel() // page.in_features
    rerank_bytes = rows * (2 * 8 + 8 + 4)
    return indices, values, implementation + IMPL_RERANK_SUFFIX, int(working + rerank_bytes)
