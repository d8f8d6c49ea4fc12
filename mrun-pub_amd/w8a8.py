"""W8A8 (int8 weight x int8 activation) matmul on gfx950 -- drop-in for
src/mrun/engine/kernels/w8a8.py.

The whole contract runs on the device through ``csrc/qs_w8a8.hip``:

1. outlier columns: ``protect_idx`` or the top-``protect_k`` columns by column max-abs
   (``qs_outlier_topk``), with the keep mask that zeroes them for quantization;
2. the exact fp32 side path operands ``x[:, P]`` and ``float(q_w[:, P]) * sc_w``
   (``qs_w8a8_side_gather``);
3. per-token activation quantization ``s = max|x*keep|/127``, ``q = clamp(rint(x*keep/s))``
   (``qs_act_quant_i8``, bit-exact with the reference recipe, w8a8.py:118-121);
4. int8 x int8 -> int32 MFMA GEMM with the epilogue
   ``y = side + (float(acc) * act_scale) * sc_w`` (``qs_w8a8_gemm``), fp32 or bf16 out.

``_int8_gemm`` exposes the raw int32 accumulators (``qs_gemm_i8i8_i32``); they equal the
exact integer product.  ``enable_w8a8`` / ``disable_w8a8`` keep the reference's public
names and keywords (w8a8.py:145-187) over a binding object of this module's own design.
"""

from __future__ import annotations

from typing import Any

import torch

from . import _native as nat

IMPL_W8A8 = "hip-gfx950-w8a8-mfma-i8-v1"


def _check_weight(q_w: torch.Tensor, sc_w: torch.Tensor) -> tuple[int, int]:
    if q_w.dtype != torch.int8 or q_w.ndim != 2 or not q_w.is_contiguous():
        raise ValueError("q_w must be a contiguous int8 [out, in] tensor")
    if sc_w.dtype != torch.float32 or sc_w.shape != (q_w.shape[0],) or not sc_w.is_contiguous():
        raise ValueError("sc_w must be a contiguous float32 [out] tensor")
    return int(q_w.shape[0]), int(q_w.shape[1])


@torch.inference_mode()
def _int8_gemm(q_x: torch.Tensor, q_w: torch.Tensor, use_int_mm: bool = True) -> torch.Tensor:
    """``[T,in] int8 @ [out,in] int8^T -> [T,out] int32`` (w8a8.py:33-64), exact.

    ``use_int_mm`` is accepted for signature compatibility; the MFMA kernel is exact for
    every shape, so no padding or lossy fallback exists.
    """
    del use_int_mm
    if q_x.dtype != torch.int8 or q_w.dtype != torch.int8 or q_x.ndim != 2 or q_w.ndim != 2:
        raise ValueError("_int8_gemm takes int8 [T, in] and int8 [out, in]")
    if q_x.shape[1] != q_w.shape[1]:
        raise ValueError("_int8_gemm contraction mismatch")
    device = nat.require_device(q_x, q_w)
    qx = q_x.contiguous()
    qw = q_w.contiguous()
    T, K = map(int, qx.shape)
    N = int(qw.shape[0])
    acc = torch.empty((T, N), dtype=torch.int32, device=device)
    if T:
        nat.call("qs_gemm_i8i8_i32", nat.ptr(qx), nat.ptr(qw), nat.ptr(acc), T, N, K, nat.stream_of(device))
    return acc


@torch.inference_mode()
def quantize_activation(
    x: torch.Tensor, keep: torch.Tensor | None = None
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token int8 codes ``[T, in]`` and fp32 scales ``[T]`` (w8a8.py:118-121)."""
    K = int(x.shape[-1])
    x2 = x.reshape(-1, K).contiguous()
    device = nat.require_device(x2, keep)
    T = int(x2.shape[0])
    q = torch.empty((T, K), dtype=torch.int8, device=device)
    s = torch.empty(T, dtype=torch.float32, device=device)
    if T:
        nat.call(
            "qs_act_quant_i8",
            nat.ptr(x2),
            nat.dtype_code(x2.dtype),
            K,
            nat.ptr(keep),
            nat.ptr(q),
            nat.ptr(s),
            T,
            K,
            nat.stream_of(device),
        )
    return q, s


def _fused_front_end_ok(x2: torch.Tensor, protect_k: int, inn: int) -> bool:
    """qs_w8a8_protect_quant's limits: at most 16 protected columns, K a multiple of the
    16-byte element count and at most 8192 (4096 for fp32), 16-byte aligned rows."""
    e = 4 if x2.dtype == torch.float32 else 8
    return (min(int(protect_k), inn) <= 16 and inn % e == 0 and inn <= 64 * 16 * e and inn <= 8192
            and x2.data_ptr() % 16 == 0)


@torch.inference_mode()
def w8a8_matmul(
    q_w: torch.Tensor,
    sc_w: torch.Tensor,
    x: torch.Tensor,
    *,
    protect_idx: torch.Tensor | None = None,
    protect_k: int = 0,
    use_int_mm: bool = True,
    out_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """``x @ (q_w * sc_w[:,None]).T`` via int8 x int8 with an fp32 outlier side path.

    Same arguments and fp32 result as the reference ``w8a8_matmul`` (w8a8.py:67-125);
    ``out_dtype=torch.bfloat16`` rounds the same fp32 value to bf16 in the epilogue.
    """
    del use_int_mm
    out, inn = _check_weight(q_w, sc_w)
    if int(x.shape[-1]) != inn:
        raise ValueError("activation width does not match q_w")
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError(f"activation dtype {x.dtype} not supported")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("out_dtype must be float32 or bfloat16")
    device = nat.require_device(q_w, sc_w, x)
    x2 = x.reshape(-1, inn).contiguous()
    T = int(x2.shape[0])
    y = torch.empty((T, out), dtype=out_dtype, device=device)
    if T == 0:
        return y.reshape(*x.shape[:-1], out)
    stream = nat.stream_of(device)
    xdt = nat.dtype_code(x2.dtype)

    keep = None
    idx = None
    if protect_idx is None and protect_k > 0 and _fused_front_end_ok(x2, protect_k, inn):
        # column maxima, then selection + quantization + side operands in one launch
        k = min(int(protect_k), inn)
        colws = torch.empty(((T + 1023) // 1024) * inn, dtype=torch.float32, device=device)
        q_x = torch.empty((T, inn), dtype=torch.int8, device=device)
        act_scale = torch.empty(T, dtype=torch.float32, device=device)
        xp = torch.empty((T, k), dtype=torch.float32, device=device)
        wp = torch.empty((out, k), dtype=torch.float32, device=device)
        nat.call("qs_w8a8_protect_quant", nat.ptr(x2), xdt, inn, T, inn, k, nat.ptr(q_w), nat.ptr(sc_w), out,
                 nat.ptr(colws), nat.ptr(q_x), nat.ptr(act_scale), nat.ptr(xp), nat.ptr(wp), None, None, stream)
        nat.call("qs_w8a8_gemm", nat.ptr(q_x), nat.ptr(act_scale), nat.ptr(q_w), nat.ptr(sc_w), nat.ptr(xp),
                 nat.ptr(wp), k, nat.ptr(y), nat.dtype_code(out_dtype), T, out, inn, stream)
        return y.reshape(*x.shape[:-1], out)
    if protect_idx is None and protect_k > 0:
        k = min(int(protect_k), inn)
        colmax = torch.empty(inn, dtype=torch.float32, device=device)
        idx = torch.empty(k, dtype=torch.int64, device=device)
        keep = torch.empty(inn, dtype=torch.float32, device=device)
        nat.call("qs_outlier_topk", nat.ptr(x2), xdt, inn, T, inn, k, nat.ptr(colmax), nat.ptr(idx), nat.ptr(keep), stream)
    elif protect_idx is not None:
        idx = torch.as_tensor(protect_idx, dtype=torch.long, device=device).reshape(-1).contiguous()
        if idx.numel() == 0:
            idx = None
        else:
            lo, hi = int(idx.min()), int(idx.max())
            if lo < 0 or hi >= inn:
                raise IndexError("protect_idx out of range for the activation width")
            keep = torch.ones(inn, dtype=torch.float32, device=device)
            keep[idx] = 0.0
    P = 0 if idx is None else int(idx.numel())
    if P > 64:
        raise ValueError("at most 64 protected columns are supported")
    xp = wp = None
    if P:
        xp = torch.empty((T, P), dtype=torch.float32, device=device)
        wp = torch.empty((out, P), dtype=torch.float32, device=device)
        nat.call("qs_w8a8_side_gather", nat.ptr(x2), xdt, inn, nat.ptr(q_w), nat.ptr(sc_w), nat.ptr(idx), P, T, out, inn, nat.ptr(xp), nat.ptr(wp), stream)
    q_x, act_scale = quantize_activation(x2, keep)
    nat.call(
        "qs_w8a8_gemm",
        nat.ptr(q_x),
        nat.ptr(act_scale),
        nat.ptr(q_w),
        nat.ptr(sc_w),
        nat.ptr(xp),
        nat.ptr(wp),
        P,
        nat.ptr(y),
        nat.dtype_code(out_dtype),
        T,
        out,
        inn,
        stream,
    )
    return y.reshape(*x.shape[:-1], out)


# ---- opt-in store hook (public names and keywords of w8a8.py:130-187) ----------------
#
# ``enable_w8a8`` attaches one ``_W8A8Binding`` to the store instance.  The binding owns
# the settings and the matmul the store had before; the store's ``matmul`` attribute is a
# small callable that routes qrow blocks through ``w8a8_matmul`` and everything else to
# that saved matmul.  A second ``enable_w8a8`` only replaces the settings (the saved
# matmul stays the one from before the first call), and ``disable_w8a8`` puts back exactly
# the attribute state the store had.  Any store that exposes ``compact_page(name)`` (int8
# codes + fp32 scales on the device) and ``block_kind(name)`` can be switched.


class _W8A8Binding:
    __slots__ = ("store", "previous", "had_instance_attr", "protect_k", "protect_lists", "use_int_mm")

    def __init__(self, store: Any, protect_k: int, protect_lists: dict[str, Any], use_int_mm: bool):
        self.store = store
        self.had_instance_attr = "matmul" in vars(store)
        self.previous = store.matmul
        self.configure(protect_k, protect_lists, use_int_mm)

    def configure(self, protect_k: int, protect_lists: dict[str, Any], use_int_mm: bool) -> None:
        self.protect_k = int(protect_k)
        self.protect_lists = dict(protect_lists)
        self.use_int_mm = bool(use_int_mm)

    def __call__(self, name: str, x: torch.Tensor) -> torch.Tensor:
        if self.store.block_kind(name) != "qrow":
            return self.previous(name, x)
        page = self.store.compact_page(name)
        return w8a8_matmul(page.codes, page.scales, x, protect_idx=self.protect_lists.get(name),
                           protect_k=self.protect_k, use_int_mm=self.use_int_mm)


def enable_w8a8(
    store: Any,
    *,
    protect_k: int = 8,
    protect_lists: dict[str, Any] | None = None,
    use_int_mm: bool = True,
) -> Any:
    """Route the qrow projections of one store through W8A8 (reversible, idempotent).

    ``protect_k`` outlier columns per call stay in fp32; ``protect_lists`` maps block names
    to fixed column lists, which take the place of the per-call top-k for those blocks.
    """
    for attr in ("compact_page", "block_kind"):
        if not callable(getattr(store, attr, None)):
            raise TypeError(f"enable_w8a8 needs a store with {attr}(name)")
    binding = vars(store).get("_w8a8_binding")
    if binding is None:
        binding = _W8A8Binding(store, protect_k, protect_lists or {}, use_int_mm)
        store._w8a8_binding = binding
        store.matmul = binding
    else:
        binding.configure(protect_k, protect_lists or {}, use_int_mm)
    return store


def disable_w8a8(store: Any) -> Any:
    """Give the store back the matmul it had before :func:`enable_w8a8` (no-op if not enabled)."""
    binding = vars(store).pop("_w8a8_binding", None)
    if binding is not None:
        if binding.had_instance_attr:
            store.matmul = binding.previous
        else:
            del store.matmul
    return store
