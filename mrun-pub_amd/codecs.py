"""Offline QStore codecs on the device (the store writer's row quantizers).

Same outputs, bit for bit, as the reference's numpy writers:

* ``quant_row_int8``  -- ``_quant_row_int8`` src/mrun/engine/kernels/qstore_build.py:496-501
* ``quant_row_int3``  -- ``_quant_row_int3`` + ``_pack_int3_codes`` qstore_int3.py:30-56
* ``quant_row_int2``  -- ``_quant_row_int2`` + ``_pack_int2_codes`` qstore_int2.py:24-63

Inputs are fp32 ``[out, in]`` tensors on a HIP device; outputs stay on that device, ready
for ``store.write_qstore`` after a host copy or for direct use as resident pages.
"""

from __future__ import annotations

import torch

from . import _native as nat

GROUP = 128  # the reference writers' default group (qstore_int3.py:26, qstore_int2.py:20)


def _check(W: torch.Tensor) -> tuple[int, int, torch.device]:
    if W.dtype != torch.float32 or W.ndim != 2:
        raise ValueError("codec input must be a float32 [out, in] tensor")
    device = nat.require_device(W)
    if int(W.shape[1]) < 1:
        raise ValueError("codec input needs at least one column")
    return int(W.shape[0]), int(W.shape[1]), device


@torch.inference_mode()
def quant_row_int8(W: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric int8: ``(q int8 [out, in], scale float32 [out])``."""
    n, k, device = _check(W)
    W = W if W.stride(1) == 1 else W.contiguous()
    q = torch.empty((n, k), dtype=torch.int8, device=device)
    s = torch.empty(n, dtype=torch.float32, device=device)
    nat.call("qs_quant_rows_int8", nat.ptr(W), int(W.stride(0)), n, k, nat.ptr(q), k, nat.ptr(s),
             nat.stream_of(device))
    return q, s


def _lowbit(W: torch.Tensor, bits: int, G: int) -> tuple[torch.Tensor, torch.Tensor]:
    n, k, device = _check(W)
    if isinstance(G, bool) or not isinstance(G, int) or G < 1:
        raise ValueError("group size must be a positive integer")
    W = W if W.stride(1) == 1 else W.contiguous()
    row_bytes = (k * bits + 7) // 8
    ng = (k + G - 1) // G
    packed = torch.empty((n, row_bytes), dtype=torch.uint8, device=device)
    scales = torch.empty((n, ng), dtype=torch.float32, device=device)
    codes = torch.empty(max(n * k, 1), dtype=torch.uint8, device=device)
    nat.call("qs_quant_rows_lowbit", nat.ptr(W), int(W.stride(0)), n, k, bits, G, nat.ptr(packed), row_bytes,
             nat.ptr(scales), nat.ptr(codes), nat.stream_of(device))
    return packed, scales


@torch.inference_mode()
def quant_row_int3(W: torch.Tensor, G: int = GROUP) -> tuple[torch.Tensor, torch.Tensor]:
    """Group-wise symmetric int3: ``(packed uint8 [out, ceil(in*3/8)], scales [out, ceil(in/G)])``."""
    return _lowbit(W, 3, G)


@torch.inference_mode()
def quant_row_int2(W: torch.Tensor, G: int = GROUP) -> tuple[torch.Tensor, torch.Tensor]:
    """Group-wise TWN ternary int2: ``(packed uint8 [out, ceil(in*2/8)], scales [out, ceil(in/G)])``."""
    return _lowbit(W, 2, G)
