"""ctypes binding of ``libqstore_hip.so`` (the C ABI declared in include/qstore_hip.h).

The library is loaded lazily, AFTER torch, so that its ``libamdhip64`` dependency
resolves to the HIP runtime torch already mapped into the process (one runtime, one
set of streams).  There is no fallback: if the library is missing, every operator
raises ``RuntimeError``.

Status codes map onto the reference's error conventions
(src/mrun/engine/kernels/dense_qstore_cuda.py:1113-1128; qwen3_moe_cuda.py:2191-2255):
invalid arguments -> ``ValueError``; unsupported / runtime failures -> ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libqstore_hip.so"

QS_OK = 0
QS_ERR_INVALID = -1
QS_ERR_UNSUPPORTED = -2
QS_ERR_HIP = -3
QS_ERR_LIMIT = -4

QS_F32, QS_BF16, QS_F16, QS_I32, QS_I64 = 0, 1, 2, 3, 4

_DTYPE_CODE = {
    torch.float32: QS_F32,
    torch.bfloat16: QS_BF16,
    torch.float16: QS_F16,
    torch.int32: QS_I32,
    torch.int64: QS_I64,
}

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64

# name -> (restype, argtypes).  Kept in the order of include/qstore_hip.h.
SIGNATURES: dict[str, tuple] = {
    "qs_version": (_I, []),
    "qs_last_error": (ctypes.c_char_p, []),
    "qs_qrow_dequant": (_I, [_P, _P, _P, _I, _L, _L, _L, _P]),
    "qs_qrow_dequant_rows": (_I, [_P, _P, _L, _L, _P, _L, _P, _P]),
    "qs_qrow_matmul": (_I, [_P, _I, _L, _P, _P, _P, _L, _L, _L, _L, _P]),
    "qs_qrow_matmul_row_stable": (_I, [_P, _I, _L, _P, _P, _P, _L, _L, _L, _L, _P]),
    "qs_qrow_matmul_multi": (_I, [_P, _I, _L, _I, _P, _P, _P, _P, _P, _L, _L, _P]),
    "qs_qrow_batched_workspace_bytes": (ctypes.c_size_t, [_L, _I, _P, _L, _I]),
    "qs_qrow_matmul_batched": (_I, [_P, _I, _L, _I, _P, _P, _P, _P, _P, _L, _L, _P, ctypes.c_size_t, _P]),
    "qs_qrow_swiglu_batched": (_I, [_P, _L, _P, _P, _P, _P, _P, _L, _L, _L, _L, _P, ctypes.c_size_t, _P]),
    "qs_qrow_swiglu": (_I, [_P, _L, _P, _P, _P, _P, _P, _L, _L, _L, _L, _P]),
    "qs_qrow_top2_workspace_bytes": (ctypes.c_size_t, [_L, _L]),
    "qs_qrow_top2": (_I, [_P, _I, _L, _P, _P, _L, _L, _L, _L, _P, ctypes.c_size_t, _P, _P, _P]),
    "qs_qrow_top2_noalloc": (_I, [_P, _I, _L, _P, _P, _L, _L, _L, _L, _P, _P, _P]),
    "qs_qrow_rerank_fp32": (_I, [_P, _I, _L, _P, _P, _L, _L, _L, _P, _I, _L, _P, _P, _P]),
    "qs_quant_rows_int8": (_I, [_P, _L, _L, _L, _P, _L, _P, _P]),
    "qs_quant_rows_lowbit": (_I, [_P, _L, _L, _L, _I, _I, _P, _L, _P, _P, _P]),
    "qs_act_quant_i8": (_I, [_P, _I, _L, _P, _P, _P, _L, _L, _P]),
    "qs_outlier_topk": (_I, [_P, _I, _L, _L, _L, _I, _P, _P, _P, _P]),
    "qs_w8a8_side_gather": (_I, [_P, _I, _L, _P, _P, _P, _I, _L, _L, _L, _P, _P, _P]),
    "qs_w8a8_protect_quant": (_I, [_P, _I, _L, _L, _L, _I, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _P]),
    "qs_gemm_i8i8_i32": (_I, [_P, _P, _P, _L, _L, _L, _P]),
    "qs_w8a8_gemm": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _I, _L, _L, _L, _P]),
    "qs_moe_router": (_I, [_P, _I, _L, _I, _I, _I, _P, _P, _I, _P]),
    "qs_moe_route": (_I, [_P, _I, _P, _I, _L, _I, _I, _P, _P, _P, _P, _P, _P]),
    "qs_moe_route_quant": (_I, [_P, _I, _P, _I, _L, _I, _I, _P, _P, _P, _P, _P, _P, _I, _L, _L, _P, _P, _P]),
    "qs_expert_queue_build": (_I, [_P, _I, _P, _P, _P, _I, _P, _P, _L, _I, _L, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P]),
    "qs_expert_queue_scatter_workspace_bytes": (ctypes.c_size_t, [_L, _L]),
    "qs_expert_queue_scatter": (_I, [_P, _P, _P, _P, _P, _I, _L, _L, _L, _L, _P, ctypes.c_size_t, _P, _P, _P]),
    "qs_moe_gather_quant": (_I, [_P, _I, _L, _P, _L, _L, _P, _P, _P]),
    "qs_moe_grouped_gemm_i8": (_I, [_P, _P, _P, _L, _P, _L, _P, _P, _P, _I, _L, _L, _L, _I, _P, _I, _P]),
    "qs_moe_grouped_gemm_i8_rows": (_I, [_P, _P, _P, _L, _P, _L, _P, _L, _P, _P, _P, _I, _L, _L, _L, _I, _P, _I, _P]),
    "qs_moe_grouped_gemm_w8a16": (_I, [_P, _P, _L, _P, _L, _P, _L, _P, _P, _P, _I, _L, _L, _L, _I, _P, _I, _P]),
    "qs_moe_route_reduce": (_I, [_P, _I, _P, _P, _L, _I, _L, _P, _P]),
    "qs_moe_route_reduce_to": (_I, [_P, _I, _P, _P, _L, _I, _L, _P, _I, _P]),
    "qs_lowbit_dequant": (_I, [_P, _L, _P, _I, _P, _I, ctypes.c_float, _I, _I, _P, _L, _L, _P]),
    "qs_lowbit_workspace_bytes": (ctypes.c_size_t, [_I, _L, _L, _L, _I]),
    "qs_lowbit_gemv": (_I, [_P, _I, _L, _P, _L, _P, _I, _P, _I, ctypes.c_float, _I, _I, _P, _L, _L, _L, _L, _P, ctypes.c_size_t, _P]),
    "qs_pager_create": (_I, [_P, ctypes.c_size_t, _I, ctypes.c_size_t, ctypes.POINTER(_P)]),
    "qs_pager_destroy": (_I, [_P]),
    "qs_pager_slot_ptr": (_P, [_P, _I]),
    "qs_pager_submit": (_I, [_P, _I, _P, ctypes.c_size_t, ctypes.c_size_t]),
    "qs_pager_seal": (_I, [_P, _I]),
    "qs_pager_submit_run": (_I, [_P, _I, _I, _P]),
    "qs_pager_acquire": (_I, [_P, _I, _P]),
    "qs_pager_release": (_I, [_P, _I, _P]),
    "qs_pager_acquire_many": (_I, [_P, _P, _I, _P]),
    "qs_pager_release_many": (_I, [_P, _P, _I, _P]),
    "qs_pager_sync": (_I, [_P]),
    "qs_pager_slot_landed": (_I, [_P, _I]),
    "qs_pager_wait_landed": (_I, [_P, _I]),
}

_lib: ctypes.CDLL | None = None
_lock = threading.Lock()


def library_path() -> Path:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and type the native library.  Raises RuntimeError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"QStore HIP library not built ({LIB_PATH}); run __graft_entry__.build()"
            )
        lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError as exc:
        raise ValueError(f"unsupported dtype {dtype}") from exc


def check(status: int, what: str) -> None:
    if status == QS_OK:
        return
    msg = load().qs_last_error().decode(errors="replace")
    text = f"{what}: {msg}"
    if status in (QS_ERR_INVALID, QS_ERR_LIMIT):
        raise ValueError(text)
    raise RuntimeError(text)


def call(name: str, *args) -> None:
    """Invoke an entry point and map its status onto Python exceptions."""
    check(getattr(load(), name)(*args), name)


def stream_of(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device`` (as an int)."""
    return int(torch.cuda.current_stream(device).cuda_stream)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else int(t.data_ptr())


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one HIP device; returns it."""
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError("QStore HIP operators require tensors on a HIP (cuda) device")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError("QStore HIP operator tensors must share one device")
    if device is None:
        raise ValueError("no device tensor given")
    return device


def pointer_array(values: list[int]) -> ctypes.Array:
    arr = (ctypes.c_void_p * len(values))()
    for i, v in enumerate(values):
        arr[i] = v
    return arr


def int64_array(values: list[int]) -> ctypes.Array:
    arr = (ctypes.c_int64 * len(values))()
    for i, v in enumerate(values):
        arr[i] = int(v)
    return arr
