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
