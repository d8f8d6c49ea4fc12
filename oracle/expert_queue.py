"""Oracle: expert-major packet queues (numpy, CPU).  Test infrastructure only.

Restates (reference paths relative to /root/reference/src/mrun/engine/kernels/):
* ``build_dense``  -- build_expert_queue, expert_queue.py:242-294: packets in row-major
                      (row, slot) order, stably sorted by expert; bincount/cumsum ranges;
                      each packet carries its row's epoch and deadline
* ``build_flat``   -- build_expert_queue_flat, expert_queue.py:297-398: the same over a given
                      packet list; epochs/deadlines gathered by the sorted tokens
* ``scatter``      -- scatter_committed, expert_queue.py:487-514: valid = epoch matches the
                      row's active epoch; reduced[row] += fp32(float(out) * coef) over the
                      valid packets in queue order, starting from 0 (index_add_ on CPU)

Pinned by (tests/test_oracle_queue.py): the reference's own KATs
(tests/test_expert_queue.py:16-139) and golden vectors written from the reference's CPU
functions (tests/golden/queue.npz), bit for bit.
"""

from __future__ import annotations

import numpy as np


def _ranges(experts_sorted: np.ndarray, num_experts: int):
    counts = np.bincount(experts_sorted, minlength=num_experts).astype(np.int64)
    starts = (np.cumsum(counts) - counts).astype(np.int64)
    return starts, counts


def build_dense(top_indices, top_weights, num_experts: int, epochs, deadlines) -> dict:
    idx = np.asarray(top_indices, dtype=np.int64)
    rows, k = idx.shape
    experts = idx.reshape(-1)
    order = np.argsort(experts, kind="stable")
    tokens = np.repeat(np.arange(rows, dtype=np.int64), k)
    slots = np.tile(np.arange(k, dtype=np.int64), rows)
    ep = np.repeat(np.asarray(epochs, dtype=np.int64), k)
    dl = np.repeat(np.asarray(deadlines, dtype=np.int64), k)
    w = np.asarray(top_weights, dtype=np.float32).reshape(-1)
    starts, counts = _ranges(experts[order], num_experts)
    return dict(token_ids=tokens[order], expert_ids=experts[order], route_slots=slots[order],
                coefficients=w[order], epochs=ep[order], deadlines=dl[order], starts=starts, counts=counts)


def build_flat(token_ids, expert_ids, route_slots, coefficients, num_experts: int, epochs, deadlines) -> dict:
    tok = np.asarray(token_ids, dtype=np.int64)
    exp = np.asarray(expert_ids, dtype=np.int64)
    order = np.argsort(exp, kind="stable")
    starts, counts = _ranges(exp[order], num_experts)
    st = tok[order]
    return dict(token_ids=st, expert_ids=exp[order], route_slots=np.asarray(route_slots, dtype=np.int64)[order],
                coefficients=np.asarray(coefficients, dtype=np.float32)[order],
                epochs=np.asarray(epochs, dtype=np.int64)[st], deadlines=np.asarray(deadlines, dtype=np.int64)[st],
                starts=starts, counts=counts)


def scatter(plan: dict, expert_outputs, active_epochs, num_rows: int):
    y = np.asarray(expert_outputs, dtype=np.float32)
    active = np.asarray(active_epochs, dtype=np.int64)
    valid = plan["epochs"] == active[plan["token_ids"]]
    reduced = np.zeros((num_rows, y.shape[1]), dtype=np.float32)
    for q in np.nonzero(valid)[0]:
        v = (y[q] * plan["coefficients"][q]).astype(np.float32)
        t = plan["token_ids"][q]
        reduced[t] = (reduced[t] + v).astype(np.float32)
    return reduced, valid
