"""Expert-major packet queues for routed MoE on gfx950 -- drop-in for
src/mrun/engine/kernels/expert_queue.py.

A queue plan turns router output (``[rows, top_k]`` expert ids and weights, or a pruned
flat packet list) into contiguous per-expert packet ranges; every packet carries its row
(``token_ids``), route slot, fp32 coefficient and its row's slot epoch and deadline.
``scatter_committed`` later reduces packet outputs back into rows, counting only packets
whose epoch still matches the row's active epoch.

Both directions run in ``csrc/qs_queue.hip`` (``qs_expert_queue_build``,
``qs_expert_queue_scatter``).  The build is stable (packets of one expert keep their input
order), so the CPU-validated builders and the ``_device`` builder give the same plan, and
the scatter is a fixed-order reduce (no atomics), so ``scatter_committed`` and
``scatter_committed_device`` give the same bits on every call.  The validating builders
check their inputs on the host first, with the reference's error messages; the ``_device``
builder trusts its input as the reference's does.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native as nat

_INTEGRAL = (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8)
_WEIGHT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


@dataclass(frozen=True)
class ExpertQueuePlan:
    """Packet queue of one routed layer (fields as expert_queue.py:25-37)."""

    num_rows: int
    num_experts: int
    top_k: int
    token_ids: torch.Tensor
    expert_ids: torch.Tensor
    route_slots: torch.Tensor
    coefficients: torch.Tensor
    epochs: torch.Tensor
    deadlines: torch.Tensor
    starts: torch.Tensor
    counts: torch.Tensor

    @property
    def assignments(self) -> int:
        return int(self.token_ids.numel())

    def assert_valid(self) -> None:
        """Structural invariants of a plan (expert_queue.py:43-90); AssertionError on the
        first one that fails.  Reads tensors back to the host."""

        def need(ok: bool, msg: str) -> None:
            if not ok:
                raise AssertionError(msg)

        need(self.num_rows > 0, "num_rows must be positive")
        need(self.num_experts > 0, "num_experts must be positive")
        need(self.top_k > 0, "top_k must be positive")
        a = self.assignments
        cap = self.num_rows * self.top_k
        need(a <= cap, f"assignment conservation failed: {a} > {cap}")
        for label, t in (("expert_ids", self.expert_ids), ("route_slots", self.route_slots),
                         ("coefficients", self.coefficients), ("epochs", self.epochs),
                         ("deadlines", self.deadlines)):
            need(tuple(t.shape) == (a,), f"{label} have the wrong packet shape")
        need(int(self.counts.sum()) == a, "expert counts do not conserve assignments")
        need(tuple(self.starts.shape) == (self.num_experts,), "starts have the wrong expert shape")
        need(tuple(self.counts.shape) == (self.num_experts,), "counts have the wrong expert shape")
        need(int(self.starts[0]) == 0, "the first expert queue must begin at zero")
        if self.num_experts > 1:
            need(torch.equal(self.starts[1:], self.starts[:-1] + self.counts[:-1]),
                 "expert queue ranges are not contiguous")
        if a:
            def within(t: torch.Tensor, hi: int) -> bool:
                return bool(((t >= 0) & (t < hi)).all())

            need(within(self.token_ids, self.num_rows), "token_ids contain an out-of-range row")
            need(within(self.expert_ids, self.num_experts), "expert_ids contain an out-of-range expert")
            need(within(self.route_slots, self.top_k), "route_slots contain an out-of-range slot")
            need(bool(torch.isfinite(self.coefficients).all()), "coefficients must be finite")
            need(bool((self.expert_ids[1:] >= self.expert_ids[:-1]).all()), "packets are not grouped by expert")


def _integral(label: str, t: torch.Tensor) -> None:
    if t.dtype not in _INTEGRAL:
        raise ValueError(f"{label} must contain integer values")


def _route_inputs(top_indices, top_weights, num_experts, epochs, deadlines) -> tuple[int, int]:
    """Argument checks shared by the dense builders (expert_queue.py:200-227)."""
    if top_indices.ndim != 2 or 0 in top_indices.shape:
        raise ValueError("top_indices must have non-empty shape [rows, top_k]")
    if top_weights.shape != top_indices.shape:
        raise ValueError("top_weights must match top_indices")
    if num_experts <= 0:
        raise ValueError("num_experts must be positive")
    _integral("top_indices", top_indices)
    if not torch.is_floating_point(top_weights):
        raise ValueError("top_weights must be floating point")
    rows, top_k = map(int, top_indices.shape)
    if tuple(epochs.shape) != (rows,):
        raise ValueError("epochs must have shape [rows]")
    if tuple(deadlines.shape) != (rows,):
        raise ValueError("deadlines must have shape [rows]")
    _integral("epochs", epochs)
    _integral("deadlines", deadlines)
    if top_indices.device != top_weights.device:
        raise ValueError("top_indices and top_weights must be on the same device")
    if epochs.device != top_indices.device or deadlines.device != top_indices.device:
        raise ValueError("epochs and deadlines must be on the route tensor device")
    return rows, top_k


def _weights_arg(w: torch.Tensor) -> torch.Tensor:
    w = w.reshape(-1)
    if w.dtype not in _WEIGHT_DTYPES:
        w = w.to(torch.float32)
    return w.contiguous()


def _experts_arg(e: torch.Tensor) -> torch.Tensor:
    e = e.reshape(-1)
    if e.dtype not in (torch.int32, torch.int64):
        e = e.to(torch.int64)
    return e.contiguous()


def _compile(rows: int, top_k: int, num_experts: int, experts: torch.Tensor, weights: torch.Tensor,
             epochs: torch.Tensor, deadlines: torch.Tensor, tokens: torch.Tensor | None,
             slots: torch.Tensor | None, count_dtype: torch.dtype) -> ExpertQueuePlan:
    device = nat.require_device(experts, weights, epochs, deadlines, tokens, slots)
    A = int(experts.numel())
    i64 = dict(dtype=torch.int64, device=device)
    token_ids = torch.empty(A, **i64)
    expert_ids = torch.empty(A, **i64)
    route_slots = torch.empty(A, **i64)
    coefficients = torch.empty(A, dtype=torch.float32, device=device)
    p_epochs = torch.empty(A, **i64)
    p_deadlines = torch.empty(A, **i64)
    starts = torch.empty(num_experts, dtype=count_dtype, device=device)
    counts = torch.empty(num_experts, dtype=count_dtype, device=device)
    ep = epochs.to(torch.int64).contiguous()
    dl = deadlines.to(torch.int64).contiguous()
    nat.call(
        "qs_expert_queue_build", nat.ptr(experts), nat.dtype_code(experts.dtype), nat.ptr(tokens), nat.ptr(slots),
        nat.ptr(weights), nat.dtype_code(weights.dtype), nat.ptr(ep), nat.ptr(dl), A, top_k, rows, num_experts,
        nat.ptr(token_ids), nat.ptr(expert_ids), nat.ptr(route_slots), nat.ptr(coefficients), nat.ptr(p_epochs),
        nat.ptr(p_deadlines), nat.ptr(starts), nat.ptr(counts), nat.dtype_code(count_dtype), nat.stream_of(device),
    )
    return ExpertQueuePlan(rows, num_experts, top_k, token_ids, expert_ids, route_slots, coefficients, p_epochs,
                           p_deadlines, starts, counts)


@torch.inference_mode()
def build_expert_queue(top_indices: torch.Tensor, top_weights: torch.Tensor, *, num_experts: int,
                       epochs: torch.Tensor, deadlines: torch.Tensor) -> ExpertQueuePlan:
    """Validated, stable expert-major plan of ``[rows, top_k]`` router output
    (expert_queue.py:242-294); int64 starts/counts."""
    rows, top_k = _route_inputs(top_indices, top_weights, num_experts, epochs, deadlines)
    if not bool(torch.isfinite(top_weights).all()):
        raise ValueError("top_weights must be finite")
    idx = top_indices.to(torch.int64)
    if not bool(((idx >= 0) & (idx < num_experts)).all()):
        raise ValueError("top_indices contains an out-of-range expert")
    srt = idx.sort(dim=1).values
    if bool((srt[:, 1:] == srt[:, :-1]).any()):
        raise ValueError("a routed row cannot select the same expert twice")
    plan = _compile(rows, top_k, num_experts, _experts_arg(top_indices), _weights_arg(top_weights), epochs,
                    deadlines, None, None, torch.int64)
    plan.assert_valid()
    return plan


@torch.inference_mode()
def build_expert_queue_flat(token_ids: torch.Tensor, expert_ids: torch.Tensor, route_slots: torch.Tensor,
                            coefficients: torch.Tensor, *, num_rows: int, num_experts: int, top_k: int,
                            epochs: torch.Tensor, deadlines: torch.Tensor,
                            validate: bool = True) -> ExpertQueuePlan:
    """Stable expert-major plan of a pruned packet list (expert_queue.py:297-398): rows may
    carry fewer than ``top_k`` packets; int32 starts/counts (the reference's device dtype)."""
    if num_rows <= 0:
        raise ValueError("num_rows must be positive")
    if num_experts <= 0:
        raise ValueError("num_experts must be positive")
    if top_k <= 0:
        raise ValueError("top_k must be positive")
    shape = tuple(token_ids.shape)
    if len(shape) != 1:
        raise ValueError("token_ids must have shape [assignments]")
    for label, t in (("expert_ids", expert_ids), ("route_slots", route_slots), ("coefficients", coefficients)):
        if tuple(t.shape) != shape:
            raise ValueError(f"{label} must match token_ids")
    if tuple(epochs.shape) != (num_rows,):
        raise ValueError("epochs must have shape [rows]")
    if tuple(deadlines.shape) != (num_rows,):
        raise ValueError("deadlines must have shape [rows]")
    for label, t in (("token_ids", token_ids), ("expert_ids", expert_ids), ("route_slots", route_slots),
                     ("epochs", epochs), ("deadlines", deadlines)):
        _integral(label, t)
    if not torch.is_floating_point(coefficients):
        raise ValueError("coefficients must be floating point")
    if any(t.device != token_ids.device for t in (expert_ids, route_slots, coefficients, epochs, deadlines)):
        raise ValueError("all sparse queue tensors must be on the same device")
    A = shape[0]
    if A > num_rows * top_k:
        raise ValueError("sparse queue contains more assignments than dense top-k")
    tok = token_ids.to(torch.int64).contiguous()
    exp = expert_ids.to(torch.int64).contiguous()
    slot = route_slots.to(torch.int64).contiguous()
    if validate and A:
        if not bool(((tok >= 0) & (tok < num_rows)).all()):
            raise ValueError("token_ids contains an out-of-range row")
        if not bool(((exp >= 0) & (exp < num_experts)).all()):
            raise ValueError("expert_ids contains an out-of-range expert")
        if not bool(((slot >= 0) & (slot < top_k)).all()):
            raise ValueError("route_slots contains an out-of-range slot")
        if not bool(torch.isfinite(coefficients).all()):
            raise ValueError("coefficients must be finite")
        if int(torch.unique(tok * top_k + slot).numel()) != A:
            raise ValueError("a routed row cannot use the same route slot twice")
        if int(torch.unique(tok * num_experts + exp).numel()) != A:
            raise ValueError("a routed row cannot select the same expert twice")
    plan = _compile(num_rows, top_k, num_experts, exp, _weights_arg(coefficients), epochs, deadlines, tok, slot,
                    torch.int32)
    if validate:
        plan.assert_valid()
    return plan


@torch.inference_mode()
def build_expert_queue_device(top_indices: torch.Tensor, top_weights: torch.Tensor, *, num_experts: int,
                              epochs: torch.Tensor, deadlines: torch.Tensor, block: int = 256) -> ExpertQueuePlan:
    """Plan of router output that upstream code already validated (expert_queue.py:401-484):
    no host round trip; int32 starts/counts.  ``block`` is accepted for signature
    compatibility (the kernel's launch shape is its own)."""
    del block
    rows, top_k = _route_inputs(top_indices, top_weights, num_experts, epochs, deadlines)
    if top_indices.device.type != "cuda":
        raise ValueError("build_expert_queue_device requires device (HIP) tensors")
    return _compile(rows, top_k, num_experts, _experts_arg(top_indices), _weights_arg(top_weights), epochs,
                    deadlines, None, None, torch.int32)


def _scatter(plan: ExpertQueuePlan, expert_outputs: torch.Tensor, active_epochs: torch.Tensor):
    if expert_outputs.ndim != 2 or int(expert_outputs.shape[0]) != plan.assignments:
        raise ValueError("expert_outputs must have shape [assignments, hidden]")
    if tuple(active_epochs.shape) != (plan.num_rows,):
        raise ValueError("active_epochs must have shape [rows]")
    if expert_outputs.device != plan.token_ids.device:
        raise ValueError("expert_outputs must be on the queue tensor device")
    if active_epochs.device != plan.token_ids.device:
        raise ValueError("active_epochs must be on the queue tensor device")
    _integral("active_epochs", active_epochs)
    device = nat.require_device(expert_outputs, active_epochs, plan.token_ids)
    y = expert_outputs
    if y.dtype not in _WEIGHT_DTYPES:
        y = y.to(torch.float32)
    if y.stride(1) != 1:
        y = y.contiguous()
    H = int(y.shape[1])
    A = plan.assignments
    reduced = torch.empty((plan.num_rows, H), dtype=torch.float32, device=device)
    valid = torch.empty(A, dtype=torch.uint8, device=device)
    ws_bytes = int(nat.load().qs_expert_queue_scatter_workspace_bytes(plan.num_rows, A))
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=device)
    active = active_epochs.to(torch.int64).contiguous()
    coef = plan.coefficients.to(torch.float32).contiguous()
    nat.call(
        "qs_expert_queue_scatter", nat.ptr(plan.token_ids.to(torch.int64).contiguous()), nat.ptr(coef),
        nat.ptr(plan.epochs.to(torch.int64).contiguous()), nat.ptr(active), nat.ptr(y), nat.dtype_code(y.dtype),
        int(y.stride(0)) if A else H, A, plan.num_rows, H, nat.ptr(ws), ws_bytes, nat.ptr(reduced),
        nat.ptr(valid), nat.stream_of(device),
    )
    return reduced, valid.view(torch.bool)


@torch.inference_mode()
def scatter_committed(plan: ExpertQueuePlan, expert_outputs: torch.Tensor, *,
                      active_epochs: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``(reduced [rows, hidden] fp32, valid [assignments] bool)``: packets whose epoch equals
    their row's active epoch, weighted and summed in queue order (expert_queue.py:487-514)."""
    return _scatter(plan, expert_outputs, active_epochs)


@torch.inference_mode()
def scatter_committed_device(plan: ExpertQueuePlan, expert_outputs: torch.Tensor, *, active_epochs: torch.Tensor,
                             block_assignments: int = 128,
                             block_hidden: int = 32) -> tuple[torch.Tensor, torch.Tensor]:
    """Same result as :func:`scatter_committed` (expert_queue.py:517-560); the tile
    arguments are accepted for signature compatibility."""
    del block_assignments, block_hidden
    return _scatter(plan, expert_outputs, active_epochs)
