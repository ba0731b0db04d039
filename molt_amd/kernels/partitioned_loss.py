"""Exact linear + cross-entropy with logits bounded to one token chunk: the
drop-in for ``molt_stream.kernels.partitioned_loss``
(kernels/partitioned_loss.py:18-220).

Backends, as the reference names them: "triton" is its fused path, here the
HIP reduction of :mod:`.frozen_linear_cross_entropy`; "analytical" forms
``dL/dlogits`` with torch operations per chunk; "auto" takes the fused path
when it supports the tensors. Without a precomputed frozen gradient the loss
is recomputed chunk by chunk in the backward (the head may then be trainable).
Every backend requires CUDA tensors.
"""
from __future__ import annotations

from typing import Any

import torch
from torch.nn import functional as F

from .. import ops
from ..errors import CapabilityError
from .frozen_linear_cross_entropy import (_validate_inputs, frozen_linear_cross_entropy,
                                          frozen_linear_cross_entropy_loss_only, fused_frozen_loss_supported)


def _compute_dtype(hidden: torch.Tensor, weight: torch.Tensor, autocast: torch.dtype | None) -> torch.dtype:
    """dtype of ``F.linear(hidden, weight)``: the autocast dtype when CUDA
    autocast was on at the forward, else the operands' promoted dtype."""
    return autocast if autocast is not None else torch.promote_types(hidden.dtype, weight.dtype)


def _logits(rows: torch.Tensor, weight: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """One chunk's logits in ``dtype`` (what the row kernel reads: bf16 or
    fp32; other dtypes are widened to fp32 first)."""
    z = F.linear(rows.to(dtype), weight.to(dtype))
    return z if z.dtype in (torch.bfloat16, torch.float32) else z.float()


def _spans(count: int, chunk: int):
    return ((start, min(start + chunk, count)) for start in range(0, count, chunk))


IGNORE_INDEX = -100   # F.cross_entropy's default ignore_index, which the reference's exact path uses


def _check_targets(labels: torch.Tensor, vocab: int) -> None:
    """F.cross_entropy's target rule: a target is a class in [0, vocab) or the
    ignored index; anything else is an error (one device reduction and one
    host read per forward)."""
    bad = ((labels < 0) | (labels >= vocab)) & (labels != IGNORE_INDEX)
    if bool(bad.any()):
        first = int(labels[bad][0])
        raise IndexError(f"Target {first} is out of bounds for {vocab} classes (ignore_index is {IGNORE_INDEX})")


class _ChunkedLinearCrossEntropy(torch.autograd.Function):
    """Exact mean cross-entropy of ``hidden . weight^T`` with at most one
    chunk of logits alive (kernels/partitioned_loss.py:18-103).

    Forward: per chunk, hipBLASLt logits and the HIP row kernel's per-row
    ``(lse - l_y) / count`` (no gradient pass). Backward: per chunk, the
    logits again, the row kernel in gradient mode (logits overwritten in place
    by ``(softmax - onehot) / count * g``, one rounding to the logits' dtype,
    with the upstream gradient ``g`` read on the device), then
    ``dh = dlogits . W`` and, for a trainable head, ``dW += dlogits^T . h``.
    Targets follow F.cross_entropy: rows with the ignored index -100 add
    nothing to the loss and get a zero gradient (the mean still divides by
    every token, as the reference's sum over chunks / token count does); any
    other target outside the vocabulary raises. The head's dtype decides the
    GEMM precision, as autocast does."""

    @staticmethod
    def forward(ctx: Any, hidden, weight, targets, chunk_size):
        rows, labels = hidden.flatten(0, -2), targets.reshape(-1).contiguous()
        count = labels.numel()
        _check_targets(labels, weight.shape[0])
        autocast = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else None
        dtype = _compute_dtype(hidden, weight, autocast)
        per_row = torch.empty(count, device=hidden.device, dtype=torch.float32)
        for lo, hi in _spans(count, chunk_size):
            per_row[lo:hi] = ops.direct.cross_entropy_rows_exact(_logits(rows[lo:hi], weight, dtype), labels[lo:hi],
                                                                 float(count), None, False)
        ctx.save_for_backward(hidden, weight, targets)
        ctx.chunk_size, ctx.dtype = chunk_size, dtype
        return per_row.sum()

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_output):
        hidden, weight, targets = ctx.saved_tensors
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        rows, labels = hidden.flatten(0, -2), targets.reshape(-1).contiguous()
        count = labels.numel()
        scale = grad_output.detach().to(torch.float32).reshape(1)
        grad_rows = torch.empty_like(rows) if need_h else None
        grad_w = torch.zeros(weight.shape, device=weight.device, dtype=torch.float32) if need_w else None
        w = weight.detach().to(ctx.dtype)
        for lo, hi in _spans(count, ctx.chunk_size):
            part = rows[lo:hi].detach().to(ctx.dtype)
            dlogits = _logits(part, w, ctx.dtype)
            ops.direct.cross_entropy_rows_exact(dlogits, labels[lo:hi], float(count), scale, True)
            dlogits = dlogits.to(ctx.dtype)
            if need_h:
                grad_rows[lo:hi].copy_(dlogits @ w)
            if need_w:
                grad_w.add_((dlogits.t() @ part).float())
        grad_h = grad_rows.reshape_as(hidden) if need_h else None
        return grad_h, (grad_w.to(weight.dtype) if need_w else None), None, None


class _AnalyticalHeadCrossEntropy(torch.autograd.Function):
    """The "analytical" backend: per chunk, ``dL/dlogits`` from torch's
    log-softmax (``exp(log_softmax) - onehot``, over ``count``) and the hidden
    gradient ``dlogits . W`` kept from the forward; the head is frozen
    (kernels/partitioned_loss.py:106-157)."""

    @staticmethod
    def forward(ctx: Any, hidden, weight, targets, chunk_size):
        rows, labels = hidden.flatten(0, -2), targets.reshape(-1)
        count = labels.numel()
        autocast = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else None
        dtype = _compute_dtype(hidden, weight, autocast)
        total = torch.zeros((), device=hidden.device, dtype=torch.float32)
        grad = torch.empty_like(rows)
        w = weight.detach().to(dtype)
        for lo, hi in _spans(count, chunk_size):
            logp = torch.log_softmax(F.linear(rows[lo:hi].detach().to(dtype), w).float(), dim=-1)
            picked = logp.gather(1, labels[lo:hi, None])
            total -= picked.sum() / count
            dlogits = logp.exp_().scatter_add_(1, labels[lo:hi, None], torch.full_like(picked, -1.0)).div_(count)
            grad[lo:hi].copy_(dlogits.to(dtype) @ w)
        ctx.save_for_backward(grad.reshape_as(hidden))
        return total

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_output):
        (grad,) = ctx.saved_tensors
        return grad * grad_output, None, None, None


def exact_partitioned_linear_cross_entropy(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                                           chunk_size: int, *, precompute_frozen_gradient: bool = False,
                                           backend: str = "auto") -> torch.Tensor:
    """Exact mean CE with materialised logits bounded to one chunk
    (kernels/partitioned_loss.py:160-220)."""
    if backend not in {"auto", "triton", "analytical"}:
        raise ValueError(f"Unknown backend: {backend}")
    if hidden.ndim < 2 or weight.ndim != 2:
        raise ValueError("hidden must be [..., width] and weight must be [vocab, width]")
    if hidden.shape[:-1] != targets.shape:
        raise ValueError("targets must match every non-feature hidden dimension")
    if hidden.shape[-1] != weight.shape[-1]:
        raise ValueError("hidden width and classifier weight width must match")
    if targets.dtype != torch.long:
        raise ValueError("targets must use torch.long indices")
    if chunk_size <= 0:
        raise ValueError("chunk_size must be positive")
    if targets.numel() == 0:
        raise ValueError("targets must not be empty")
    if hidden.device.type != "cuda":
        raise CapabilityError("exact partitioned linear cross-entropy is unavailable for CPU tensors "
                              "(it requires CUDA tensors on a ROCm GPU)")
    if torch.float64 in (hidden.dtype, weight.dtype):
        raise CapabilityError("exact partitioned linear cross-entropy reduces rows in fp32; float64 is unsupported")
    if precompute_frozen_gradient:
        if weight.requires_grad:
            raise ValueError("Gradient precomputation requires a frozen classifier")
        fused = fused_frozen_loss_supported(hidden, weight)
        if backend == "triton" and not fused:
            raise RuntimeError("the fused frozen-loss backend is unavailable for these tensors")
        if not torch.is_grad_enabled() or not hidden.requires_grad:
            if backend in {"auto", "triton"} and fused:
                return frozen_linear_cross_entropy_loss_only(hidden, weight, targets, chunk_size)
            return _ChunkedLinearCrossEntropy.apply(hidden, weight, targets, chunk_size)
        if backend in {"auto", "triton"} and fused:
            return frozen_linear_cross_entropy(hidden, weight, targets, chunk_size)
        if backend == "analytical":
            _validate_inputs(hidden, weight, targets, chunk_size)
            return _AnalyticalHeadCrossEntropy.apply(hidden, weight, targets, chunk_size)
    return _ChunkedLinearCrossEntropy.apply(hidden, weight, targets, chunk_size)
