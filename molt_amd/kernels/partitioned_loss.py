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

from contextlib import nullcontext
from typing import Any

import torch
from torch.nn import functional as F

from ..errors import CapabilityError
from .frozen_linear_cross_entropy import (_validate_inputs, frozen_linear_cross_entropy,
                                          frozen_linear_cross_entropy_loss_only, fused_frozen_loss_supported)


def _autocast(device_type: str, enabled: bool, dtype: torch.dtype):
    return torch.autocast(device_type=device_type, enabled=enabled, dtype=dtype) if device_type == "cuda" \
        else nullcontext()


def _ce_sum(logits: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
    return F.cross_entropy(logits.float() if logits.dtype in (torch.float16, torch.bfloat16) else logits, labels,
                           reduction="sum")


class _ExactPartitionedLinearCrossEntropy(torch.autograd.Function):
    """Chunked linear + CE, recomputing each chunk in the backward
    (kernels/partitioned_loss.py:18-103)."""

    @staticmethod
    def forward(ctx: Any, hidden, weight, targets, chunk_size):
        flat, labels = hidden.flatten(0, -2), targets.reshape(-1)
        count = labels.numel()
        total = torch.zeros((), device=hidden.device, dtype=torch.float32)
        enabled = torch.is_autocast_enabled("cuda")
        dtype = torch.get_autocast_dtype("cuda")
        with _autocast(hidden.device.type, enabled, dtype):
            for start in range(0, count, chunk_size):
                end = min(start + chunk_size, count)
                total = total + _ce_sum(F.linear(flat[start:end], weight), labels[start:end])
        ctx.save_for_backward(hidden, weight, targets)
        ctx.chunk_size, ctx.enabled, ctx.dtype = chunk_size, enabled, dtype
        return total / count

    @staticmethod
    def backward(ctx: Any, grad_output):
        hidden, weight, targets = ctx.saved_tensors
        flat, labels = hidden.flatten(0, -2), targets.reshape(-1)
        count = labels.numel()
        dh = torch.zeros_like(flat) if ctx.needs_input_grad[0] else None
        dw = torch.zeros_like(weight) if ctx.needs_input_grad[1] else None
        for start in range(0, count, ctx.chunk_size):
            end = min(start + ctx.chunk_size, count)
            with torch.enable_grad():
                hc = flat[start:end].detach().requires_grad_(ctx.needs_input_grad[0])
                wc = weight.detach().requires_grad_(ctx.needs_input_grad[1])
                with _autocast(hidden.device.type, ctx.enabled, ctx.dtype):
                    loss = _ce_sum(F.linear(hc, wc), labels[start:end])
                inputs = [t for t, need in ((hc, ctx.needs_input_grad[0]), (wc, ctx.needs_input_grad[1])) if need]
                grads = torch.autograd.grad(loss, inputs, grad_outputs=grad_output / count)
            i = 0
            if dh is not None:
                dh[start:end].copy_(grads[0])
                i = 1
            if dw is not None:
                dw.add_(grads[i])
        return (dh.reshape_as(hidden) if dh is not None else None), dw, None, None


class _FrozenHeadCrossEntropy(torch.autograd.Function):
    """One head projection per chunk, dL/dlogits formed with torch operations,
    only the hidden gradient kept (kernels/partitioned_loss.py:106-157)."""

    @staticmethod
    def forward(ctx: Any, hidden, weight, targets, chunk_size):
        flat, labels = hidden.flatten(0, -2), targets.reshape(-1)
        count = labels.numel()
        enabled = torch.is_autocast_enabled("cuda")
        dtype = torch.get_autocast_dtype("cuda")
        gradient = torch.empty_like(flat)
        total = torch.zeros((), device=hidden.device, dtype=torch.float32)
        rows = torch.arange(min(chunk_size, count), device=hidden.device)
        for start in range(0, count, chunk_size):
            end = min(start + chunk_size, count)
            with _autocast(hidden.device.type, enabled, dtype):
                logits = F.linear(flat[start:end].detach(), weight)
            red = logits.float() if logits.dtype in (torch.float16, torch.bfloat16) else logits
            total.add_(F.cross_entropy(red, labels[start:end], reduction="sum").detach() / count)
            prob = red.softmax(dim=-1)
            prob[rows[: end - start], labels[start:end]] -= 1.0
            prob /= count
            with _autocast(hidden.device.type, enabled, dtype):
                local = prob.to(weight.dtype) @ weight
            gradient[start:end].copy_(local.to(gradient.dtype))
        ctx.save_for_backward(gradient.reshape_as(hidden))
        return total

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_output):
        (gradient,) = ctx.saved_tensors
        return gradient * grad_output, None, None, None


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
    if precompute_frozen_gradient:
        if weight.requires_grad:
            raise ValueError("Gradient precomputation requires a frozen classifier")
        fused = fused_frozen_loss_supported(hidden, weight)
        if backend == "triton" and not fused:
            raise RuntimeError("the fused frozen-loss backend is unavailable for these tensors")
        if not torch.is_grad_enabled() or not hidden.requires_grad:
            if backend in {"auto", "triton"} and fused:
                return frozen_linear_cross_entropy_loss_only(hidden, weight, targets, chunk_size)
            return _ExactPartitionedLinearCrossEntropy.apply(hidden, weight, targets, chunk_size)
        if backend in {"auto", "triton"} and fused:
            return frozen_linear_cross_entropy(hidden, weight, targets, chunk_size)
        if backend == "analytical":
            _validate_inputs(hidden, weight, targets, chunk_size)
            return _FrozenHeadCrossEntropy.apply(hidden, weight, targets, chunk_size)
    return _ExactPartitionedLinearCrossEntropy.apply(hidden, weight, targets, chunk_size)
