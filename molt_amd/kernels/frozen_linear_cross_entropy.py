"""Exact cross-entropy of a frozen linear head (the LM head), tiled over token
chunks: the drop-in for ``molt_stream.kernels.frozen_linear_cross_entropy``
(kernels/frozen_linear_cross_entropy.py:142-392).

Per chunk of tokens: ``logits = hidden_chunk . W^T`` (hipBLASLt through
``F.linear``, in the head's dtype), then one HIP kernel per chunk
(``molt_cross_entropy_rows``) reduces every row with an online log-sum-exp
in fp32, writes the row's loss, and overwrites the logits in place with
``(softmax - onehot(target)) / tokens``; ``grad_chunk . W`` (hipBLASLt) is the
hidden gradient of the chunk. Complete ``[tokens, vocabulary]`` logits never
exist, and the frozen head's gradient is computed in the forward and returned
by the backward scaled by the incoming gradient, as the reference does.

The fused path needs CUDA tensors; unlike the reference there is no CPU or
eager fallback inside this op.
"""
from __future__ import annotations

from typing import Any

import torch
from torch.nn import functional as F

from .. import ops
from ..errors import CapabilityError


def _validate_inputs(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor, chunk_size: int) -> None:
    """kernels/frozen_linear_cross_entropy.py:278-300 (same checks and messages)."""
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
    if weight.requires_grad:
        raise ValueError(
            "frozen_linear_cross_entropy requires a frozen classifier (weight.requires_grad=False)")


def fused_frozen_loss_supported(hidden: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether this invocation can use the fused GPU path
    (kernels/frozen_linear_cross_entropy.py:303-314): CUDA tensors, bf16/fp32
    hidden and head of one dtype, or fp32 hidden with a bf16 head."""
    return bool(
        hidden.device.type == "cuda" and weight.device == hidden.device
        and hidden.dtype in (torch.bfloat16, torch.float32) and weight.dtype in (torch.bfloat16, torch.float32)
        and (weight.dtype == hidden.dtype or (hidden.dtype == torch.float32 and weight.dtype == torch.bfloat16)))


# The reference's name for the same predicate (its fused path is Triton).
triton_frozen_loss_supported = fused_frozen_loss_supported


def _chunks(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor, chunk_size: int, with_grad: bool):
    flat = hidden.flatten(0, -2)
    labels = targets.reshape(-1).contiguous()
    count = labels.numel()
    losses = torch.empty(count, device=hidden.device, dtype=torch.float32)
    gradient = torch.empty_like(flat) if with_grad else None
    for start in range(0, count, chunk_size):
        end = min(start + chunk_size, count)
        part = flat[start:end]
        logits = F.linear(part if part.dtype == weight.dtype else part.to(weight.dtype), weight)
        losses[start:end] = ops.direct.cross_entropy_rows(logits, labels[start:end], float(count), with_grad)
        if with_grad:
            gradient[start:end].copy_(logits @ weight)   # logits now hold dL/dlogits
        del logits
    return losses.sum(), (gradient.reshape_as(hidden) if with_grad else None)


def _fused_frozen_head_forward(hidden, weight, targets, chunk_size) -> tuple[torch.Tensor, torch.Tensor]:
    if not fused_frozen_loss_supported(hidden, weight):
        raise CapabilityError("the fused frozen-head loss needs CUDA bf16/fp32 tensors (fp32 hidden may use a bf16 head)")
    return _chunks(hidden, weight, targets, chunk_size, True)


def frozen_linear_cross_entropy_loss_only(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                                          chunk_size: int = 256) -> torch.Tensor:
    """The training loss without its gradient pass; bitwise the loss that
    :func:`frozen_linear_cross_entropy` returns (kernels/frozen_linear_cross_entropy.py:212-251)."""
    _validate_inputs(hidden, weight, targets, chunk_size)
    if not fused_frozen_loss_supported(hidden, weight):
        raise RuntimeError("the fused frozen-loss backend is unavailable for these tensors")
    return _chunks(hidden, weight, targets, chunk_size, False)[0]


@ops._custom_op(f"{ops.NS}::frozen_linear_cross_entropy")
def frozen_linear_cross_entropy(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                                chunk_size: int = 256) -> torch.Tensor:
    """Exact mean cross-entropy and its hidden gradient for a frozen linear
    head, tiled over token chunks (kernels/frozen_linear_cross_entropy.py:335-392)."""
    _validate_inputs(hidden, weight, targets, chunk_size)
    loss, grad = _fused_frozen_head_forward(hidden, weight, targets, chunk_size)
    loss._molt_saved_grad = grad  # type: ignore[attr-defined]
    return loss


@frozen_linear_cross_entropy.register_fake
def _(hidden, weight, targets, chunk_size=256):
    _validate_inputs(hidden, weight, targets, chunk_size)
    return torch.empty((), device=hidden.device, dtype=torch.float32)


def _setup_context(ctx: Any, inputs: tuple[Any, ...], output: torch.Tensor) -> None:
    hidden, weight, targets, chunk_size = inputs
    saved = getattr(output, "_molt_saved_grad", None)
    if saved is not None:
        ctx.save_for_backward(saved)
    else:
        ctx.save_for_backward(hidden, weight, targets)
    ctx.chunk_size = chunk_size


def _backward(ctx: Any, grad_output: torch.Tensor):
    tensors = ctx.saved_tensors
    if len(tensors) == 1:
        return tensors[0] * grad_output, None, None, None
    hidden, weight, targets = tensors
    _, grad = _fused_frozen_head_forward(hidden, weight, targets, ctx.chunk_size)
    return grad * grad_output, None, None, None


frozen_linear_cross_entropy.register_autograd(_backward, setup_context=_setup_context)
