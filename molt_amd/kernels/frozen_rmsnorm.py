"""Frozen RMSNorm with a bf16 output: the drop-in for
``molt_stream.kernels.frozen_rmsnorm`` (kernels/frozen_rmsnorm.py:9-97), on the
HIP RMSNorm kernels.

The row's mean square is reduced in fp32, the output is rounded to bf16 once,
and the input gradient (frozen weight) is returned in the input's dtype, as the
reference does. Unlike the reference there is no CPU path: CPU tensors raise
CapabilityError."""
from __future__ import annotations

from typing import Any

import torch
from torch import nn

from .. import ops
from ..errors import CapabilityError

# Weight offset per decoder family (kernels/execution_plan.py:33-64): Gemma
# stores the norm weight as (scale - 1).
_FAMILY_OFFSETS: tuple[tuple[str, tuple[str, ...], float], ...] = (
    ("qwen", ("qwen2", "qwen2_moe", "qwen3", "qwen3_moe"), 0.0),
    ("llama", ("llama", "mistral", "mixtral"), 0.0),
    ("gemma", ("gemma", "gemma2", "gemma3_text"), 1.0),
)


def rmsnorm_weight_offset(model_or_config: object) -> tuple[str, float]:
    """(family, weight offset) of a supported decoder, else CapabilityError
    (kernels/execution_plan.py:66-80)."""
    config = getattr(model_or_config, "config", model_or_config)
    model_type = str(getattr(config, "model_type", "")).lower()
    for family, types, offset in _FAMILY_OFFSETS:
        if model_type in types:
            return family, offset
    supported = ", ".join(t for _, types, _ in _FAMILY_OFFSETS for t in types)
    raise CapabilityError(
        f"MOLT-native kernels do not support model_type={model_type or '<missing>'}; "
        f"supported model types: {supported}")


class _FrozenRMSNormFunction(torch.autograd.Function):
    """kernels/frozen_rmsnorm.py:9-37."""

    @staticmethod
    def forward(ctx: Any, hidden: torch.Tensor, weight: torch.Tensor, eps: float,
                weight_offset: float) -> torch.Tensor:
        if weight.requires_grad:
            raise ValueError("frozen RMSNorm requires a frozen weight")
        if hidden.device.type != "cuda":
            raise CapabilityError("frozen RMSNorm requires CUDA tensors on a ROCm GPU")
        ctx.save_for_backward(hidden, weight)
        ctx.eps = float(eps)
        ctx.weight_offset = float(weight_offset)
        return ops.direct.rmsnorm_forward(hidden, weight, float(eps), float(weight_offset))

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_output: torch.Tensor):
        hidden, weight = ctx.saved_tensors
        grad_hidden = ops.direct.rmsnorm_backward(grad_output, hidden, weight, ctx.eps, ctx.weight_offset)
        return grad_hidden, None, None, None


_EPS_FIELDS = ("variance_epsilon", "eps")


def _norm_epsilon(norm: nn.Module) -> float | None:
    for field in _EPS_FIELDS:
        value = getattr(norm, field, None)
        if value is not None:
            return float(value)
    return None


class FrozenRMSNormBF16(nn.Module):
    """A decoder RMSNorm with a frozen weight, run by the HIP kernels: fp32
    mean square, one bf16 rounding of the output, input gradient in the input's
    dtype (kernels/frozen_rmsnorm.py:40-58). Built from the module it replaces,
    sharing that module's weight parameter."""

    def __init__(self, original: nn.Module, *, weight_offset: float = 0.0) -> None:
        super().__init__()
        weight, eps = getattr(original, "weight", None), _norm_epsilon(original)
        frozen = isinstance(weight, nn.Parameter) and not weight.requires_grad
        if not frozen or eps is None:
            raise CapabilityError("RMSNorm replacement requires a frozen weight and epsilon")
        self.weight = weight
        self.variance_epsilon = eps
        self.weight_offset = float(weight_offset)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return _FrozenRMSNormFunction.apply(hidden_states, self.weight, self.variance_epsilon, self.weight_offset)


def enable_frozen_rmsnorm_bf16(model: nn.Module) -> int:
    """Replace every submodule whose class name contains "rmsnorm" by a
    :class:`FrozenRMSNormBF16` with the decoder family's weight offset
    (kernels/frozen_rmsnorm.py:61-86). Returns the number replaced."""
    family, offset = rmsnorm_weight_offset(model)
    norms = [name for name, module in model.named_modules()
             if name and "rmsnorm" in type(module).__name__.lower()]
    if not norms:
        raise CapabilityError(f"{family} RMSNorm modules were not found")
    for name in norms:
        parent_name, _, attr = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, attr, FrozenRMSNormBF16(getattr(parent, attr), weight_offset=offset))
    return len(norms)


def enable_qwen2_frozen_rmsnorm_bf16(model: nn.Module) -> int:
    """The Qwen2-only entry point (kernels/frozen_rmsnorm.py:89-97)."""
    if getattr(getattr(model, "config", None), "model_type", None) != "qwen2":
        raise CapabilityError("Qwen2 RMSNorm replacement requires model_type=qwen2")
    return enable_frozen_rmsnorm_bf16(model)
