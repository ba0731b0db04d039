"""Fused SiLU-multiply: the drop-in for ``molt_stream.kernels.gated_activation``
(kernels/gated_activation.py:54-130), on the HIP SwiGLU kernels.

Unlike the reference there is no eager CPU fallback: CPU tensors raise
CapabilityError (the shipped path never computes on the host)."""
from __future__ import annotations

from types import MethodType
from typing import Any

import torch

from .. import ops
from ..errors import CapabilityError


class _FusedSiLUMultiply(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
        if gate.shape != up.shape or gate.dtype != up.dtype or gate.device != up.device:
            raise ValueError("gate and up tensors must have identical shape, dtype, and device")
        if gate.device.type != "cuda":
            raise CapabilityError("fused SiLU multiply requires CUDA tensors on a ROCm GPU")
        g, u = gate.contiguous(), up.contiguous()
        out = ops.direct.silu_mul_forward(g, u, False)
        ctx.original_shape = gate.shape
        ctx.save_for_backward(g, u)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_output: torch.Tensor):
        gate, up = ctx.saved_tensors
        dg, du = ops.direct.silu_mul_backward(grad_output.contiguous().to(gate.dtype), gate, up)
        return dg.reshape(ctx.original_shape), du.reshape(ctx.original_shape)


def fused_silu_multiply(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """kernels/gated_activation.py:96-97."""
    return _FusedSiLUMultiply.apply(gate, up)


def _fused_mlp_forward(module: torch.nn.Module, hidden: torch.Tensor) -> torch.Tensor:
    return module.down_proj(fused_silu_multiply(module.gate_proj(hidden), module.up_proj(hidden)))


def enable_fused_silu_mlp(model: torch.nn.Module) -> int:
    """Patch compatible SiLU-gated decoder MLPs without changing state keys
    (kernels/gated_activation.py:106-130)."""
    config = getattr(model, "config", None)
    activation = str(getattr(config, "hidden_activation", getattr(config, "hidden_act", ""))).lower()
    family = str(getattr(config, "model_type", "<unknown>"))
    if activation not in {"silu", "swish"}:
        raise CapabilityError(
            f"fused SiLU MLP requires silu/swish, but {family} uses {activation or '<unknown>'}"
        )
    patched = 0
    for module in model.modules():
        if hasattr(module, "_molt_original_mlp_forward"):
            continue
        if not all(hasattr(module, name) for name in ("gate_proj", "up_proj", "down_proj")):
            continue
        module._molt_original_mlp_forward = module.forward
        module.forward = MethodType(_fused_mlp_forward, module)
        patched += 1
    if patched == 0:
        raise CapabilityError(f"No compatible {family} gated MLP modules found")
    return patched
