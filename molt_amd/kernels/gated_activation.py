"""Fused SiLU-multiply: the drop-in for ``molt_stream.kernels.gated_activation``
(kernels/gated_activation.py:54-130), on the HIP SwiGLU kernels.

Unlike the reference there is no eager CPU fallback: CPU tensors raise
CapabilityError (the shipped path never computes on the host)."""
from __future__ import annotations

from typing import Any

import torch

from .. import ops
from ..errors import CapabilityError
from ..patching import is_swapped, swap_forward


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


_MLP_ORIGINAL = "_molt_original_mlp_forward"
_GATED = ("gate_proj", "up_proj", "down_proj")


def _silu_gated_forward(module: torch.nn.Module, hidden: torch.Tensor) -> torch.Tensor:
    """``down(silu(gate(hidden)) * up(hidden))`` with the HIP SiLU-multiply."""
    gate, up = module.gate_proj(hidden), module.up_proj(hidden)
    return module.down_proj(fused_silu_multiply(gate, up))


def enable_fused_silu_mlp(model: torch.nn.Module) -> int:
    """Swap the forward of every gated MLP (a module with gate/up/down
    projections) of a silu/swish model for :func:`_silu_gated_forward`; state
    keys do not change (kernels/gated_activation.py:106-130). The replaced
    forward is kept as ``_molt_original_mlp_forward``. Returns the count."""
    config = getattr(model, "config", None)
    activation = str(getattr(config, "hidden_activation", None) or getattr(config, "hidden_act", "")).lower()
    family = str(getattr(config, "model_type", "<unknown>"))
    if activation not in {"silu", "swish"}:
        raise CapabilityError(f"fused SiLU MLP requires silu/swish, but {family} uses {activation or '<unknown>'}")
    mlps = [m for m in model.modules()
            if all(hasattr(m, n) for n in _GATED) and not is_swapped(m, _MLP_ORIGINAL)]
    if not mlps:
        raise CapabilityError(f"No compatible {family} gated MLP modules found")
    for mlp in mlps:
        swap_forward(mlp, _silu_gated_forward, key=_MLP_ORIGINAL)
    return len(mlps)
