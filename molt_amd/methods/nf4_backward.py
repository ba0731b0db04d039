"""Packed NF4 input gradients without a dense weight: the drop-in for
``molt_stream.methods.nf4_backward`` (methods/nf4_backward.py:145-284).

The Triton kernel of the reference is replaced by the NF4-fused MFMA GEMM of
libmolt_amd.so (column-contract staging: each thread decodes an 8-row x
4-column patch of the packed weight and transposes it in registers into LDS).
Unlike the reference, the fused LoRA term has no rank limit.
"""
from __future__ import annotations

from typing import Any

import torch

from .. import ops
from ..errors import CapabilityError
from ..nf4 import _rows_cols, nibble_order
from ..nf4 import resolved_nf4_scales as _resolved


def resolved_nf4_scales(quant_state: Any) -> torch.Tensor:
    """Resolve double-quantized block scales once without expanding weights
    (methods/nf4_backward.py:145-164)."""
    if getattr(quant_state, "quant_type", None) != "nf4":
        raise CapabilityError("packed backward requires NF4 quantization")
    if int(getattr(quant_state, "blocksize", 0)) != 64:
        raise CapabilityError("packed backward currently requires NF4 block size 64")
    return _resolved(quant_state)


def _prepare(grad_output: torch.Tensor, quant_state: Any, what: str) -> tuple[torch.Tensor, int, int]:
    if grad_output.device.type != "cuda":
        raise CapabilityError(f"{what} requires CUDA tensors on a ROCm GPU")
    if grad_output.dtype != torch.bfloat16:
        raise CapabilityError(f"{what} currently requires BF16 gradients")
    shape = tuple(int(v) for v in quant_state.shape)
    if len(shape) != 2 or grad_output.shape[-1] != shape[0]:
        raise ValueError("gradient width must match the NF4 output dimension")
    n, k = shape
    return grad_output.contiguous().reshape(-1, n), n, k


def packed_nf4_backward_input(
    grad_output: torch.Tensor,
    packed_weight: torch.Tensor,
    quant_state: Any,
    scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """``grad_output @ dequant(weight)`` without dense weight storage
    (methods/nf4_backward.py:167-217)."""
    flat, n, k = _prepare(grad_output, quant_state, "packed NF4 backward")
    resolved = resolved_nf4_scales(quant_state) if scales is None else scales
    out = ops.direct.nf4_lora_backward_input(flat, packed_weight.reshape(-1), resolved, quant_state.code, n, k,
                                      nibble_order(quant_state), int(quant_state.blocksize), None, None, 1.0)
    return out.reshape(*grad_output.shape[:-1], k)


def packed_nf4_lora_backward_input(
    grad_output: torch.Tensor,
    packed_weight: torch.Tensor,
    quant_state: Any,
    lora_grad: torch.Tensor,
    lora_a: torch.Tensor,
    scaling: float,
    scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """``grad_output @ dequant(weight) + scaling * lora_grad @ bf16(lora_a)``
    (methods/nf4_backward.py:220-284); any rank."""
    flat, n, k = _prepare(grad_output, quant_state, "packed NF4-LoRA backward")
    if lora_grad.dtype != torch.bfloat16:
        raise CapabilityError("packed NF4-LoRA backward requires BF16 gradients")
    if lora_a.dtype not in {torch.bfloat16, torch.float32}:
        raise CapabilityError("LoRA A must use BF16 compute or an FP32 master")
    flat_lora = lora_grad.contiguous().reshape(-1, lora_grad.shape[-1])
    if flat_lora.shape[0] != flat.shape[0]:
        raise ValueError("LoRA gradient rows must match the output gradient")
    if lora_a.ndim != 2 or flat_lora.shape[1] != lora_a.shape[0] or lora_a.shape[1] != k:
        raise ValueError("LoRA gradient and A matrix dimensions are incompatible")
    resolved = resolved_nf4_scales(quant_state) if scales is None else scales
    out = ops.direct.nf4_lora_backward_input(flat, packed_weight.reshape(-1), resolved, quant_state.code, n, k,
                                      nibble_order(quant_state), int(quant_state.blocksize), flat_lora,
                                      lora_a, float(scaling))
    return out.reshape(*grad_output.shape[:-1], k)
