"""Scheduled NF4-LoRA linear on MI355X: the drop-in for
``molt_stream.methods.nf4_lora`` (methods/nf4_lora.py:12-220).

Same public names, signatures, saved-state contract and error behaviour; the
bitsandbytes + cuBLAS calls underneath are replaced by hand-written HIP
kernels (libmolt_amd.so):

* forward: ``T = bf16(X bf16(A)^T)`` (rank-r projection), then one NF4-fused
  MFMA GEMM ``Y = X deq(W)^T + T bf16(s B)^T`` with a single bf16 rounding;
* backward: ``U = bf16(bf16(s dY) bf16(B))`` (scale before the matmul, as
  methods/nf4_lora.py:87-90), ``dX = dY deq(W) + U bf16(A)`` in one NF4-fused
  GEMM, and the adapter gradients ``dA = U^T X``, ``dB = s dY^T T`` as
  deterministic split-M reductions returned in fp32.
"""
from __future__ import annotations

from types import MethodType
from typing import Any

import torch

from .. import ops
from ..errors import CapabilityError
from ..nf4 import _rows_cols, nibble_order, resolved_nf4_scales


def _geometry(quant_state: Any) -> tuple[int, int]:
    return _rows_cols(quant_state.shape)


class _ScheduledNF4LoRA(torch.autograd.Function):
    """NF4 + LoRA linear with a manually scheduled backward
    (methods/nf4_lora.py:12-113)."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, packed_weight: torch.Tensor, lora_a: torch.Tensor,
                lora_b: torch.Tensor, quant_state: Any, scaling: float,
                decoded_backward_weight: torch.Tensor | None) -> torch.Tensor:
        if x.device.type != "cuda" or packed_weight.device.type != "cuda":
            raise CapabilityError("scheduled NF4-LoRA requires CUDA tensors")
        if packed_weight.requires_grad:
            raise CapabilityError("scheduled NF4-LoRA requires frozen NF4 weights")
        if lora_a.dtype != torch.float32 or lora_b.dtype != torch.float32:
            raise CapabilityError("scheduled NF4-LoRA requires FP32 adapter masters")
        if x.dtype != torch.bfloat16:
            raise CapabilityError("scheduled NF4-LoRA requires BF16 activations")
        n, k = _geometry(quant_state)
        if x.shape[-1] != k:
            raise ValueError(f"input width {x.shape[-1]} does not match in_features {k}")
        if decoded_backward_weight is not None and (
            decoded_backward_weight.shape != (lora_b.shape[0], x.shape[-1])
            or decoded_backward_weight.device != x.device
            or decoded_backward_weight.dtype != x.dtype
        ):
            raise CapabilityError(
                "cached NF4 backward weight must match the decoded weight geometry, "
                "device, and compute dtype"
            )
        flat_x = x.reshape(-1, k)
        scales = resolved_nf4_scales(quant_state)
        low_rank = ops.direct.lora_project(flat_x, None, 0, 1.0, lora_a, 0)
        result = ops.direct.nf4_lora_forward(flat_x, packed_weight.reshape(-1), scales, quant_state.code, n, k,
                                      nibble_order(quant_state), int(quant_state.blocksize), low_rank,
                                      lora_b, float(scaling))
        ctx.quant_state = quant_state
        ctx.scaling = float(scaling)
        ctx.input_shape = x.shape
        # The fused backward decodes NF4 tiles in LDS; a cached dense weight is
        # validated for contract compatibility and holds bit-identical values.
        ctx.has_cached_backward_weight = decoded_backward_weight is not None
        ctx.save_for_backward(x, packed_weight, lora_a, lora_b, low_rank)
        return result.reshape(*x.shape[:-1], n)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_output: torch.Tensor):
        x, packed_weight, lora_a, lora_b, low_rank = ctx.saved_tensors
        qs = ctx.quant_state
        n, k = _geometry(qs)
        flat_x = x.reshape(-1, k)
        flat_grad = grad_output.reshape(-1, n).to(torch.bfloat16)
        scales = resolved_nf4_scales(qs)
        grad_through_b = ops.direct.lora_project(flat_grad, None, 2, ctx.scaling, lora_b, 1)
        grad_x = ops.direct.nf4_lora_backward_input(flat_grad, packed_weight.reshape(-1), scales, qs.code, n, k,
                                             nibble_order(qs), int(qs.blocksize), grad_through_b, lora_a, 1.0)
        grad_a = ops.direct.lora_grad(flat_x, None, 0, grad_through_b, 1.0, 1)
        grad_b = ops.direct.lora_grad(flat_grad, None, 0, low_rank, ctx.scaling, 0)
        return (grad_x.reshape(ctx.input_shape), None, grad_a.to(lora_a.dtype), grad_b.to(lora_b.dtype),
                None, None, None)


def scheduled_nf4_lora(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    lora_a: torch.Tensor,
    lora_b: torch.Tensor,
    quant_state: Any,
    scaling: float,
    decoded_backward_weight: torch.Tensor | None = None,
) -> torch.Tensor:
    """methods/nf4_lora.py:116-133."""
    return _ScheduledNF4LoRA.apply(x, packed_weight, lora_a, lora_b, quant_state, scaling,
                                   decoded_backward_weight)


def _scheduled_forward(module: torch.nn.Module, x: torch.Tensor, *args: Any, **kwargs: Any) -> torch.Tensor:
    """PEFT Linear4bit adapter entry point with strict safe fallback
    (methods/nf4_lora.py:136-165)."""
    if (
        args or kwargs or module.disable_adapters or module.merged
        or x.dtype != torch.bfloat16
        or not torch.is_autocast_enabled("cuda")
        or torch.get_autocast_dtype("cuda") != torch.bfloat16
    ):
        return module._molt_original_forward(x, *args, **kwargs)
    active = list(module.active_adapters)
    if len(active) != 1:
        return module._molt_original_forward(x, *args, **kwargs)
    adapter = active[0]
    if (
        adapter not in module.lora_A
        or adapter in module.lora_variant
        or module.use_dora.get(adapter, False)
        or not isinstance(module.lora_dropout[adapter], torch.nn.Identity)
        or module.base_layer.bias is not None
    ):
        return module._molt_original_forward(x, *args, **kwargs)
    return scheduled_nf4_lora(
        x,
        module.base_layer.weight,
        module.lora_A[adapter].weight,
        module.lora_B[adapter].weight,
        module.base_layer.weight.quant_state,
        float(module.scaling[adapter]),
        getattr(module, "_molt_decoded_backward_weight", None),
    )


def nf4_lora_module_types() -> tuple[type, ...]:
    """Module classes the patchers accept: PEFT's bitsandbytes ``Linear4bit``
    when PEFT is installed, and :class:`molt_amd.modules.NF4LoRALinear`."""
    from ..modules import NF4LoRALinear

    types: list[type] = [NF4LoRALinear]
    try:
        from peft.tuners.lora.bnb import Linear4bit  # type: ignore
        types.append(Linear4bit)
    except Exception:  # PEFT is optional
        pass
    return tuple(types)


def enable_scheduled_nf4_lora(
    model: torch.nn.Module,
    *,
    module_suffixes: tuple[str, ...] | None = None,
    require_narrow_output: bool = False,
    cache_backward_weights: bool = False,
) -> int:
    """Patch compatible NF4-LoRA modules (methods/nf4_lora.py:168-220)."""
    types = nf4_lora_module_types()
    patched = 0
    for module_name, module in model.named_modules():
        if not isinstance(module, types) or hasattr(module, "_molt_original_forward"):
            continue
        if module_suffixes is not None and not module_name.endswith(module_suffixes):
            continue
        if require_narrow_output and not (
            isinstance(getattr(module, "in_features", None), int)
            and isinstance(getattr(module, "out_features", None), int)
            and module.out_features < module.in_features
        ):
            continue
        module._molt_original_forward = module.forward
        if cache_backward_weights:
            from ..nf4 import dequantize_4bit

            with torch.no_grad():
                module._molt_decoded_backward_weight = dequantize_4bit(
                    module.base_layer.weight.data, module.base_layer.weight.quant_state
                ).to(dtype=torch.bfloat16)
        module.forward = MethodType(_scheduled_forward, module)
        patched += 1
    if patched == 0:
        requested = "all modules" if module_suffixes is None else ", ".join(module_suffixes)
        raise CapabilityError(
            f"No compatible PEFT NF4-LoRA modules were found for {requested}"
            + (" with grouped-query geometry" if require_narrow_output else "")
        )
    return patched
