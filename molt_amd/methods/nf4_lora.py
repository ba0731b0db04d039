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

A biased base (Qwen2's q/k/v) adds its bias to the bf16 GEMM output, as the
base linear's own ``F.linear(x, W, bias)`` would before the LoRA term; the
reference's patcher instead falls back to PEFT's forward for such a base
(methods/nf4_lora.py:154). A trainable bias gets ``dY`` summed over tokens.
"""
from __future__ import annotations

from typing import Any

import torch

from .. import ops
from ..errors import CapabilityError
from ..nf4 import _rows_cols, gemv_applies, nf4_gemv_linear, nibble_order, resolved_nf4_scales
from ..patching import is_swapped, lora_operands, original_forward, refusal, swap_forward


def _geometry(quant_state: Any) -> tuple[int, int]:
    return _rows_cols(quant_state.shape)


class _ScheduledNF4LoRA(torch.autograd.Function):
    """NF4 + LoRA linear with a manually scheduled backward
    (methods/nf4_lora.py:12-113)."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, packed_weight: torch.Tensor, lora_a: torch.Tensor,
                lora_b: torch.Tensor, quant_state: Any, scaling: float,
                decoded_backward_weight: torch.Tensor | None, bias: torch.Tensor | None = None,
                decode: bool = False) -> torch.Tensor:
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
        if bias is not None and (bias.shape != (n,) or bias.device != x.device):
            raise ValueError(f"bias must be a ({n},) tensor on {x.device}, got {tuple(bias.shape)} on {bias.device}")
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
        # A (for this projection) and, when a gradient will flow, B (for the
        # backward's) packed in one launch
        ctx.b_packed = None
        if any(ctx.needs_input_grad):
            a_packed, ctx.b_packed = ops.direct.lora_pack_many([lora_a, lora_b], [None, None], [0, 1])
        else:
            a_packed = ops.direct.lora_pack_many([lora_a], [None], [0])[0]
        low_rank = ops.direct.lora_project_packed(flat_x, None, 0, 1.0, a_packed, lora_a.shape[0])
        ctx.wt = None
        if decode and gemv_applies(flat_x, quant_state, lora_a.shape[0]):
            # decode-sized batch with no gradient to flow: the HBM-bound skinny-M
            # GEMV (block scale applied to each block's partial sum), the role
            # bitsandbytes' gemv_4bit plays inside bnb.matmul_4bit. A forward that
            # carries a gradient takes the GEMM on bf16(code * scale) per element,
            # the dequantize_4bit + matmul function of the training forward.
            result = nf4_gemv_linear(flat_x, packed_weight, quant_state, low_rank, lora_b, scaling)
        else:
            args = (flat_x, packed_weight.reshape(-1), resolved_nf4_scales(quant_state), quant_state.code, n, k,
                    nibble_order(quant_state), int(quant_state.blocksize), low_rank, lora_b, float(scaling))
            if ops.keep_weight_transposes() and any(ctx.needs_input_grad):
                # the GEMM also leaves deq(W)^T for the input gradient when it stages the weight
                result, wt = ops.direct.nf4_lora_forward_keep_wt(*args)
                ctx.wt = wt if wt.numel() else None
            else:
                result = ops.direct.nf4_lora_forward(*args)
        if bias is not None:
            result.add_(bias.to(result.dtype))
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
        b_packed, ctx.b_packed = ctx.b_packed, None
        if b_packed is not None:
            grad_through_b = ops.direct.lora_project_packed(flat_grad, None, 2, ctx.scaling, b_packed,
                                                            lora_b.shape[1])
        else:
            grad_through_b = ops.direct.lora_project(flat_grad, None, 2, ctx.scaling, lora_b, 1)
        wt, ctx.wt = ctx.wt, None
        grad_x = ops.direct.nf4_lora_backward_input(flat_grad, packed_weight.reshape(-1), scales, qs.code, n, k,
                                             nibble_order(qs), int(qs.blocksize), grad_through_b, lora_a, 1.0, wt)
        del wt
        # dA = U^T X and dB = s dY^T T in one launch pair (bitwise as two calls)
        grad_a, grad_b = ops.direct.lora_grad_many([flat_x, flat_grad], [None, None], [0, 0],
                                                   [grad_through_b, low_rank], [1.0, ctx.scaling], [1, 0])
        grad_bias = flat_grad.float().sum(0) if ctx.needs_input_grad[7] else None
        return (grad_x.reshape(ctx.input_shape), None, grad_a.to(lora_a.dtype), grad_b.to(lora_b.dtype),
                None, None, None, grad_bias, None)


def scheduled_nf4_lora(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    lora_a: torch.Tensor,
    lora_b: torch.Tensor,
    quant_state: Any,
    scaling: float,
    decoded_backward_weight: torch.Tensor | None = None,
    *,
    bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """methods/nf4_lora.py:116-133, plus an optional base ``bias`` (keyword
    only, so the reference's positional signature is unchanged).

    The skinny-M GEMV serves only calls through which no gradient can flow
    (grad mode off, or no operand requiring grad): decode. Any other call takes
    the dequantised-weight GEMM, whatever its token count."""
    decode = not (torch.is_grad_enabled()
                  and any(t is not None and t.requires_grad for t in (x, lora_a, lora_b, bias)))
    return _ScheduledNF4LoRA.apply(x, packed_weight, lora_a, lora_b, quant_state, scaling,
                                   decoded_backward_weight, bias, decode)


def _scheduled_forward(module: torch.nn.Module, x: torch.Tensor, *args: Any, **kwargs: Any) -> torch.Tensor:
    """Forward of a patched NF4-LoRA projection: the HIP path when the call and
    the adapter allow it, else the projection's own forward (the strict
    fallback of methods/nf4_lora.py:136-165)."""
    why = refusal(x, args, kwargs)
    operands = lora_operands(module, allow_bias=True) if why is None else why
    if isinstance(operands, str):
        return original_forward(module)(x, *args, **kwargs)
    return scheduled_nf4_lora(x, operands.packed, operands.lora_a, operands.lora_b, operands.quant_state,
                              operands.scaling, getattr(module, "_molt_decoded_backward_weight", None),
                              bias=operands.bias)


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


def _narrow(module: torch.nn.Module) -> bool:
    """Grouped-query geometry: integer features with fewer outputs than inputs."""
    width_in, width_out = getattr(module, "in_features", None), getattr(module, "out_features", None)
    return isinstance(width_in, int) and isinstance(width_out, int) and width_out < width_in


def enable_scheduled_nf4_lora(
    model: torch.nn.Module,
    *,
    module_suffixes: tuple[str, ...] | None = None,
    require_narrow_output: bool = False,
    cache_backward_weights: bool = False,
) -> int:
    """Route every selected NF4-LoRA projection of ``model`` through
    :func:`scheduled_nf4_lora` (methods/nf4_lora.py:168-220). A projection is
    selected when it is not yet patched, its qualified name ends with one of
    ``module_suffixes`` (all when None) and, with ``require_narrow_output``, it
    has fewer outputs than inputs. ``cache_backward_weights`` keeps a dense
    bf16 decode of each selected weight (validated by the autograd node; the
    HIP backward decodes bit-identical values in LDS). Returns the count and
    raises CapabilityError when nothing is selected."""
    kinds = nf4_lora_module_types()
    suffixes = None if module_suffixes is None else tuple(module_suffixes)
    selected = [
        module for name, module in model.named_modules()
        if isinstance(module, kinds) and not is_swapped(module)
        and (suffixes is None or name.endswith(suffixes))
        and (not require_narrow_output or _narrow(module))
    ]
    if not selected:
        requested = "all modules" if suffixes is None else ", ".join(suffixes)
        raise CapabilityError(
            f"No compatible PEFT NF4-LoRA modules were found for {requested}"
            + (" with grouped-query geometry" if require_narrow_output else "")
        )
    for module in selected:
        state = {}
        if cache_backward_weights:
            from ..nf4 import dequantize_4bit

            weight = module.base_layer.weight
            with torch.no_grad():
                state["_molt_decoded_backward_weight"] = dequantize_4bit(weight.data, weight.quant_state).to(
                    torch.bfloat16)
        swap_forward(module, _scheduled_forward, **state)
    return len(selected)
