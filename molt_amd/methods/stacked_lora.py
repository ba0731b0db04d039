"""Projections that share one input as one NF4-LoRA node: a decoder layer's
q, k and v projections stacked along their output rows.

The reference runs each projection as its own scheduled node
(methods/nf4_lora.py:12-113, once per projection); this node computes, for
every output column, the product that projection's own node computes — its
NF4 base weight, its own adapter and scale, the same bf16 rounding points —
with the three projections in one launch each where the separate nodes take
three:

* forward: the adapters stacked (``A_stack = [A_q; A_k; A_v; 0]``,
  block-diagonal ``B_blocks``, one launch) and packed (one launch), one
  rank-``lr`` projection ``T = X A_stack^T``, and one GEMM over the weights
  stacked along the output rows (each dequantised into its rows of the staged
  copy), which also leaves ``deq(W)^T`` for the input gradient;
* backward: ``U = bf16(s dY) bf16(B_blocks)`` (one projection), one
  input-gradient GEMM ``dX = dY deq(W) + U bf16(A_stack)`` from the kept
  transpose, and ``dA`` of the stack plus each ``dB`` in one launch pair.

The fp32 sums run in another order than the separate nodes' (a longer
contraction in ``U``, zero blocks in the stacked adapters), so results agree
to rounding, not bitwise. A call the stacked GEMM does not take (a small token
batch, a biased base, differing ranks or scales, anything the scheduled path
refuses) runs each projection's own forward.
"""
from __future__ import annotations

from typing import Any

import torch

from .. import ops
from ..errors import CapabilityError
from ..nf4 import _rows_cols, nibble_order, resolved_nf4_scales
from ..patching import lora_operands, refusal, swap_forward
from .nf4_lora import nf4_lora_module_types

_UNSTACKED = "_molt_unstacked_forward"


def _pad64(n: int) -> int:
    return (n + 63) // 64 * 64


class _StackedNF4LoRA(torch.autograd.Function):
    """Forward and backward of the stacked projections (see the module
    docstring). Inputs: x, the quant states (a tuple), the shared scale, then
    the packed weights, the A and the B masters of every projection."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, quant_states: tuple, scaling: float, *tensors: torch.Tensor):
        n = len(quant_states)
        packed, lora_a, lora_b = tensors[:n], tensors[n:2 * n], tensors[2 * n:]
        k = x.shape[-1]
        rows = [_rows_cols(qs.shape)[0] for qs in quant_states]
        r = lora_a[0].shape[0]
        lr = _pad64(n * r)
        flat_x = x.reshape(-1, k)
        grad = any(ctx.needs_input_grad)
        a_stack, b_blocks = ops.stack_adapters(list(lora_a), list(lora_b), lr)
        a_packed, b_packed = ops.direct.lora_pack_many([a_stack, b_blocks], [None, None], [0, 1])
        low_rank = ops.direct.lora_project_packed(flat_x, None, 0, 1.0, a_packed, lr)
        qs0 = quant_states[0]
        weights = [(p.reshape(-1), resolved_nf4_scales(qs), rw) for p, qs, rw in zip(packed, quant_states, rows)]
        y, wt = ops.nf4_stacked_forward(flat_x, weights, qs0.code, k, nibble_order(qs0), int(qs0.blocksize),
                                        low_rank, b_blocks, float(scaling), grad)
        if grad and wt is None:
            raise CapabilityError("stacked NF4-LoRA: the forward did not leave the transposed weight")
        ctx.quant_states = quant_states
        ctx.rows, ctx.r, ctx.lr, ctx.scaling = rows, r, lr, float(scaling)
        ctx.input_shape = x.shape
        ctx.wt, ctx.b_packed = wt, b_packed
        ctx.save_for_backward(x, a_stack, low_rank, *packed)
        lead = x.shape[:-1]
        outs, n0 = [], 0
        for rw in rows:
            outs.append(y.narrow(1, n0, rw).view(*lead, rw))
            n0 += rw
        return tuple(outs)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, *grads: torch.Tensor):
        x, a_stack, low_rank, *packed = ctx.saved_tensors
        quant_states, rows, r, s = ctx.quant_states, ctx.rows, ctx.r, ctx.scaling
        n = len(rows)
        k = x.shape[-1]
        flat_x = x.reshape(-1, k)
        m = flat_x.shape[0]
        parts = [torch.zeros((m, rw), device=x.device, dtype=torch.bfloat16) if g is None
                 else g.reshape(m, rw).to(torch.bfloat16) for g, rw in zip(grads, rows)]
        flat_grad = torch.cat(parts, dim=1)
        del parts
        b_packed, ctx.b_packed = ctx.b_packed, None
        wt, ctx.wt = ctx.wt, None
        grad_through_b = ops.direct.lora_project_packed(flat_grad, None, 2, s, b_packed, ctx.lr)
        qs0 = quant_states[0]
        weights = [(p.reshape(-1), resolved_nf4_scales(qs), rw) for p, qs, rw in zip(packed, quant_states, rows)]
        grad_x = ops.nf4_stacked_backward_input(flat_grad, weights, qs0.code, k, nibble_order(qs0),
                                                int(qs0.blocksize), wt, grad_through_b, a_stack, 1.0)
        del wt
        # dA of the whole stack (rows of the zero padding are zero) and each
        # dB = s dY_i^T T_i over its column slices, one launch pair
        ls, rmats, n0 = [flat_x], [grad_through_b], 0
        for i, rw in enumerate(rows):
            ls.append(flat_grad[:, n0:n0 + rw])
            rmats.append(low_rank[:, i * r:(i + 1) * r])
            n0 += rw
        grads_ab = ops.direct.lora_grad_many(ls, [None] * (n + 1), [0] * (n + 1), rmats, [1.0] + [s] * n,
                                             [1] + [0] * n)
        grad_a_stack, grad_b = grads_ab[0], grads_ab[1:]
        grad_a = [grad_a_stack[i * r:(i + 1) * r] for i in range(n)]
        return (grad_x.reshape(ctx.input_shape), None, None, *([None] * n), *grad_a, *grad_b)


def stacked_nf4_lora(x: torch.Tensor, packed_weights: list, lora_a: list, lora_b: list, quant_states: list,
                     scaling: float) -> tuple:
    """The outputs of the NF4-LoRA projections of ``x`` (one per weight, each
    ``[..., rows_i]``) through one stacked node; all adapters of one rank and
    one scale. Raises CapabilityError where the stacked GEMM does not apply."""
    return _StackedNF4LoRA.apply(x, tuple(quant_states), float(scaling), *packed_weights, *lora_a, *lora_b)


def _stackable(operands: list, *, compare_codes: bool = False) -> str | None:
    """Why these projections' operands cannot share one node, or None. The
    code tables are compared by value only with ``compare_codes`` (a device
    synchronisation: the patcher does it once; the node then reads the first
    projection's table for all)."""
    first = operands[0]
    qs0 = first.quant_state
    for op in operands:
        if op.bias is not None:
            return "a biased base"
        if op.scaling != first.scaling or op.lora_a.shape[0] != first.lora_a.shape[0]:
            return "adapters of different ranks or scales"
        if op.lora_a.dtype != torch.float32 or op.lora_b.dtype != torch.float32:
            return "adapters that are not FP32 masters"
        qs = op.quant_state
        if (_rows_cols(qs.shape)[1] != _rows_cols(qs0.shape)[1] or int(qs.blocksize) != int(qs0.blocksize)
                or nibble_order(qs) != nibble_order(qs0)
                or (compare_codes and not torch.equal(qs.code.float(), qs0.code.float()))):
            return "weights of different widths or formats"
    if (first.lora_a.shape[0] * len(operands)) > 128:
        return "a stacked rank above 128"
    return None


def _stacked_forward(module: torch.nn.Module, x: torch.Tensor, *args: Any, **kwargs: Any) -> torch.Tensor:
    """Forward of a projection in a stacked group: the first one called
    computes the group through one node and leaves the others their outputs
    for the same input tensor; any other call (another input, a refused call,
    a group the stacked GEMM does not take) runs the projection's own
    forward."""
    stash = module.__dict__.get("_molt_stacked_out")
    if stash is not None:
        module._molt_stacked_out = None
        if stash[0] is x and not args and not kwargs:
            return stash[1]
    group = module._molt_stack_group
    own = getattr(module, _UNSTACKED)
    if module is not group[0] or refusal(x, args, kwargs) is not None:
        return own(x, *args, **kwargs)
    operands = [lora_operands(m) for m in group]
    if any(isinstance(op, str) for op in operands) or _stackable(operands) is not None:
        return own(x, *args, **kwargs)
    if x.dtype != torch.bfloat16 or x.device.type != "cuda":
        return own(x, *args, **kwargs)
    k = x.shape[-1]
    m = x.numel() // k
    n = sum(_rows_cols(op.quant_state.shape)[0] for op in operands)
    if not (x.is_contiguous() and ops._keeps_wt(m, n, k, 1)):
        return own(x, *args, **kwargs)
    try:
        outs = stacked_nf4_lora(x, [op.packed for op in operands], [op.lora_a for op in operands],
                                [op.lora_b for op in operands], [op.quant_state for op in operands],
                                operands[0].scaling)
    except CapabilityError:
        return own(x, *args, **kwargs)
    for other, out in zip(group[1:], outs[1:]):
        other._molt_stacked_out = (x, out)
    return outs[0]


def _clear_stacked_outputs(parent: torch.nn.Module, args: Any) -> None:
    for group in parent._molt_stack_groups:
        for mod in group:
            mod._molt_stacked_out = None


def enable_stacked_nf4_lora(
    model: torch.nn.Module,
    *,
    groups: tuple[tuple[str, ...], ...] = (("q_proj", "k_proj", "v_proj"),),
) -> int:
    """Run each group of sibling NF4-LoRA projections of ``model`` that read
    the same input (a module's children named by one entry of ``groups``, in
    the order its forward calls them) as one stacked node
    (:func:`stacked_nf4_lora`). Each projection keeps the forward it had (the
    scheduled HIP path, say) for the calls the node does not take. Returns the
    number of groups; raises CapabilityError when there is none."""
    kinds = nf4_lora_module_types()
    count = 0
    for parent in model.modules():
        for names in groups:
            members = [getattr(parent, name, None) for name in names]
            if not all(isinstance(mod, kinds) for mod in members):
                continue
            if any(mod.__dict__.get("_molt_stack_group") is not None for mod in members):
                continue
            operands = [lora_operands(mod, check_state=False) for mod in members]
            if any(isinstance(op, str) for op in operands) or _stackable(operands, compare_codes=True) is not None:
                continue
            group = tuple(members)
            for mod in group:
                swap_forward(mod, _stacked_forward, key=_UNSTACKED, _molt_stack_group=group, _molt_stacked_out=None)
            if parent.__dict__.get("_molt_stack_groups") is None:
                # outputs left for a later sibling live only within one call of the parent, so a
                # sibling called before the first projection never takes an earlier call's output
                parent._molt_stack_groups = []
                parent.register_forward_pre_hook(_clear_stacked_outputs)
            parent._molt_stack_groups.append(group)
            count += 1
    if not count:
        raise CapabilityError("No compatible PEFT NF4-LoRA projection groups were found for "
                              + "; ".join("/".join(g) for g in groups))
    return count
