"""Gated NF4-LoRA MLP on MI355X: the drop-in for
``molt_stream.methods.gated_replay`` (methods/gated_replay.py:211-607), plus a
fully fused gate/up/down autograd node.

``asymmetric_gated_nf4_lora`` keeps the reference contract (gate and up come
from their own projection nodes; only the down projection and SwiGLU are
inside this node; up can be rematerialised or offloaded to pinned host
memory). Backward runs the down projection's input gradient and the SwiGLU
backward as ONE NF4-fused GEMM whose epilogue writes ``dgate`` and ``dup``
(``dh`` never reaches HBM), and the down adapter's ``dA = U^T h`` replays
``h = bf16(bf16(silu(g)) u)`` in registers while staging ``g`` and ``u``.

``fused_gated_nf4_lora_mlp`` takes all three projections (the shape of
``_ResidualRecipeGatedNF4LoRA``, methods/gated_replay.py:50-208): gate and up
are ONE dual-accumulator GEMM that also emits ``h``; only ``g`` and ``u`` are
saved, and backward computes ``dX = dg deq(Wg) + du deq(Wu) + LoRA`` as one
contraction over 2I.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from .. import ops
from ..errors import CapabilityError
from ..nf4 import _rows_cols, nibble_order, resolved_nf4_scales
from ..patching import is_swapped, lora_operands, original_forward, refusal, swap_forward
from .nf4_lora import nf4_lora_module_types


def _nf4_lora_forward(x: torch.Tensor, packed_weight: torch.Tensor, lora_a: torch.Tensor,
                      lora_b: torch.Tensor, quant_state: Any, scaling: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(Y, T) for ``Y = X deq(W)^T + s (X A^T) B^T`` (methods/gated_replay.py:211-224)."""
    n, k = _rows_cols(quant_state.shape)
    flat = x.reshape(-1, k)
    t = ops.direct.lora_project(flat, None, 0, 1.0, lora_a, 0)
    y = ops.direct.nf4_lora_forward(flat, packed_weight.reshape(-1), resolved_nf4_scales(quant_state),
                             quant_state.code, n, k, nibble_order(quant_state), int(quant_state.blocksize),
                             t, lora_b, float(scaling))
    return y.reshape(*x.shape[:-1], n), t


class _AsymmetricGatedNF4LoRA(torch.autograd.Function):
    """methods/gated_replay.py:256-407."""

    @staticmethod
    def forward(ctx: Any, x, gate, up, up_packed_weight, up_lora_a, up_lora_b, down_packed_weight,
                down_lora_a, down_lora_b, up_quant_state, down_quant_state, up_scaling, down_scaling,
                rematerialize_up, offload_up, host_up, offload_gate, host_gate):
        if x.device.type != "cuda" or x.dtype != torch.bfloat16:
            raise CapabilityError("asymmetric gated replay requires CUDA BF16 tensors")
        ctx.up_quant_state = up_quant_state
        ctx.down_quant_state = down_quant_state
        ctx.up_scaling = float(up_scaling)
        ctx.down_scaling = float(down_scaling)
        ctx.rematerialize_up = bool(rematerialize_up)
        ctx.offload_up = bool(offload_up)
        ctx.offload_gate = bool(offload_gate)
        if ctx.rematerialize_up and ctx.offload_up:
            raise CapabilityError("up projection cannot be replayed and offloaded")
        if ctx.offload_up:
            if host_up.device.type != "cpu" or not host_up.is_pinned():
                raise CapabilityError("gated activation offload requires pinned host storage")
            if host_up.shape != up.shape or host_up.dtype != up.dtype:
                raise CapabilityError("gated activation host storage must match the up result")
        if ctx.offload_gate:
            if host_gate.device.type != "cpu" or not host_gate.is_pinned():
                raise CapabilityError("gated activation offload requires pinned gate storage")
            if host_gate.shape != gate.shape or host_gate.dtype != gate.dtype:
                raise CapabilityError("gated activation host storage must match the gate result")
        gated = ops.direct.silu_mul_forward(gate, up, True)
        result, low_rank = _nf4_lora_forward(gated, down_packed_weight, down_lora_a, down_lora_b,
                                             down_quant_state, down_scaling)
        del gated
        if ctx.offload_up:
            host_up.copy_(up.detach(), non_blocking=True)
        if ctx.offload_gate:
            host_gate.copy_(gate.detach(), non_blocking=True)
        saved = (x, host_gate if ctx.offload_gate else gate, up_packed_weight, up_lora_a, up_lora_b,
                 down_packed_weight, down_lora_a, down_lora_b, low_rank)
        if ctx.offload_up:
            saved += (host_up,)
        elif not ctx.rematerialize_up:
            saved += (up,)
        ctx.save_for_backward(*saved)
        return result

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_output: torch.Tensor):
        (x, stored_gate, up_packed_weight, up_lora_a, up_lora_b, down_packed_weight, down_lora_a,
         down_lora_b, low_rank, *retained) = ctx.saved_tensors
        gate = stored_gate.to(grad_output.device, non_blocking=True) if ctx.offload_gate else stored_gate
        if ctx.rematerialize_up:
            up, _ = _nf4_lora_forward(x, up_packed_weight, up_lora_a, up_lora_b, ctx.up_quant_state,
                                      ctx.up_scaling)
        elif ctx.offload_up:
            up = retained[0].to(grad_output.device, non_blocking=True)
        else:
            up = retained[0]
        qs = ctx.down_quant_state
        h_dim, i_dim = _rows_cols(qs.shape)
        dy = grad_output.reshape(-1, h_dim).to(torch.bfloat16)
        g2, u2 = gate.reshape(-1, i_dim), up.reshape(-1, i_dim)
        grad_through_b = ops.direct.lora_project(dy, None, 2, ctx.down_scaling, down_lora_b, 1)
        grad_gate, grad_up = ops.direct.nf4_swiglu_backward(dy, down_packed_weight.reshape(-1), resolved_nf4_scales(qs),
                                                     qs.code, h_dim, i_dim, nibble_order(qs), grad_through_b,
                                                     down_lora_a, g2, u2)
        grad_down_a = ops.direct.lora_grad(g2, u2, 1, grad_through_b, 1.0, 1)
        grad_down_b = ops.direct.lora_grad(dy, None, 0, low_rank, ctx.down_scaling, 0)
        return (None, grad_gate.reshape(gate.shape), grad_up.reshape(up.shape), None, None, None, None,
                grad_down_a.to(down_lora_a.dtype), grad_down_b.to(down_lora_b.dtype),
                None, None, None, None, None, None, None, None, None)


def asymmetric_gated_nf4_lora(
    x: torch.Tensor,
    gate: torch.Tensor,
    up: torch.Tensor,
    up_packed_weight: torch.Tensor,
    up_lora_a: torch.Tensor,
    up_lora_b: torch.Tensor,
    down_packed_weight: torch.Tensor,
    down_lora_a: torch.Tensor,
    down_lora_b: torch.Tensor,
    up_quant_state: Any,
    down_quant_state: Any,
    up_scaling: float,
    down_scaling: float,
    rematerialize_up: bool = True,
    offload_up: bool = False,
    host_up: torch.Tensor | None = None,
    offload_gate: bool = False,
    host_gate: torch.Tensor | None = None,
) -> torch.Tensor:
    """methods/gated_replay.py:410-457."""
    if offload_up and host_up is None:
        raise CapabilityError("gated activation offload requires a host buffer")
    if host_up is None:
        host_up = torch.empty(0)
    if offload_gate and host_gate is None:
        raise CapabilityError("gated activation offload requires a gate host buffer")
    if host_gate is None:
        host_gate = torch.empty(0)
    return _AsymmetricGatedNF4LoRA.apply(
        x, gate, up, up_packed_weight, up_lora_a, up_lora_b, down_packed_weight, down_lora_a,
        down_lora_b, up_quant_state, down_quant_state, up_scaling, down_scaling, rematerialize_up,
        offload_up, host_up, offload_gate, host_gate,
    )


# --------------------------------------------------------------------------
# Fully fused gate/up/down node
# --------------------------------------------------------------------------
def _keep_wt(ctx) -> bool:
    """Keep the forward's transposed bf16 weights for the backward (when both
    stage them) if a gradient will be taken and the policy allows
    (:func:`molt_amd.ops.keep_weight_transposes`)."""
    return ops.keep_weight_transposes() and any(ctx.needs_input_grad)


def _take_wts(ctx):
    """The transposed weights the forward kept, dropped from ``ctx`` so the
    backward holds the only references."""
    wts, ctx.wts = ctx.wts, None
    return wts


def _fused_forward(x, gate_packed, gate_a, gate_b, up_packed, up_a, up_b, down_packed, down_a, down_b,
                   gate_qs, up_qs, down_qs, gate_scaling, up_scaling, down_scaling, keep_wt=False, grad=False):
    """Forward of the fused gated MLP on ``x`` [..., H]: gate/up as one
    dual-accumulator GEMM that also emits h, then the down projection.
    Returns (y [tokens, H], gate, up, h, T_gu, T_d, (H, I, r), wts, bpacks)
    with wts the bf16 transposed weights (deq(Wg)^T, deq(Wu)^T, deq(Wd)^T) the
    GEMMs wrote for the backward when ``keep_wt`` (each an empty tensor where
    they did not stage the weight), else None, and bpacks the backward
    projections' packed B_d, B_g, B_u when ``grad`` (packed in the same launch
    as the forward's adapters), else None."""
    if x.device.type != "cuda" or x.dtype != torch.bfloat16:
        raise CapabilityError("fused gated NF4-LoRA MLP requires CUDA BF16 tensors")
    for t in (gate_a, gate_b, up_a, up_b, down_a, down_b):
        if t.dtype != torch.float32:
            raise CapabilityError("fused gated NF4-LoRA MLP requires FP32 adapter masters")
    i_dim, h_dim = _rows_cols(gate_qs.shape)
    if _rows_cols(up_qs.shape) != (i_dim, h_dim) or _rows_cols(down_qs.shape) != (h_dim, i_dim):
        raise ValueError("gate/up must be [I, H] and down [H, I]")
    if nibble_order(gate_qs) != nibble_order(up_qs) or int(gate_qs.blocksize) != 64 \
            or int(up_qs.blocksize) != 64 or int(down_qs.blocksize) != 64:
        raise CapabilityError("fused gated MLP requires NF4 block size 64 with a shared packing")
    r = gate_a.shape[0]
    if up_a.shape[0] != r:
        raise ValueError("gate and up adapters must share a rank")
    flat = x.reshape(-1, h_dim)
    # every adapter operand of the step in one launch: [A_gate; A_up] and A_down
    # for the forward's projections, B_down, B_gate, B_up for the backward's
    if grad:
        packs = ops.direct.lora_pack_many([gate_a, down_a, down_b, gate_b, up_b], [up_a, None, None, None, None],
                                          [0, 0, 1, 1, 1])
        bpacks = tuple(packs[2:])
    else:
        packs = ops.direct.lora_pack_many([gate_a, down_a], [up_a, None], [0, 0])
        bpacks = None
    t_gu = ops.direct.lora_project_packed(flat, None, 0, 1.0, packs[0], 2 * r)
    gu_args = (flat, gate_packed.reshape(-1), resolved_nf4_scales(gate_qs), up_packed.reshape(-1),
               resolved_nf4_scales(up_qs), gate_qs.code, i_dim, h_dim, nibble_order(gate_qs), t_gu, gate_b, up_b,
               float(gate_scaling), float(up_scaling))
    wts = None
    if keep_wt:
        gate, up, gated, wgt, wut = ops.direct.nf4_gateup_forward_keep_wt(*gu_args)
    else:
        gate, up, gated = ops.direct.nf4_gateup_forward(*gu_args)
    t_d = ops.direct.lora_project_packed(gated, None, 0, 1.0, packs[1], r)
    d_args = (gated, down_packed.reshape(-1), resolved_nf4_scales(down_qs), down_qs.code, h_dim, i_dim,
              nibble_order(down_qs), 64, t_d, down_b, float(down_scaling))
    if keep_wt:
        y, wdt = ops.direct.nf4_lora_forward_keep_wt(*d_args)
        wts = (wgt, wut, wdt)
    else:
        y = ops.direct.nf4_lora_forward(*d_args)
    return y, gate, up, gated, t_gu, t_d, (h_dim, i_dim, r), wts, bpacks


def _fused_backward(grad_output, flat, gate, up, gated, t_gu, t_d, gate_packed, gate_a, gate_b, up_packed,
                    up_a, up_b, down_packed, down_a, down_b, qs, scaling, dims, norm=None, wts=None, bpacks=None):
    """Backward of the fused gated MLP. ``flat`` is the projections' input
    [tokens, H]; ``gated`` is h when the forward kept it, else None (replayed
    from gate and up). With ``norm = (source, inv_rms, weight, offset)`` and
    ``flat`` None, the input is the frozen RMSNorm's output, replayed from its
    bf16 source as the gate/up adapters' gradient stages it. ``wts``: the
    transposed weights a keep_wt forward wrote (or None); the input gradients
    read them instead of staging the weights again (bitwise the same).
    ``bpacks``: the packed B_d, B_g, B_u the forward made (or None: packed
    here); the projections give bitwise the same U either way.
    Returns (dX [tokens, H], dA_g, dB_g, dA_u, dB_u, dA_d, dB_d)."""
    wgt, wut, wdt = wts if wts is not None else (None, None, None)
    del wts   # each copy is released as soon as its input gradient has run
    gate_qs, up_qs, down_qs = qs
    s_g, s_u, s_d = scaling
    h_dim, i_dim, r = dims
    dy = grad_output.reshape(-1, h_dim).to(torch.bfloat16)
    if bpacks is not None:
        u_d = ops.direct.lora_project_packed(dy, None, 2, s_d, bpacks[0], r)
    else:
        u_d = ops.direct.lora_project(dy, None, 2, s_d, down_b, 1)
    dg, du = ops.direct.nf4_swiglu_backward(dy, down_packed.reshape(-1), resolved_nf4_scales(down_qs), down_qs.code,
                                     h_dim, i_dim, nibble_order(down_qs), u_d, down_a, gate, up, wdt)
    del wdt
    # U_g and U_u as the column halves of one [tokens, 2r] matrix: the paired
    # input gradient reads the halves in place and dA_gate/dA_up share one pass
    if bpacks is not None:
        u_gu = ops.direct.lora_project_pair_packed(dg, du, s_g, s_u, bpacks[1], bpacks[2], r)
    else:
        u_gu = ops.direct.lora_project_pair(dg, du, s_g, s_u, gate_b, up_b)
    u_g, u_u = u_gu[:, :r], u_gu[:, r:]
    dx = ops.direct.nf4_lora_backward_input_pair(
        dg, du, gate_packed.reshape(-1), resolved_nf4_scales(gate_qs), up_packed.reshape(-1),
        resolved_nf4_scales(up_qs), gate_qs.code, i_dim, h_dim, nibble_order(gate_qs), u_g, u_u, gate_a,
        up_a, wgt, wut)
    del wgt, wut
    # Every adapter gradient in one call with one split-sum launch, each bitwise
    # its own call: dB_d over dY, dB_g over dg and dB_u over du (one launch
    # together), dA_d over h (kept from the forward, or replayed from gate and
    # up: bitwise the same), and dA_gate / dA_up as one pass over X with
    # [U_g | U_u] (X materialised, or the frozen RMSNorm's output replayed
    # from its source).
    ls, l2s, modes = [dy, dg, du], [None, None, None], [0, 0, 0]
    rmats, scales = [t_d, t_gu[:, :r], t_gu[:, r:]], [float(s_d), float(s_g), float(s_u)]
    if gated is not None:
        ls.append(gated); l2s.append(None); modes.append(0)
    else:
        ls.append(gate); l2s.append(up); modes.append(1)
    norm_args = ()
    if norm is None:
        ls.append(flat); l2s.append(None); modes.append(0)
    else:
        ls.append(norm[0]); l2s.append(None); modes.append(2)
        norm_args = (norm[1], norm[2], float(norm[3]))
    rmats += [u_d, u_gu]
    scales += [1.0, 1.0]
    d_down_b, d_gate_b, d_up_b, d_down_a, d_gu_a = ops.direct.lora_grad_many(ls, l2s, modes, rmats, scales,
                                                                            [0, 0, 0, 1, 1], *norm_args)
    return dx, d_gu_a[:r], d_gate_b, d_gu_a[r:], d_up_b, d_down_a, d_down_b


class _FusedGatedNF4LoRA(torch.autograd.Function):
    """Gated NF4-LoRA MLP with gate/up as one dual-accumulator GEMM and the
    SwiGLU backward fused into the down projection's input gradient."""

    @staticmethod
    def forward(ctx: Any, x, gate_packed, gate_a, gate_b, up_packed, up_a, up_b, down_packed, down_a,
                down_b, gate_qs, up_qs, down_qs, gate_scaling, up_scaling, down_scaling, save_gated):
        y, gate, up, gated, t_gu, t_d, dims, wts, bpacks = _fused_forward(
            x, gate_packed, gate_a, gate_b, up_packed, up_a, up_b, down_packed, down_a, down_b, gate_qs,
            up_qs, down_qs, gate_scaling, up_scaling, down_scaling, keep_wt=_keep_wt(ctx),
            grad=any(ctx.needs_input_grad))
        if not save_gated:
            gated = None  # replayed in backward from (gate, up)
        ctx.qs = (gate_qs, up_qs, down_qs)
        ctx.scaling = (float(gate_scaling), float(up_scaling), float(down_scaling))
        ctx.dims = dims
        ctx.input_shape = x.shape
        ctx.save_for_backward(x.reshape(-1, dims[0]), gate, up, gated, t_gu, t_d, gate_packed, gate_a, gate_b,
                              up_packed, up_a, up_b, down_packed, down_a, down_b)
        ctx.wts, ctx.bpacks = wts, bpacks
        return y.reshape(*x.shape[:-1], dims[0])

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_output: torch.Tensor):
        (flat, gate, up, gated, t_gu, t_d, gate_packed, gate_a, gate_b, up_packed, up_a, up_b, down_packed,
         down_a, down_b) = ctx.saved_tensors
        dx, dag, dbg, dau, dbu, dad, dbd = _fused_backward(
            grad_output, flat, gate, up, gated, t_gu, t_d, gate_packed, gate_a, gate_b, up_packed, up_a, up_b,
            down_packed, down_a, down_b, ctx.qs, ctx.scaling, ctx.dims, wts=_take_wts(ctx),
            bpacks=ctx.bpacks)
        return (dx.reshape(ctx.input_shape), None, dag, dbg, None, dau, dbu, None, dad, dbd,
                None, None, None, None, None, None, None)


def fused_gated_nf4_lora_mlp(
    x: torch.Tensor,
    gate_packed_weight: torch.Tensor, gate_lora_a: torch.Tensor, gate_lora_b: torch.Tensor,
    up_packed_weight: torch.Tensor, up_lora_a: torch.Tensor, up_lora_b: torch.Tensor,
    down_packed_weight: torch.Tensor, down_lora_a: torch.Tensor, down_lora_b: torch.Tensor,
    gate_quant_state: Any, up_quant_state: Any, down_quant_state: Any,
    gate_scaling: float, up_scaling: float, down_scaling: float, save_gated: bool = True,
) -> torch.Tensor:
    """``down(silu(gate(x)) * up(x))`` with NF4-LoRA projections as one autograd node.

    ``save_gated`` keeps ``h = silu(gate) * up`` (bf16 [tokens, I]) for the
    backward, whose down-adapter gradient then reads h instead of replaying it
    from gate and up (half the bytes, no SiLU). ``False`` replays it, as the
    reference's gated-replay node does, saving that memory."""
    return _FusedGatedNF4LoRA.apply(
        x, gate_packed_weight, gate_lora_a, gate_lora_b, up_packed_weight, up_lora_a, up_lora_b,
        down_packed_weight, down_lora_a, down_lora_b, gate_quant_state, up_quant_state, down_quant_state,
        gate_scaling, up_scaling, down_scaling, bool(save_gated))


# --------------------------------------------------------------------------
# RMSNorm replay (methods/gated_replay.py:13-208)
# --------------------------------------------------------------------------
@dataclass
class _RMSNormReplayRecipe:
    """What recomputes the normalised MLP input from the residual stream
    (methods/gated_replay.py:13-30); ``materialize`` runs the HIP RMSNorm
    forward, bitwise the output of FrozenRMSNormBF16 on the same source."""
    source: torch.Tensor
    weight: torch.Tensor
    eps: float
    weight_offset: float
    packed_count: int = 0
    target: torch.Tensor | None = None

    def materialize(self) -> torch.Tensor:
        return ops.direct.rmsnorm_forward(self.source, self.weight, float(self.eps), float(self.weight_offset))


def _leave_recipe(mlp: torch.nn.Module, norm: torch.nn.Module, source: torch.Tensor, output: torch.Tensor) -> None:
    keep = torch.is_grad_enabled() and output.dtype == torch.bfloat16
    mlp._molt_norm_replay_recipe = _RMSNormReplayRecipe(
        source=source, weight=norm.weight, eps=float(norm.variance_epsilon),
        weight_offset=float(norm.weight_offset), target=output) if keep else None


def _leave_replay_recipe(mlp: torch.nn.Module):
    """Forward hook for a frozen RMSNorm: after each call it leaves on ``mlp``
    the recipe that recomputes the norm's output from its input, or None when
    the output will not be differentiated as bf16 (grad mode off, or another
    dtype). The MLP's patched forward consumes the recipe when its input is
    that very output (methods/gated_replay.py:13-47)."""

    def hook(norm: torch.nn.Module, inputs: tuple, output: torch.Tensor) -> None:
        _leave_recipe(mlp, norm, inputs[0], output)

    return hook


def _replayable_norm_forward(module: torch.nn.Module, hidden: torch.Tensor, *args: Any, **kwargs: Any) -> torch.Tensor:
    """The reference's forward replacement for a norm wired by hand
    (methods/gated_replay.py:32-47): runs ``module._molt_original_forward`` and
    leaves the recipe on ``module._molt_target_mlp``, as the hook of
    :func:`enable_rmsnorm_replay` does."""
    result = module._molt_original_forward(hidden, *args, **kwargs)
    _leave_recipe(module._molt_target_mlp, module, hidden, result)
    return result


class _ResidualRecipeGatedNF4LoRA(torch.autograd.Function):
    """Gated NF4+LoRA MLP that retains the residual instead of the normalised
    input (methods/gated_replay.py:50-208).

    Forward is the fused gated MLP on ``normalized``. It saves the residual
    ``source``, gate and up (h is replayed from them, as the reference does),
    and the two rank-r projections. Backward runs the fused backward, in which
    only the gate/up adapters' gradient reads the normalised input: for a bf16
    source that gradient applies the norm to the source as it stages it (one
    pass for the per-row scale, nothing stored; bitwise the materialised
    values), otherwise the RMSNorm kernel re-materialises the input first. It
    returns the gradient of ``normalized`` (the norm's own node carries it to
    the residual) and the six adapter gradients."""

    @staticmethod
    def forward(ctx: Any, source, normalized, gate_packed_weight, gate_lora_a, gate_lora_b, up_packed_weight,
                up_lora_a, up_lora_b, down_packed_weight, down_lora_a, down_lora_b, gate_quant_state,
                up_quant_state, down_quant_state, gate_scaling, up_scaling, down_scaling, norm_weight,
                norm_eps, norm_weight_offset):
        if source.shape != normalized.shape:
            raise ValueError("the residual source and the normalised input must have the same shape")
        y, gate, up, _, t_gu, t_d, dims, wts, bpacks = _fused_forward(
            normalized, gate_packed_weight, gate_lora_a, gate_lora_b, up_packed_weight, up_lora_a, up_lora_b,
            down_packed_weight, down_lora_a, down_lora_b, gate_quant_state, up_quant_state, down_quant_state,
            gate_scaling, up_scaling, down_scaling, keep_wt=_keep_wt(ctx), grad=any(ctx.needs_input_grad))
        ctx.wts, ctx.bpacks = wts, bpacks
        ctx.qs = (gate_quant_state, up_quant_state, down_quant_state)
        ctx.scaling = (float(gate_scaling), float(up_scaling), float(down_scaling))
        ctx.dims = dims
        ctx.input_shape = normalized.shape
        ctx.norm_eps = float(norm_eps)
        ctx.norm_weight_offset = float(norm_weight_offset)
        ctx.save_for_backward(source, gate, up, t_gu, t_d, gate_packed_weight, gate_lora_a, gate_lora_b,
                              up_packed_weight, up_lora_a, up_lora_b, down_packed_weight, down_lora_a,
                              down_lora_b, norm_weight)
        return y.reshape(*normalized.shape[:-1], dims[0])

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_output: torch.Tensor):
        (source, gate, up, t_gu, t_d, gate_packed, gate_a, gate_b, up_packed, up_a, up_b, down_packed, down_a,
         down_b, norm_weight) = ctx.saved_tensors
        flat_source = source.reshape(-1, ctx.dims[0])
        if ops.norm_replay_fusable(flat_source):
            # the normalised input is formed as the adapters' gradient stages
            # it, from the source and the norm's per-row scale: never stored
            inv = ops.direct.rmsnorm_inv(flat_source, norm_weight, ctx.norm_eps)
            flat, norm = None, (flat_source, inv, norm_weight, ctx.norm_weight_offset)
        else:
            normalized = _RMSNormReplayRecipe(source, norm_weight, ctx.norm_eps, ctx.norm_weight_offset).materialize()
            flat, norm = normalized.reshape(-1, ctx.dims[0]), None
        dx, dag, dbg, dau, dbu, dad, dbd = _fused_backward(
            grad_output, flat, gate, up, None, t_gu, t_d, gate_packed, gate_a, gate_b, up_packed, up_a, up_b,
            down_packed, down_a, down_b, ctx.qs, ctx.scaling, ctx.dims, norm, wts=_take_wts(ctx),
            bpacks=ctx.bpacks)
        return (None, dx.reshape(ctx.input_shape), None, dag, dbg, None, dau, dbu, None, dad, dbd,
                None, None, None, None, None, None, None, None, None)


_REPLAY_HOOK = "_molt_replay_hook"
_NORM_FIELDS = ("weight", "variance_epsilon", "weight_offset")


def enable_rmsnorm_replay(model: torch.nn.Module) -> int:
    """Pair each decoder layer's ``post_attention_layernorm`` with its ``mlp``
    through a forward hook (:func:`_leave_replay_recipe`), so an MLP routed by
    :func:`enable_fused_gated_nf4_lora` keeps the residual instead of the
    normalised input (``_ResidualRecipeGatedNF4LoRA``). The norm must carry
    ``weight``, ``variance_epsilon`` and ``weight_offset`` (FrozenRMSNormBF16).
    The reference defines the recipe but wires no caller; this is that wiring.
    Returns the number of pairs; a norm already wired is skipped."""
    pairs = []
    for layer in model.modules():
        norm, mlp = getattr(layer, "post_attention_layernorm", None), getattr(layer, "mlp", None)
        if norm is None or mlp is None or hasattr(norm, _REPLAY_HOOK):
            continue
        if all(hasattr(norm, f) for f in _NORM_FIELDS):
            pairs.append((norm, mlp))
    if not pairs:
        raise CapabilityError("No frozen RMSNorm -> MLP pairs were found (run enable_frozen_rmsnorm_bf16 first)")
    for norm, mlp in pairs:
        mlp._molt_norm_replay_recipe = None
        setattr(norm, _REPLAY_HOOK, norm.register_forward_hook(_leave_replay_recipe(mlp)))
    return len(pairs)


# --------------------------------------------------------------------------
# Patchers (methods/gated_replay.py:460-607)
# --------------------------------------------------------------------------
_PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
_SILU_NAMES = frozenset({"SiLU", "SiLUActivation"})


def _gated_mlp(module: torch.nn.Module, kinds: tuple[type, ...], adapted: tuple[str, ...]) -> bool:
    """A not yet patched SiLU-gated MLP whose three projections are NF4-LoRA
    modules and whose ``adapted`` projections have a usable adapter."""
    if is_swapped(module) or not all(hasattr(module, n) for n in _PROJECTIONS + ("act_fn",)):
        return False
    if type(module.act_fn).__name__ not in _SILU_NAMES:
        return False
    if not all(isinstance(getattr(module, n), kinds) for n in _PROJECTIONS):
        return False
    return all(not isinstance(lora_operands(getattr(module, n), check_state=False), str) for n in adapted)


def _gated_mlps(model: torch.nn.Module, adapted: tuple[str, ...]) -> list[torch.nn.Module]:
    kinds = nf4_lora_module_types()
    return [m for m in model.modules() if _gated_mlp(m, kinds, adapted)]


def _pinned_like(module: torch.nn.Module, slot: str, like: torch.Tensor, what: str) -> torch.Tensor:
    """The pinned host buffer kept in ``module.<slot>``, (re)allocated to match
    ``like``; allocation is refused while a CUDA graph is being captured."""
    buf = getattr(module, slot, None)
    if buf is None or buf.shape != like.shape or buf.dtype != like.dtype:
        if torch.cuda.is_current_stream_capturing():
            raise CapabilityError(f"gated activation {what} was not warmed up")
        buf = torch.empty_like(like, device="cpu", pin_memory=True)
        setattr(module, slot, buf)
    return buf


def _asymmetric_mlp_forward(module: torch.nn.Module, x: torch.Tensor, *args: Any, **kwargs: Any) -> torch.Tensor:
    why = refusal(x, args, kwargs, need_grad=True)
    up_ops = lora_operands(module.up_proj) if why is None else why
    down_ops = lora_operands(module.down_proj) if why is None else why
    if isinstance(up_ops, str) or isinstance(down_ops, str):
        return original_forward(module)(x, *args, **kwargs)
    gate = module.gate_proj(x)
    up = module.up_proj(x)
    host_up = _pinned_like(module, "_molt_host_up", up, "host storage") if module._molt_offload_up else None
    host_gate = (_pinned_like(module, "_molt_host_gate", gate, "gate storage")
                 if module._molt_offload_gate else None)
    return asymmetric_gated_nf4_lora(
        x, gate, up, up_ops.packed, up_ops.lora_a, up_ops.lora_b, down_ops.packed, down_ops.lora_a,
        down_ops.lora_b, up_ops.quant_state, down_ops.quant_state, up_ops.scaling, down_ops.scaling,
        module._molt_rematerialize_up, module._molt_offload_up, host_up, module._molt_offload_gate, host_gate)


def enable_asymmetric_gated_replay(
    model: torch.nn.Module,
    *,
    rematerialize_up: bool = True,
    rematerialize_blocks: int | None = None,
    offload_blocks: int = 0,
    offload_gate_blocks: int = 0,
) -> int:
    """Route SiLU-gated NF4-LoRA MLP blocks through
    :func:`asymmetric_gated_nf4_lora` (methods/gated_replay.py:540-607). The
    first ``rematerialize_blocks`` blocks (all when None) replay the up
    projection in the backward; the first ``offload_blocks`` /
    ``offload_gate_blocks`` keep up / gate in pinned host memory instead.
    Returns the number of blocks patched."""
    limits = (("rematerialize_blocks", rematerialize_blocks, "replay"), ("offload_blocks", offload_blocks, "offload"),
              ("offload_gate_blocks", offload_gate_blocks, "gate offload"))
    for name, value, _ in limits:
        if value is not None and value < 0:
            raise ValueError(f"{name} cannot be negative")
    if rematerialize_up and (offload_blocks or offload_gate_blocks):
        raise ValueError("up projection replay and offload are mutually exclusive")
    blocks = _gated_mlps(model, ("up_proj", "down_proj"))
    if not blocks:
        raise CapabilityError("No compatible SiLU-gated PEFT NF4 MLP blocks were found")
    for _, value, label in limits:
        if value is not None and value > len(blocks):
            raise CapabilityError(f"requested {value} {label} blocks but only {len(blocks)} compatible blocks "
                                  "were found")
    replayed = len(blocks) if rematerialize_blocks is None else rematerialize_blocks
    for index, block in enumerate(blocks):
        swap_forward(block, _asymmetric_mlp_forward, _molt_rematerialize_up=bool(rematerialize_up and index < replayed),
                     _molt_offload_up=index < offload_blocks, _molt_offload_gate=index < offload_gate_blocks)
    return len(blocks)


def _fused_mlp_forward(module: torch.nn.Module, x: torch.Tensor, *args: Any, **kwargs: Any) -> torch.Tensor:
    recipe, module._molt_norm_replay_recipe = getattr(module, "_molt_norm_replay_recipe", None), None
    why = refusal(x, args, kwargs)
    parts = [lora_operands(getattr(module, n)) if why is None else why for n in _PROJECTIONS]
    if any(isinstance(p, str) for p in parts):
        return original_forward(module)(x, *args, **kwargs)
    g, u, d = parts
    weights = (g.packed, g.lora_a, g.lora_b, u.packed, u.lora_a, u.lora_b, d.packed, d.lora_a, d.lora_b,
               g.quant_state, u.quant_state, d.quant_state, g.scaling, u.scaling, d.scaling)
    if recipe is not None and recipe.target is x and recipe.source.shape == x.shape:
        return _ResidualRecipeGatedNF4LoRA.apply(recipe.source, x, *weights, recipe.weight, recipe.eps,
                                                 recipe.weight_offset)
    return fused_gated_nf4_lora_mlp(x, *weights)


def enable_fused_gated_nf4_lora(model: torch.nn.Module) -> int:
    """Route every compatible SiLU-gated NF4-LoRA MLP through
    :func:`fused_gated_nf4_lora_mlp` (all three adapters must be usable); an
    MLP paired with its norm by :func:`enable_rmsnorm_replay` runs the
    residual-recipe node instead. Returns the number patched."""
    blocks = _gated_mlps(model, _PROJECTIONS)
    if not blocks:
        raise CapabilityError("No compatible SiLU-gated PEFT NF4 MLP blocks were found")
    for block in blocks:
        swap_forward(block, _fused_mlp_forward)
    return len(blocks)
