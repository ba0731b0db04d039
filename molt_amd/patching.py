"""Forward swapping and per-call routing for the patched modules.

The patchers of this package replace a module instance's ``forward`` and keep
the replaced callable under a fixed attribute, ``_molt_original_forward`` for
the NF4-LoRA projections and gated MLPs (``_molt_original_mlp_forward`` for
the fused SiLU MLP): other MOLT code tests for those attributes to tell a
patched module from an unpatched one. :func:`swap_forward` and
:func:`original_forward` own that bookkeeping.

Whether a patched NF4-LoRA projection may run the HIP kernels on a given call
is decided by two ordered rule tables: :data:`ADAPTER_STRUCTURE` (what the
module is: one LoRA adapter without DoRA, dropout or a variant, over an NF4
base that, for the gated-MLP nodes, has no bias) and :data:`ADAPTER_STATE`
plus :data:`CALL_RULES` (what the call is: adapters enabled and unmerged, a
bf16 input under bf16 CUDA autocast, no extra arguments). The first rule that
fails names the reason the original forward runs instead, and :func:`refusal`
returns it, so a caller can see why a module stayed on the original path. The
conditions are those the reference's patchers check (methods/nf4_lora.py:136-165;
methods/gated_replay.py:460-520), except that the scheduled projection also
runs a biased base (Qwen2's q/k/v): its autograd node adds the bias after the
NF4 GEMM, where the reference falls back to PEFT's forward.
"""
from __future__ import annotations

from dataclasses import dataclass
from types import MethodType
from typing import Any, Callable

import torch
from torch import nn

ORIGINAL_FORWARD = "_molt_original_forward"


def swap_forward(module: nn.Module, replacement: Callable[..., Any], *, key: str = ORIGINAL_FORWARD,
                 **state: Any) -> None:
    """Bind ``replacement(module, ...)`` as the instance's forward, keep the
    forward it replaces under ``key`` and set the per-module ``state``
    attributes the replacement reads."""
    setattr(module, key, module.forward)
    for name, value in state.items():
        setattr(module, name, value)
    module.forward = MethodType(replacement, module)


def is_swapped(module: nn.Module, key: str = ORIGINAL_FORWARD) -> bool:
    return hasattr(module, key)


def original_forward(module: nn.Module, key: str = ORIGINAL_FORWARD) -> Callable[..., Any]:
    return getattr(module, key)


@dataclass(frozen=True)
class LoraOperands:
    """What the kernels read from one NF4 projection with a single active
    LoRA adapter: the packed base weight and its quant state, the fp32 LoRA
    masters, the adapter's scale and the base's bias (None for most)."""
    packed: torch.Tensor
    lora_a: torch.Tensor
    lora_b: torch.Tensor
    quant_state: Any
    scaling: float
    bias: torch.Tensor | None = None


def _single_adapter(module: nn.Module) -> str | None:
    names = list(module.active_adapters)
    return names[0] if len(names) == 1 else None


# (reason, predicate(module, adapter name)); adapter name is None unless
# exactly one adapter is active, so that rule comes first.
ADAPTER_STRUCTURE: tuple[tuple[str, Callable[[nn.Module, Any], bool]], ...] = (
    ("not exactly one active adapter", lambda m, a: a is not None),
    ("the active adapter has no LoRA A", lambda m, a: a in m.lora_A),
    ("the adapter is a LoRA variant", lambda m, a: a not in m.lora_variant),
    ("the adapter uses DoRA", lambda m, a: not m.use_dora.get(a, False)),
    ("the adapter applies dropout", lambda m, a: isinstance(m.lora_dropout[a], nn.Identity)),
)

# The gated-MLP nodes have no bias term; only the scheduled projection takes one.
BIAS_RULE = ("the NF4 base projection has a bias", lambda m, a: getattr(m.base_layer, "bias", None) is None)

ADAPTER_STATE: tuple[tuple[str, Callable[[nn.Module, Any], bool]], ...] = (
    ("adapters are disabled", lambda m, a: not m.disable_adapters),
    ("the adapter is merged into the base", lambda m, a: not m.merged),
)


def _bf16_autocast() -> bool:
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16


# (reason, predicate(x, args, kwargs))
CALL_RULES: tuple[tuple[str, Callable[[torch.Tensor, tuple, dict], bool]], ...] = (
    ("extra forward arguments", lambda x, args, kwargs: not args and not kwargs),
    ("the input is not bf16", lambda x, args, kwargs: x.dtype == torch.bfloat16),
    ("bf16 CUDA autocast is not active", lambda x, args, kwargs: _bf16_autocast()),
)

GRAD_RULE = ("autograd is disabled", lambda x, args, kwargs: torch.is_grad_enabled())


def lora_operands(module: nn.Module, *, check_state: bool = True, allow_bias: bool = False) -> LoraOperands | str:
    """The operands of ``module``'s active adapter, or the reason it has none
    the kernels can use. ``check_state=False`` applies only the structural
    rules (what a patcher checks once, at patch time); ``allow_bias`` accepts a
    biased base (the scheduled projection adds it)."""
    name = _single_adapter(module)
    rules = ADAPTER_STRUCTURE + (() if allow_bias else (BIAS_RULE,)) + (ADAPTER_STATE if check_state else ())
    for reason, ok in rules:
        if not ok(module, name):
            return reason
    base = module.base_layer
    return LoraOperands(base.weight, module.lora_A[name].weight, module.lora_B[name].weight,
                        base.weight.quant_state, float(module.scaling[name]), getattr(base, "bias", None))


def refusal(x: torch.Tensor, args: tuple = (), kwargs: dict | None = None, *, need_grad: bool = False) -> str | None:
    """The first call rule ``x`` fails, or None when the HIP path may run."""
    rules = CALL_RULES + ((GRAD_RULE,) if need_grad else ())
    for reason, ok in rules:
        if not ok(x, args, kwargs or {}):
            return reason
    return None
