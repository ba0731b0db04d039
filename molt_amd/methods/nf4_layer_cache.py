"""Scoped dense decode of one decoder layer's NF4 projections: the drop-in for
``molt_stream.methods.nf4_layer_cache`` (methods/nf4_layer_cache.py:22-66).

Inside the context every NF4 base projection of the layer computes
``F.linear`` over a bf16 decode of its weight, made once on entry by the HIP
dequant kernel (bit-exact with the reference's decode); the LoRA modules and
their fp32 masters are untouched. Every base is validated before anything is
decoded or swapped, and each swap is an entry of one ``ExitStack``, so leaving
the context, normally or by an exception, puts every forward back in reverse
order and drops the dense weights."""
from __future__ import annotations

from contextlib import ExitStack, contextmanager
from functools import partial
from typing import Iterator

import torch
from torch.nn import functional as F

from ..errors import CapabilityError
from ..nf4 import dequantize_4bit
from .nf4_lora import nf4_lora_module_types


def _refuse(base: torch.nn.Module) -> str | None:
    weight = base.weight
    if weight.requires_grad or getattr(weight, "quant_state", None) is None:
        return "layer cache requires frozen NF4 base weights"
    if base.bias is not None:
        return "layer cache has not qualified biased NF4 projections"
    return None


@contextmanager
def _dense_forward(base: torch.nn.Module) -> Iterator[None]:
    """Make ``base`` a plain bf16 linear over its decoded weight until exit."""
    own = base.__dict__.get("forward")          # an instance-level forward to put back, if any
    weight = base.weight
    dense = dequantize_4bit(weight.data, weight.quant_state).to(torch.bfloat16)
    base.forward = partial(F.linear, weight=dense, bias=None)
    try:
        yield
    finally:
        if own is None:
            del base.forward
        else:
            base.forward = own


@contextmanager
def dense_nf4_layer_cache(layer: torch.nn.Module) -> Iterator[int]:
    """Decode the frozen NF4 base projections of ``layer`` for the duration of
    the context; yields how many were decoded. Raises CapabilityError for a
    trainable or quant-state-less base, a biased base, or a layer without NF4
    projections."""
    kinds = nf4_lora_module_types()
    bases = [module.base_layer for module in layer.modules() if isinstance(module, kinds)]
    for base in bases:
        reason = _refuse(base)
        if reason:
            raise CapabilityError(reason)
    if not bases:
        raise CapabilityError("decoder layer contains no PEFT NF4 projections")
    with ExitStack() as swaps:
        for base in bases:
            swaps.enter_context(_dense_forward(base))
        yield len(bases)
