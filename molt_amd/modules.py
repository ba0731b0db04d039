"""NF4-LoRA modules with the attribute structure of PEFT's bitsandbytes
``Linear4bit`` adapter layer, the type MOLT's patchers dispatch on
(methods/nf4_lora.py:185-212; methods/gated_replay.py:460-479,556-580).

PEFT and bitsandbytes are not part of this stack, so :class:`NF4LoRALinear`
provides what those patchers read: ``base_layer.weight`` (a frozen uint8
parameter carrying ``quant_state``), ``base_layer.bias``, ``lora_A`` /
``lora_B`` / ``lora_dropout`` / ``scaling`` keyed by adapter name,
``active_adapters``, ``disable_adapters``, ``merged``, ``use_dora``,
``lora_variant``, ``in_features`` and ``out_features``. Its own forward is the
PEFT dataflow (dense NF4 base GEMM plus the separate LoRA branch under bf16
autocast), which the patchers keep as ``_molt_original_forward``.
"""
from __future__ import annotations

import math

import torch
from torch import nn
from torch.nn import functional as F

from .nf4 import QuantState, dequantize_4bit, gemv_applies, nf4_gemv_linear, quantize_4bit


class NF4Linear(nn.Module):
    """Frozen NF4 base projection (the ``base_layer`` of a LoRA adapter), with
    an optional frozen bias (bitsandbytes' ``Linear4bit`` keeps the linear's
    bias unquantised; Qwen2's q/k/v projections carry one)."""

    def __init__(self, packed: torch.Tensor, quant_state: QuantState, bias: torch.Tensor | None = None) -> None:
        super().__init__()
        self.weight = nn.Parameter(packed, requires_grad=False)
        self.weight.quant_state = quant_state
        self.out_features, self.in_features = int(quant_state.shape[0]), int(quant_state.shape[1])
        if bias is not None and tuple(bias.shape) != (self.out_features,):
            raise ValueError(f"bias shape {tuple(bias.shape)} does not match out_features {self.out_features}")
        self.bias = None if bias is None else nn.Parameter(bias.detach(), requires_grad=False)

    @classmethod
    def from_dense(cls, dense: torch.Tensor, blocksize: int = 64, compress_statistics: bool = True,
                   bias: torch.Tensor | None = None) -> "NF4Linear":
        packed, qs = quantize_4bit(dense, blocksize=blocksize, compress_statistics=compress_statistics)
        return cls(packed, qs, bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        qs = self.weight.quant_state
        bias_grad = self.bias is not None and self.bias.requires_grad
        if not (torch.is_grad_enabled() and (x.requires_grad or bias_grad)) and x.device.type == "cuda":
            flat = x.reshape(-1, self.in_features)
            if gemv_applies(flat, qs):
                # decode (1..16 tokens, no autograd): stream the packed weight once
                y = nf4_gemv_linear(flat, self.weight, qs)
                if self.bias is not None:
                    y = y + self.bias.to(y.dtype)
                return y.reshape(*x.shape[:-1], self.out_features)
        dense = dequantize_4bit(self.weight.data, qs).to(x.dtype)
        return F.linear(x, dense, None if self.bias is None else self.bias.to(x.dtype))


class NF4LoRALinear(nn.Module):
    """LoRA adapter over an :class:`NF4Linear` base, laid out like PEFT's ``Linear4bit``."""

    def __init__(self, base: NF4Linear, r: int, lora_alpha: float, adapter_name: str = "default") -> None:
        super().__init__()
        self.base_layer = base
        self.in_features, self.out_features = base.in_features, base.out_features
        self.r = {adapter_name: r}
        self.lora_alpha = {adapter_name: lora_alpha}
        self.scaling = {adapter_name: lora_alpha / r}
        dev = base.weight.device
        self.lora_A = nn.ModuleDict({adapter_name: nn.Linear(self.in_features, r, bias=False, device=dev)})
        self.lora_B = nn.ModuleDict({adapter_name: nn.Linear(r, self.out_features, bias=False, device=dev)})
        self.lora_dropout = nn.ModuleDict({adapter_name: nn.Identity()})
        self.use_dora = {adapter_name: False}
        self.lora_variant: dict = {}
        self.active_adapters = [adapter_name]
        self.disable_adapters = False
        self.merged = False
        nn.init.kaiming_uniform_(self.lora_A[adapter_name].weight, a=math.sqrt(5))
        nn.init.zeros_(self.lora_B[adapter_name].weight)

    def forward(self, x: torch.Tensor, *args, **kwargs) -> torch.Tensor:
        result = self.base_layer(x)
        if self.disable_adapters or self.merged:
            return result
        for name in self.active_adapters:
            a, b = self.lora_A[name], self.lora_B[name]
            result = result + b(a(self.lora_dropout[name](x))) * self.scaling[name]
        return result


class GatedMLP(nn.Module):
    """SiLU-gated MLP ``down(silu(gate(x)) * up(x))`` (kernels/fused.py:24-32)
    with NF4-LoRA projections named as in Qwen2/Llama decoders."""

    def __init__(self, gate_proj: nn.Module, up_proj: nn.Module, down_proj: nn.Module) -> None:
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj
        self.act_fn = nn.SiLU()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))


def synthetic_nf4_lora(out_features: int, in_features: int, r: int, alpha: float, *, device,
                       generator: torch.Generator, weight_std: float = 0.02,
                       b_std: float = 0.01) -> NF4LoRALinear:
    """Seeded NF4-LoRA projection: W ~ N(0, weight_std) quantised to NF4 with
    block 64 and double-quantised absmax, A ~ U(+-1/sqrt(in)), B ~ N(0, b_std)."""
    dense = torch.randn(out_features, in_features, generator=generator, device=device) * weight_std
    base = NF4Linear.from_dense(dense)
    del dense
    mod = NF4LoRALinear(base, r, alpha)
    bound = 1.0 / math.sqrt(in_features)
    with torch.no_grad():
        mod.lora_A["default"].weight.copy_(
            torch.rand(r, in_features, generator=generator, device=device) * (2 * bound) - bound)
        mod.lora_B["default"].weight.copy_(
            torch.randn(out_features, r, generator=generator, device=device) * b_std)
    return mod
