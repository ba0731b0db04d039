"""Load-time preparation of a decoder for the NF4 QLoRA path, and the
bitsandbytes 4-bit serialisation of an NF4 weight.

MOLT quantises at load time. transformers' ``from_pretrained`` with
``BitsAndBytesConfig(load_in_4bit=True, bnb_4bit_quant_type="nf4",
bnb_4bit_use_double_quant=True, bnb_4bit_compute_dtype=bfloat16)`` turns every
linear projection into a bitsandbytes ``Params4bit``; the remaining weights
are frozen, and PEFT's ``get_peft_model(LoraConfig(r, lora_alpha,
target_modules))`` wraps the targets with LoRA adapters
(training/qlora.py:323-347,393-420; target names from
training/qlora.py:212-215). :func:`prepare_nf4_qlora` does the same for a
loaded ``nn.Module`` with this library's GPU quantiser
(``molt_nf4_quantize`` + ``molt_nf4_double_quantize``, block 64, nested
statistics in blocks of 256), producing :class:`~molt_amd.modules.NF4LoRALinear`
modules that the patchers accept.

A checkpoint that bitsandbytes already quantised (``save_pretrained`` of a
4-bit model) stores, per projection ``<prefix>``: ``<prefix>.weight`` (the
packed bytes), ``<prefix>.weight.absmax``, ``<prefix>.weight.quant_map`` and,
with nested statistics, ``<prefix>.weight.nested_absmax`` and
``<prefix>.weight.nested_quant_map``, plus
``<prefix>.weight.quant_state.bitsandbytes__nf4``: a uint8 tensor holding the
UTF-8 JSON of the non-tensor fields (``quant_type``, ``blocksize``, ``dtype``,
``shape``, ``nested_blocksize``, ``nested_dtype``, ``nested_offset``). This is
bitsandbytes' ``QuantState.as_dict(packed=True)`` layout (bitsandbytes 0.50.2,
``uv.lock:46-47``; the library is absent from the reference tree and from this
image, so the layout is restated from its published format and its parity is
unpinned: no file written by bitsandbytes itself is available to test against).
:func:`nf4_state_dict` writes it and :func:`load_prequantized_nf4` reads it.
"""
from __future__ import annotations

import json
from typing import Any, Iterable

import torch
from torch import nn

from .errors import CapabilityError
from .modules import NF4Linear, NF4LoRALinear
from .nf4 import NIBBLE_HIGH_FIRST, QuantState

_QS_KEY = "quant_state.bitsandbytes__nf4"
_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).split(".")[-1]


def _targets(model: nn.Module, target_modules: str | Iterable[str]) -> list[tuple[nn.Module, str, nn.Linear, str]]:
    """(parent, attribute, module, qualified name) of every nn.Linear the
    target spec selects. "all-linear" is PEFT's meaning: every linear layer
    except the output embedding."""
    output = model.get_output_embeddings() if hasattr(model, "get_output_embeddings") else None
    names = None if target_modules == "all-linear" else tuple(target_modules)
    found = []
    for parent_name, parent in model.named_modules():
        for attr, child in parent.named_children():
            if not isinstance(child, nn.Linear) or child is output:
                continue
            if names is not None and attr not in names:
                continue
            found.append((parent, attr, child, f"{parent_name}.{attr}" if parent_name else attr))
    return found


def quantize_linears_nf4(model: nn.Module, target_modules: str | Iterable[str] = "all-linear", *,
                         device: torch.device | str = "cuda", blocksize: int = 64,
                         compress_statistics: bool = True, bias_dtype: torch.dtype | None = None) -> int:
    """Replace each selected ``nn.Linear`` with a frozen :class:`NF4Linear`
    quantised on ``device``, one module at a time so that only one dense weight
    is on the GPU at once. A bias stays unquantised and frozen, on ``device`` in
    ``bias_dtype`` (the linear's own dtype when None), as bitsandbytes'
    ``Linear4bit`` keeps it (Qwen2's q/k/v projections carry one). Returns the
    number replaced."""
    count = 0
    for parent, attr, lin, name in _targets(model, target_modules):
        dense = lin.weight.detach().to(device=device, dtype=torch.float32)
        bias = None
        if lin.bias is not None:
            bias = lin.bias.detach().to(device=device, dtype=bias_dtype or lin.bias.dtype)
        setattr(parent, attr, NF4Linear.from_dense(dense, blocksize=blocksize,
                                                   compress_statistics=compress_statistics, bias=bias))
        del dense
        count += 1
    if not count:
        raise CapabilityError("No linear projections matched the NF4 targets")
    return count


def add_lora_adapters(model: nn.Module, r: int, lora_alpha: float,
                      target_modules: str | Iterable[str] = "all-linear", adapter_name: str = "default") -> int:
    """Wrap each selected :class:`NF4Linear` with an :class:`NF4LoRALinear`
    (PEFT's initialisation: A Kaiming-uniform, B zero; fp32 masters)."""
    names = None if target_modules == "all-linear" else tuple(target_modules)
    count = 0
    for parent in list(model.modules()):
        for attr, child in list(parent.named_children()):
            if isinstance(child, NF4Linear) and (names is None or attr in names):
                setattr(parent, attr, NF4LoRALinear(child, r, lora_alpha, adapter_name))
                count += 1
    if not count:
        raise CapabilityError("No NF4 projections matched the LoRA targets")
    return count


def prepare_nf4_qlora(model: nn.Module, r: int, lora_alpha: float,
                      target_modules: str | Iterable[str] = "all-linear", *,
                      device: torch.device | str = "cuda", dtype: torch.dtype = torch.bfloat16) -> nn.Module:
    """Freeze the model, quantise the target projections to NF4 on the GPU,
    move every other weight to ``device`` in ``dtype`` (embeddings, norms,
    output head) and add LoRA adapters with fp32 masters. Returns the model."""
    for p in model.parameters():
        p.requires_grad_(False)
    quantize_linears_nf4(model, target_modules, device=device, bias_dtype=dtype)
    for module in model.modules():
        if isinstance(module, (NF4Linear, NF4LoRALinear)):
            continue
        for name, p in list(module.named_parameters(recurse=False)):
            p.data = p.data.to(device=device, dtype=dtype if p.is_floating_point() else p.dtype)
        for name, b in list(module.named_buffers(recurse=False)):
            module._buffers[name] = b.to(device)
    add_lora_adapters(model, r, lora_alpha, target_modules)
    return model


# --------------------------------------------------------------------------
# bitsandbytes 4-bit serialisation
# --------------------------------------------------------------------------
def quant_state_as_dict(qs: QuantState) -> dict[str, Any]:
    """The fields of bitsandbytes' ``QuantState.as_dict(packed=True)``."""
    if qs.quant_type != "nf4":
        raise CapabilityError(f"only NF4 states serialise here (got {qs.quant_type})")
    if int(getattr(qs, "nibble_order", NIBBLE_HIGH_FIRST)) != NIBBLE_HIGH_FIRST:
        raise CapabilityError("bitsandbytes stores element 2i in the high nibble; repack first")
    meta: dict[str, Any] = {"quant_type": "nf4", "blocksize": int(qs.blocksize),
                            "dtype": _dtype_name(qs.dtype), "shape": [int(v) for v in qs.shape]}
    out: dict[str, Any] = {"absmax": qs.absmax, "quant_map": qs.code}
    if qs.nested:
        s2 = qs.state2
        out["nested_absmax"] = s2.absmax
        out["nested_quant_map"] = s2.code
        meta.update({"nested_blocksize": int(s2.blocksize), "nested_dtype": _dtype_name(s2.dtype),
                     "nested_offset": float(qs.offset)})
    out[_QS_KEY] = torch.tensor(list(json.dumps(meta).encode("utf-8")), dtype=torch.uint8)
    return out


def quant_state_from_dict(entries: dict[str, torch.Tensor], device: torch.device | str | None = None) -> QuantState:
    """Inverse of :func:`quant_state_as_dict` (keys without the weight prefix)."""
    if _QS_KEY not in entries:
        raise CapabilityError(f"not a bitsandbytes NF4 state (missing {_QS_KEY})")
    meta = json.loads(bytes(entries[_QS_KEY].cpu().tolist()).decode("utf-8"))
    if meta.get("quant_type") != "nf4":
        raise CapabilityError(f"only NF4 states load here (got {meta.get('quant_type')})")
    dev = device if device is not None else entries["absmax"].device
    dtype = _DTYPES.get(meta.get("dtype", "bfloat16"), torch.bfloat16)
    state2 = offset = None
    if "nested_absmax" in entries:
        state2 = QuantState(entries["nested_absmax"].to(dev, torch.float32), entries["nested_absmax"].shape,
                            entries["nested_quant_map"].to(dev, torch.float32), int(meta["nested_blocksize"]),
                            "dynamic", torch.float32)
        offset = torch.tensor(float(meta["nested_offset"]), dtype=torch.float32, device=dev)
    absmax = entries["absmax"].to(dev)
    return QuantState(absmax, meta["shape"], entries["quant_map"].to(dev, torch.float32), int(meta["blocksize"]),
                      "nf4", dtype, offset, state2, NIBBLE_HIGH_FIRST)


def nf4_state_dict(model: nn.Module) -> dict[str, torch.Tensor]:
    """State dict of ``model`` with every NF4 weight in bitsandbytes' packed
    layout (``<prefix>.weight`` plus ``<prefix>.weight.<field>``); other
    entries as ``model.state_dict()`` has them. Tensors are moved to the CPU."""
    out: dict[str, torch.Tensor] = {}
    nf4_prefixes = set()
    for name, module in model.named_modules():
        if isinstance(module, NF4Linear):
            key = f"{name}.weight" if name else "weight"
            nf4_prefixes.add(key)
            out[key] = module.weight.detach().reshape(-1, 1).cpu()
            for field, value in quant_state_as_dict(module.weight.quant_state).items():
                out[f"{key}.{field}"] = value.detach().cpu()
    for key, value in model.state_dict().items():
        if key not in nf4_prefixes and key not in out:
            out[key] = value.detach().cpu()
    return out


def load_prequantized_nf4(model: nn.Module, state: dict[str, torch.Tensor], *,
                          device: torch.device | str = "cuda") -> int:
    """Replace each ``nn.Linear`` whose ``<prefix>.weight`` carries a
    bitsandbytes NF4 quant state in ``state`` with an :class:`NF4Linear` holding
    those bytes and statistics on ``device``, and its bias: ``<prefix>.bias``
    from ``state`` when present, else the module's own (a module with a bias
    keeps one; a checkpoint bias for a bias-free module is an error). Returns
    the number replaced; the other entries are left for
    ``model.load_state_dict(strict=False)``."""
    count = 0
    for parent_name, parent in list(model.named_modules()):
        for attr, child in list(parent.named_children()):
            key = f"{parent_name}.{attr}.weight" if parent_name else f"{attr}.weight"
            if f"{key}.{_QS_KEY}" not in state or not isinstance(child, (nn.Linear, NF4Linear)):
                continue
            fields = {k[len(key) + 1:]: v for k, v in state.items() if k.startswith(key + ".")}
            qs = quant_state_from_dict(fields, device)
            out_f, in_f = int(qs.shape[0]), int(qs.shape[1])
            if isinstance(child, nn.Linear) and (child.out_features, child.in_features) != (out_f, in_f):
                raise ValueError(f"{key}: checkpoint shape {(out_f, in_f)} does not match the module")
            packed = state[key].to(device=device, dtype=torch.uint8).reshape(-1, 1)
            if packed.numel() != (out_f * in_f + 1) // 2:
                raise ValueError(f"{key}: {packed.numel()} packed bytes for a {out_f}x{in_f} weight")
            bias_key = key[:-len("weight")] + "bias"
            own_bias = child.bias
            if bias_key in state:
                if own_bias is None and isinstance(child, nn.Linear):
                    raise ValueError(f"{bias_key}: the checkpoint has a bias but the module is bias-free")
                dtype = own_bias.dtype if own_bias is not None else state[bias_key].dtype
                bias = state[bias_key].to(device=device, dtype=dtype)
            else:
                bias = None if own_bias is None else own_bias.detach().to(device)
            setattr(parent, attr, NF4Linear(packed, qs, bias))
            count += 1
    return count
