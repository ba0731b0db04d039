"""NF4 formats and their GPU codec.

Two layouts are supported, both decoded by the same HIP kernels:

* the bitsandbytes layout consumed by MOLT's training path
  (methods/nf4_lora.py, methods/nf4_backward.py:97-105,145-164): element 2i in
  the high nibble, block size 64, absmax double-quantised to uint8 against a
  256-entry dynamic map in blocks of 256 with an fp32 ``absmax2`` per block and
  a mean ``offset``. :class:`QuantState` mirrors the attributes of
  ``bitsandbytes.functional.QuantState`` that the hot path reads;
* MOLT's clean-room layout (streaming/nf4.py:21-91, :class:`NF4Tensor`):
  element 2i in the low nibble, one fp32 absmax per block, any even block size
  >= 16, zero padding to a whole block.

Quantisation decisions follow streaming/nf4.py:57-61 in both layouts: fp32
``x / absmax`` and the first index of the nearest code.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from . import ops
from .errors import CapabilityError

NIBBLE_LOW_FIRST = 0
NIBBLE_HIGH_FIRST = 1

# streaming/nf4.py:10-18 (MOLT's NormalFloat-4 literals).
NF4_CODEBOOK = torch.tensor(
    [
        -1.0, -0.6961928, -0.52507305, -0.3949175,
        -0.28444138, -0.18477343, -0.09105004, 0.0,
        0.0795803, 0.1609302, 0.2461123, 0.33791524,
        0.44070983, 0.562617, 0.72295684, 1.0,
    ],
    dtype=torch.float32,
)


def dynamic_map(signed: bool = True, max_exponent_bits: int = 7, total_bits: int = 8) -> torch.Tensor:
    """The 256-entry dynamic quantisation map of bitsandbytes'
    ``create_dynamic_map`` (bitsandbytes 0.50.2; the dependency is not part of
    the reference tree), used as ``state2.code`` for nested absmax.

    Decade i (of ``max_exponent_bits``) holds the midpoints of an fp32
    ``linspace(0.1, 1, 2**i + 1)`` scaled by ``10**(i - 6)`` (the scale rounded
    to fp32, the product in fp32), with both signs when ``signed``; 0 and 1
    complete the table, which is returned sorted."""
    non_sign_bits = total_bits - 1
    extra = 2 ** (non_sign_bits - max_exponent_bits) - 1
    plan = [(i, 2 ** (i + non_sign_bits - max_exponent_bits + (0 if signed else 1)) + 1)
            for i in range(max_exponent_bits)]
    if extra > 0:
        plan.append((max_exponent_bits - 1, extra + 1))
    parts = [torch.tensor([0.0, 1.0])]
    for decade, points in plan:
        edges = torch.linspace(0.1, 1.0, points, dtype=torch.float32)
        mids = (edges[1:] + edges[:-1]) / 2.0
        level = mids * (10.0 ** (decade - (max_exponent_bits - 1)))
        parts += [level, -level] if signed else [level]
    table = torch.cat(parts)
    table = torch.cat([table, torch.zeros(2 ** total_bits - table.numel())])
    return torch.sort(table).values


class QuantState:
    """The QuantState attributes MOLT's hot path reads
    (methods/nf4_backward.py:147-163,180,197,215): ``quant_type``, ``blocksize``,
    ``shape``, ``code``, ``absmax``, ``nested``, ``state2``, ``offset``, ``dtype``
    and the ``_molt_resolved_scales`` cache slot. ``nibble_order`` records the
    packing (1 = bitsandbytes, high nibble first)."""

    def __init__(self, absmax: torch.Tensor, shape, code: torch.Tensor, blocksize: int = 64,
                 quant_type: str = "nf4", dtype: torch.dtype = torch.bfloat16,
                 offset: torch.Tensor | float | None = None, state2: "QuantState | None" = None,
                 nibble_order: int = NIBBLE_HIGH_FIRST) -> None:
        self.absmax = absmax
        self.shape = torch.Size(shape)
        self.code = code
        self.blocksize = int(blocksize)
        self.quant_type = quant_type
        self.dtype = dtype
        self.offset = offset
        self.state2 = state2
        self.nested = state2 is not None
        self.nibble_order = int(nibble_order)
        self._molt_offset_value: float | None = None

    @property
    def offset_value(self) -> float:
        """``float(offset)``, read from the device once and cached."""
        if self._molt_offset_value is None:
            self._molt_offset_value = 0.0 if self.offset is None else float(self.offset)
        return self._molt_offset_value

    def to(self, device) -> "QuantState":
        moved = QuantState(
            self.absmax.to(device), self.shape, self.code.to(device), self.blocksize, self.quant_type,
            self.dtype, self.offset.to(device) if isinstance(self.offset, torch.Tensor) else self.offset,
            self.state2.to(device) if self.state2 is not None else None, self.nibble_order)
        moved._molt_offset_value = self._molt_offset_value
        return moved


def _check_state(quant_state: Any) -> None:
    if getattr(quant_state, "quant_type", None) != "nf4":
        raise CapabilityError("packed backward requires NF4 quantization")


def nibble_order(quant_state: Any) -> int:
    return int(getattr(quant_state, "nibble_order", NIBBLE_HIGH_FIRST))


def _offset(quant_state: Any) -> float:
    if isinstance(quant_state, QuantState):
        return quant_state.offset_value
    return float(quant_state.offset)


def quantize_4bit(A: torch.Tensor, blocksize: int = 64, compress_statistics: bool = True,
                  quant_type: str = "nf4", code: torch.Tensor | None = None,
                  nibble_order: int = NIBBLE_HIGH_FIRST) -> tuple[torch.Tensor, QuantState]:
    """GPU NF4 quantiser with the signature of
    ``bitsandbytes.functional.quantize_4bit`` as MOLT calls it
    (tests/kernels/test_nf4_lora.py:24-26; training/qlora.py:332-337).

    Returns the packed bytes as a ``[(n+1)//2, 1]`` uint8 column and a
    :class:`QuantState`. ``compress_statistics`` double-quantises the absmax."""
    if quant_type != "nf4":
        raise CapabilityError("only NF4 quantization is implemented")
    if A.device.type != "cuda":
        raise CapabilityError("NF4 quantization requires a CUDA tensor on a ROCm GPU")
    dev = A.device
    cb = (NF4_CODEBOOK if code is None else code).to(dev, torch.float32)
    packed, absmax = ops.direct.nf4_quantize(A, blocksize, nibble_order, cb)
    n = A.numel()
    packed = packed[: (n + 1) // 2].reshape(-1, 1)
    dtype = A.dtype if A.dtype in (torch.bfloat16, torch.float16, torch.float32) else torch.bfloat16
    if not compress_statistics:
        return packed, QuantState(absmax, A.shape, cb, blocksize, "nf4", dtype, None, None, nibble_order)
    code2 = dynamic_map().to(dev)
    q, absmax2, offset = ops.direct.nf4_double_quantize(absmax, code2, 256)
    state2 = QuantState(absmax2, (absmax2.numel(),), code2, 256, "dynamic", torch.float32)
    qs = QuantState(q, A.shape, cb, blocksize, "nf4", dtype, offset, state2, nibble_order)
    return packed, qs


def resolved_nf4_scales(quant_state: Any) -> torch.Tensor:
    """fp32 scale per block, resolved once and cached on the state
    (methods/nf4_backward.py:145-164). Nested statistics resolve as
    ``fp32(fp32(code2[q] * absmax2[j]) + offset)``."""
    _check_state(quant_state)
    cached = getattr(quant_state, "_molt_resolved_scales", None)
    if isinstance(cached, torch.Tensor) and cached.device == quant_state.absmax.device:
        return cached
    if quant_state.nested:
        s2 = quant_state.state2
        scales = ops.direct.nf4_resolve_scales(quant_state.absmax, s2.absmax, s2.code, _offset(quant_state),
                                        int(s2.blocksize))
    else:
        scales = quant_state.absmax.float()
    quant_state._molt_resolved_scales = scales
    return scales


def dequantize_4bit(A: torch.Tensor, quant_state: Any, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Dense decode ``bf16(fp32(code[nibble] * scale))`` with the signature of
    ``bitsandbytes.functional.dequantize_4bit`` (methods/nf4_lora.py:97-98)."""
    _check_state(quant_state)
    n_rows, n_cols = _rows_cols(quant_state.shape)
    dtype = out_dtype or getattr(quant_state, "dtype", torch.bfloat16)
    if dtype not in (torch.bfloat16, torch.float32):
        raise CapabilityError(f"NF4 dequantize supports bf16 and fp32 outputs (got {dtype})")
    packed = A.reshape(-1)
    if quant_state.nested:
        s2 = quant_state.state2
        dense = ops.direct.nf4_dequantize_nested(packed, quant_state.absmax, s2.absmax, s2.code, quant_state.code,
                                          _offset(quant_state), n_rows, n_cols, int(quant_state.blocksize),
                                          int(s2.blocksize), nibble_order(quant_state), dtype)
    else:
        dense = ops.direct.nf4_dequantize(packed, quant_state.absmax, quant_state.code, n_rows, n_cols,
                                   int(quant_state.blocksize), nibble_order(quant_state), dtype)
    return dense.reshape(quant_state.shape)


GEMV_MAX_TOKENS = 16
GEMV_MAX_RANK = 128


def gemv_applies(flat_x: torch.Tensor, quant_state: Any, rank: int = 0) -> bool:
    """True when ``flat_x`` [tokens, in_features] is a decode-sized batch the
    skinny-M GEMV serves: 1..16 tokens, NF4 block 64, in_features a multiple of
    64, LoRA rank <= 128 and 16-byte aligned contiguous bf16 rows."""
    _, k = _rows_cols(quant_state.shape)
    return (1 <= flat_x.shape[0] <= GEMV_MAX_TOKENS and flat_x.dtype == torch.bfloat16
            and int(quant_state.blocksize) == 64 and k % 64 == 0 and rank <= GEMV_MAX_RANK
            and flat_x.is_contiguous() and flat_x.data_ptr() % 16 == 0)


def nf4_gemv_linear(flat_x: torch.Tensor, packed: torch.Tensor, quant_state: Any,
                    low_rank: torch.Tensor | None = None, lora_b: torch.Tensor | None = None,
                    scaling: float = 0.0) -> torch.Tensor:
    """``Y = X deq(W)^T (+ T bf16(s B)^T)`` for 1..16 tokens through the
    skinny-M NF4 GEMV (the decode step of training/qlora.py:1332-1358). Reads
    nested statistics directly, so the weight needs no resolved scale cache."""
    n, k = _rows_cols(quant_state.shape)
    if quant_state.nested:
        s2 = quant_state.state2
        return ops.direct.nf4_gemv(flat_x, packed.reshape(-1), None, quant_state.absmax, s2.absmax, s2.code,
                                   _offset(quant_state), int(s2.blocksize), quant_state.code, n, k,
                                   nibble_order(quant_state), low_rank, lora_b, float(scaling))
    return ops.direct.nf4_gemv(flat_x, packed.reshape(-1), quant_state.absmax.float(), None, None, None, 0.0, 256,
                               quant_state.code, n, k, nibble_order(quant_state), low_rank, lora_b,
                               float(scaling))


def _rows_cols(shape) -> tuple[int, int]:
    shape = tuple(int(v) for v in shape)
    if len(shape) == 0:
        return 1, 1
    rows = shape[0]
    cols = 1
    for v in shape[1:]:
        cols *= v
    return rows, cols


# ------------------------------------------------------------------------
# MOLT clean-room layout (streaming/nf4.py:21-91)
# ------------------------------------------------------------------------
@dataclass(frozen=True)
class NF4DevicePayload:
    packed: torch.Tensor
    scales: torch.Tensor
    shape: tuple[int, ...]
    block_size: int
    elements: int

    def dequantize(self, dtype: torch.dtype) -> torch.Tensor:
        """``code[nibble] * scale`` in fp32, cast to ``dtype`` (streaming/nf4.py:29-35)."""
        if self.packed.device.type != "cuda":
            raise CapabilityError("NF4 dequantize requires CUDA tensors on a ROCm GPU")
        out_dtype = torch.float32 if dtype not in (torch.bfloat16, torch.float32) else dtype
        dense = ops.direct.nf4_dequantize(self.packed, self.scales, NF4_CODEBOOK.to(self.packed.device), 1,
                                   self.elements, self.block_size, NIBBLE_LOW_FIRST, out_dtype)
        return dense.reshape(self.shape).to(dtype)


@dataclass(frozen=True)
class NF4Tensor:
    """Host-resident NF4 tensor (streaming/nf4.py:38-91); quantised on the GPU."""
    packed: torch.Tensor
    scales: torch.Tensor
    shape: tuple[int, ...]
    block_size: int
    elements: int

    @classmethod
    def quantize(cls, value: torch.Tensor, *, block_size: int = 64, pin_memory: bool = False,
                 device: torch.device | str | None = None) -> "NF4Tensor":
        if value.numel() == 0 or block_size < 16 or block_size % 2:
            raise ValueError("invalid tensor or NF4 block size")
        if device is None:
            device = value.device if value.device.type == "cuda" else torch.device("cuda")
        if not torch.cuda.is_available():
            raise CapabilityError("NF4 quantization requires a ROCm GPU")
        src = value.detach().float().to(device)
        packed, scales = ops.direct.nf4_quantize(src, block_size, NIBBLE_LOW_FIRST, NF4_CODEBOOK.to(device))
        packed, scales = packed.cpu(), scales.cpu()
        if pin_memory:
            packed, scales = packed.pin_memory(), scales.pin_memory()
        return cls(packed, scales, tuple(value.shape), block_size, value.numel())

    @property
    def storage_bytes(self) -> int:
        return self.packed.numel() * self.packed.element_size() + self.scales.numel() * 4

    def dequantize(self, *, device: torch.device | str = "cuda", dtype: torch.dtype = torch.float32,
                   non_blocking: bool = False) -> torch.Tensor:
        return self.stage(torch.device(device), non_blocking=non_blocking).dequantize(dtype)

    def stage(self, device: torch.device | str, *, non_blocking: bool = False) -> NF4DevicePayload:
        target = torch.device(device)
        return NF4DevicePayload(self.packed.to(target, non_blocking=non_blocking),
                                self.scales.to(target, non_blocking=non_blocking), self.shape,
                                self.block_size, self.elements)
