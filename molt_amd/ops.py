"""torch.library custom ops over the C ABI of libmolt_amd.so.

Each op checks devices, dtypes and shapes, allocates its outputs (and any
workspace) with the PyTorch caching allocator and launches on the current
stream of the input's device. Fake (meta) implementations are registered so
the ops trace under torch.compile and pass ``torch.library.opcheck``. The
registration pattern follows the reference's own custom op
(kernels/frozen_linear_cross_entropy.py:335-392).

There is no CPU path: a CPU tensor raises CapabilityError.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

import torch
from torch import Tensor

from . import _lib
from .errors import CapabilityError

NS = "molt_amd"


def _require_gpu(*tensors: Optional[Tensor], what: str) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise CapabilityError(f"{what} requires CUDA tensors on a ROCm GPU (got {t.device})")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{what}: tensors on different devices ({dev} vs {t.device})")
    if dev is None:
        raise ValueError(f"{what}: no tensor arguments")
    return dev


def _stream(dev: torch.device) -> int:
    """Raw handle of the device's current stream (what the kernels launch on)."""
    return _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())


def _raw_stream_fallback(index: int) -> int:
    return torch.cuda.current_stream(index).cuda_stream


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", _raw_stream_fallback)

# Implementations of the registered ops, by name. The autograd nodes of the
# hot path call them through ``direct`` in eager mode: the dispatcher costs
# about 13 us per call on the host, more than the GPU time of the small
# projections. Under torch.compile ``direct`` returns the registered op.
_RAW: dict = {}


def _custom_op(qualname: str, mutates_args=()):
    def deco(fn):
        _RAW[qualname.split("::", 1)[1]] = fn
        return torch.library.custom_op(qualname, mutates_args=mutates_args)(fn)
    return deco


def _plain(args) -> bool:
    """True when every tensor argument is an ordinary tensor (not a fake,
    functional or other subclass tensor of a tracing pass)."""
    for a in args:
        if isinstance(a, Tensor) and type(a) is not Tensor and type(a) is not torch.nn.Parameter:
            return False
    return True


class _Direct:
    def __getattr__(self, name: str):
        raw, op = _RAW.get(name) or _late_raw(name), globals()[name]

        def call(*args, **kwargs):
            if torch.compiler.is_compiling() or not _plain(args):
                return op(*args, **kwargs)
            return raw(*args, **kwargs)

        call.__name__ = name
        setattr(self, name, call)
        return call


def _late_raw(name: str):
    raise AttributeError(f"molt_amd.ops has no registered op {name!r}")


direct = _Direct()


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _bf16(t: Tensor, name: str, what: str) -> Tensor:
    if t.dtype != torch.bfloat16:
        raise CapabilityError(f"{what} requires BF16 {name} (got {t.dtype})")
    return t.contiguous()


def _bf16_rows(t: Tensor, name: str, what: str) -> Tensor:
    """A BF16 matrix whose rows may be strided (a column slice of a wider
    matrix): passed as is with its row stride when the elements of a row are
    contiguous, else made contiguous."""
    if t.dtype != torch.bfloat16:
        raise CapabilityError(f"{what} requires BF16 {name} (got {t.dtype})")
    if t.dim() == 2 and t.stride(1) == 1 and t.stride(0) >= t.shape[1]:
        return t
    return t.contiguous()


def _f32(t: Tensor) -> Tensor:
    if t.dtype == torch.float32 and t.is_contiguous():
        return t           # only its address is passed on
    return t.detach().to(torch.float32).contiguous()


# Workspace sizes by (query, arguments, tuning generation): a host lookup
# instead of a library call per launch. The sizes follow the kernel choice,
# which only the tuning settings change; a size gone stale through a change
# made outside ``_lib.tuning`` only makes the GEMMs run unsplit.
_WS: dict = {}


def _workspace(query: str, *args: int) -> int:
    key = (query, args, _lib.tuning_generation)
    n = _WS.get(key)
    if n is None:
        if len(_WS) > 4096:
            _WS.clear()
        n = _WS[key] = int(getattr(_lib.load(), query)(*args))
    return n


# Weight descriptors by content: the pointers and geometry they hold. A hit
# describes the very memory of the tensors passed in, so the cache holds no
# references to them. Callers bind every tensor they pass (including fp32 or
# contiguous copies made for the call) to a local that lives until the launch
# has been enqueued: a temporary freed earlier could be handed to a workspace
# or output allocated before the launch and overwritten by a staging kernel
# ahead of the GEMM that reads it.
_DESC: dict = {}


def _weight(packed: Tensor, scales: Optional[Tensor], code: Tensor, rows: int, cols: int,
            block_size: int, order: int, absmax_q: Optional[Tensor] = None,
            absmax2: Optional[Tensor] = None, code2: Optional[Tensor] = None,
            offset: float = 0.0, dq_block: int = 256) -> _lib.NF4Weight:
    key = (packed.data_ptr(), _ptr(scales), code.data_ptr(), _ptr(absmax_q), _ptr(absmax2), _ptr(code2),
           float(offset), int(block_size), int(dq_block), int(order), int(rows), int(cols))
    w = _DESC.get(key)
    if w is None:
        if len(_DESC) > 4096:
            _DESC.clear()
        w = _DESC[key] = _descriptor(packed, scales, code, rows, cols, block_size, order, absmax_q, absmax2,
                                     code2, offset, dq_block)
    return w


def _descriptor(packed, scales, code, rows, cols, block_size, order, absmax_q, absmax2, code2, offset,
                dq_block) -> _lib.NF4Weight:
    w = _lib.NF4Weight()
    w.packed = packed.data_ptr()
    w.scales = _ptr(scales)
    w.absmax_q = _ptr(absmax_q)
    w.absmax2 = _ptr(absmax2)
    w.code2 = _ptr(code2)
    w.code = code.data_ptr()
    w.offset = float(offset)
    w.nested = int(absmax_q is not None)
    w.block_size = int(block_size)
    w.dq_block = int(dq_block)
    w.nibble_order = int(order)
    w.rows = int(rows)
    w.cols = int(cols)
    return w


def _check_packed(packed: Tensor, rows: int, cols: int, what: str) -> Tensor:
    if packed.dtype != torch.uint8:
        raise CapabilityError(f"{what} requires uint8 packed NF4 weights")
    if packed.numel() * 2 < rows * cols:
        raise ValueError(f"{what}: packed weight holds {packed.numel()} bytes, "
                         f"{(rows * cols + 1) // 2} needed for {rows}x{cols}")
    return packed.contiguous()


def _check_stats(what: str, rows: int, cols: int, block_size: int, code: Tensor,
                 scales: Optional[Tensor] = None, absmax_q: Optional[Tensor] = None,
                 absmax2: Optional[Tensor] = None, code2: Optional[Tensor] = None,
                 dq_block: int = 256) -> None:
    """Every block statistic the kernels read must exist: one scale (or one
    nested code) per ``block_size`` elements of the flattened weight, one
    absmax2 per ``dq_block`` codes, 16 NF4 levels and 256 nested levels."""
    if block_size <= 0 or (absmax_q is not None and dq_block <= 0):
        raise ValueError(f"{what}: block sizes must be positive")
    nblocks = -(-rows * cols // block_size)
    if code.numel() < 16:
        raise ValueError(f"{what}: the NF4 code table needs 16 entries, got {code.numel()}")
    if absmax_q is None:
        if scales is None or scales.numel() < nblocks:
            have = 0 if scales is None else scales.numel()
            raise ValueError(f"{what}: {have} block scales for {nblocks} blocks of {rows}x{cols}")
        return
    if absmax_q.dtype != torch.uint8 or absmax_q.numel() < nblocks:
        raise ValueError(f"{what}: nested absmax must be uint8 with {nblocks} entries "
                         f"(got {absmax_q.dtype}, {absmax_q.numel()})")
    if absmax2 is None or absmax2.numel() < -(-nblocks // dq_block):
        raise ValueError(f"{what}: {0 if absmax2 is None else absmax2.numel()} second-level absmax "
                         f"values for {-(-nblocks // dq_block)} blocks")
    if code2 is None or code2.numel() < 256:
        raise ValueError(f"{what}: the nested code table needs 256 entries")


def _check_rows(what: str, name: str, t: Optional[Tensor], rows: int) -> None:
    if t is not None and (t.dim() != 2 or t.shape[0] != rows):
        raise ValueError(f"{what}: {name} must have {rows} rows, got {tuple(t.shape)}")


# Optional per-launch event probe: name -> list of (start, end) torch.cuda.Event
# pairs recorded on the launch stream around each call of that entry point.
_probes: dict[str, list] = {}
# Event pairs made ahead of the calls they will time (GEMM entry points only).
_probe_pool: dict[str, list] = {}


def probe_events(name: str, enable: bool = True, reserve: int = 0) -> list:
    """Start (or stop) recording HIP events around every call of the C entry
    point ``name``; returns the list that collects (start, end) pairs. For the
    NF4 GEMM entry points the library records them around the GEMM kernel
    itself (``molt_amd_time_next_gemm``), leaving out weight staging and
    split-K sums. ``reserve`` makes that many event pairs now (each recorded
    once, which is what creates a HIP event), so that the first ``reserve``
    GEMM calls put only the library's two timing markers in the stream
    instead of four (each marker leaves the GPU idle for a few µs)."""
    if enable:
        if reserve and name in _GEMM_ENTRIES:
            pool = _probe_pool.setdefault(name, [])
            for _ in range(reserve):
                pair = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                pair[0].record()
                pair[1].record()
                pool.append(pair)
        return _probes.setdefault(name, [])
    _probe_pool.pop(name, None)
    return _probes.pop(name, [])


_FNS: dict = {}


def _call(fn_name: str, *args) -> None:
    fn = _FNS.get(fn_name)
    if fn is None:
        fn = _FNS[fn_name] = getattr(_lib.load(), fn_name)
    key = _PROBE_AS.get(fn_name, fn_name)
    pairs = _probes.get(key) if _probes else None
    if pairs is None:
        rc = fn(*args)
        if rc:
            _lib.check(rc)
        return
    lib = _lib.load()
    pool = _probe_pool.get(key)
    if pool:
        start, end = pool.pop()
    else:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        if key in _GEMM_ENTRIES:
            end.record()   # creates the event; the library records both again around the kernel
    if key in _GEMM_ENTRIES:
        _lib.check(lib.molt_amd_time_next_gemm(C.c_void_p(start.cuda_event), C.c_void_p(end.cuda_event)))
    _lib.check(getattr(lib, fn_name)(*args))
    if key not in _GEMM_ENTRIES:
        end.record()
    pairs.append((start, end))


_GEMM_ENTRIES = frozenset(("molt_nf4_lora_forward", "molt_nf4_gateup_forward", "molt_nf4_lora_backward_input",
                           "molt_nf4_lora_backward_input_pair", "molt_nf4_swiglu_backward"))
# the variants that hand the staged weights over run the same GEMM kernels:
# probes of a GEMM entry point also time them
_PROBE_AS = {"molt_nf4_lora_forward_keep_wt": "molt_nf4_lora_forward",
             "molt_nf4_gateup_forward_keep_wt": "molt_nf4_gateup_forward",
             "molt_nf4_lora_backward_input_wt": "molt_nf4_lora_backward_input",
             "molt_nf4_lora_backward_input_pair_wt": "molt_nf4_lora_backward_input_pair",
             "molt_nf4_swiglu_backward_wt": "molt_nf4_swiglu_backward"}


# ----------------------------------------------------------------- codec
@_custom_op(f"{NS}::nf4_dequantize", mutates_args=())
def nf4_dequantize(packed: Tensor, scales: Tensor, code: Tensor, rows: int, cols: int,
                   block_size: int, order: int, out_dtype: torch.dtype) -> Tensor:
    """bf16/fp32 decode with resolved fp32 scales (streaming/nf4.py:29-35)."""
    what = "NF4 dequantize"
    dev = _require_gpu(packed, scales, code, what=what)
    packed = _check_packed(packed, rows, cols, what)
    _check_stats(what, rows, cols, block_size, code, scales=scales)
    out = torch.empty((rows, cols), device=dev, dtype=out_dtype)
    sc, cd = _f32(scales), _f32(code)
    w = _weight(packed, sc, cd, rows, cols, block_size, order)
    dt = _lib.DTYPE_F32 if out_dtype == torch.float32 else _lib.DTYPE_BF16
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise CapabilityError(f"{what}: output dtype {out_dtype} unsupported (bf16, fp32)")
    _call("molt_nf4_dequantize", C.byref(w), out.data_ptr(), dt, _stream(dev))
    return out


@nf4_dequantize.register_fake
def _(packed, scales, code, rows, cols, block_size, order, out_dtype):
    return packed.new_empty((rows, cols), dtype=out_dtype)


@_custom_op(f"{NS}::nf4_dequantize_nested", mutates_args=())
def nf4_dequantize_nested(packed: Tensor, absmax_q: Tensor, absmax2: Tensor, code2: Tensor,
                          code: Tensor, offset: float, rows: int, cols: int, block_size: int,
                          dq_block: int, order: int, out_dtype: torch.dtype) -> Tensor:
    """bitsandbytes.functional.dequantize_4bit with nested absmax
    (methods/nf4_lora.py:97-98)."""
    what = "NF4 dequantize"
    dev = _require_gpu(packed, absmax_q, absmax2, code2, code, what=what)
    packed = _check_packed(packed, rows, cols, what)
    _check_stats(what, rows, cols, block_size, code, absmax_q=absmax_q, absmax2=absmax2, code2=code2,
                 dq_block=dq_block)
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise CapabilityError(f"{what}: output dtype {out_dtype} unsupported (bf16, fp32)")
    out = torch.empty((rows, cols), device=dev, dtype=out_dtype)
    cd, q, a2, c2 = _f32(code), absmax_q.contiguous(), _f32(absmax2), _f32(code2)
    w = _weight(packed, None, cd, rows, cols, block_size, order, q, a2, c2, offset, dq_block)
    dt = _lib.DTYPE_F32 if out_dtype == torch.float32 else _lib.DTYPE_BF16
    _call("molt_nf4_dequantize", C.byref(w), out.data_ptr(), dt, _stream(dev))
    return out


@nf4_dequantize_nested.register_fake
def _(packed, absmax_q, absmax2, code2, code, offset, rows, cols, block_size, dq_block, order, out_dtype):
    return packed.new_empty((rows, cols), dtype=out_dtype)


@_custom_op(f"{NS}::nf4_resolve_scales", mutates_args=())
def nf4_resolve_scales(absmax_q: Tensor, absmax2: Tensor, code2: Tensor, offset: float,
                       dq_block: int) -> Tensor:
    """fp32 block scales from nested statistics (methods/nf4_backward.py:145-164)."""
    dev = _require_gpu(absmax_q, absmax2, code2, what="NF4 scale resolution")
    _check_stats("NF4 scale resolution", 1, absmax_q.numel(), 1, torch.empty(16, device="meta"),
                 absmax_q=absmax_q, absmax2=absmax2, code2=code2, dq_block=dq_block)
    q = absmax_q.contiguous()
    out = torch.empty(q.numel(), device=dev, dtype=torch.float32)
    # rows*cols only matter through ceil(n / block_size); describe n = nblocks with block 1
    dummy_packed, dummy_code = torch.empty(1, dtype=torch.uint8, device=dev), torch.empty(16, device=dev)
    a2, c2 = _f32(absmax2), _f32(code2)
    w = _weight(dummy_packed, None, dummy_code, 1, q.numel(), 1, 1, q, a2, c2, offset, dq_block)
    _call("molt_nf4_resolve_scales", C.byref(w), out.data_ptr(), _stream(dev))
    return out


@nf4_resolve_scales.register_fake
def _(absmax_q, absmax2, code2, offset, dq_block):
    return absmax_q.new_empty(absmax_q.numel(), dtype=torch.float32)


@_custom_op(f"{NS}::nf4_quantize", mutates_args=())
def nf4_quantize(x: Tensor, block_size: int, order: int, code: Tensor) -> tuple[Tensor, Tensor]:
    """Blockwise NF4 codes + fp32 absmax (streaming/nf4.py:46-68)."""
    what = "NF4 quantize"
    dev = _require_gpu(x, code, what=what)
    if x.numel() == 0 or block_size < 16 or block_size % 2:
        raise ValueError("invalid tensor or NF4 block size")
    if code.numel() < 16:
        raise ValueError(f"{what}: the NF4 code table needs 16 entries, got {code.numel()}")
    if x.dtype == torch.bfloat16:
        src, dt = x.contiguous(), _lib.DTYPE_BF16
    else:
        src, dt = x.detach().to(torch.float32).contiguous(), _lib.DTYPE_F32
    n = src.numel()
    nblocks = -(-n // block_size)
    packed = torch.empty(nblocks * block_size // 2, device=dev, dtype=torch.uint8)
    absmax = torch.empty(nblocks, device=dev, dtype=torch.float32)
    _call("molt_nf4_quantize", src.data_ptr(), dt, n, block_size, order, _f32(code).data_ptr(),
          packed.data_ptr(), absmax.data_ptr(), _stream(dev))
    return packed, absmax


@nf4_quantize.register_fake
def _(x, block_size, order, code):
    nblocks = -(-x.numel() // block_size)
    return (x.new_empty(nblocks * block_size // 2, dtype=torch.uint8),
            x.new_empty(nblocks, dtype=torch.float32))


@_custom_op(f"{NS}::nf4_double_quantize", mutates_args=())
def nf4_double_quantize(absmax: Tensor, code2: Tensor, dq_block: int) -> tuple[Tensor, Tensor, Tensor]:
    """Nested statistics (bitsandbytes compress_statistics=True)."""
    dev = _require_gpu(absmax, code2, what="NF4 double quantize")
    if code2.numel() < 256 or dq_block <= 0:
        raise ValueError("NF4 double quantize: needs a 256-entry code table and a positive block size")
    a = _f32(absmax)
    n = a.numel()
    q = torch.empty(n, device=dev, dtype=torch.uint8)
    absmax2 = torch.empty(-(-n // dq_block), device=dev, dtype=torch.float32)
    offset = torch.empty((), device=dev, dtype=torch.float32)
    lib = _lib.load()
    ws_bytes = int(lib.molt_nf4_double_quantize_workspace(n))
    ws = torch.empty(max(ws_bytes, 8), device=dev, dtype=torch.uint8)
    _call("molt_nf4_double_quantize", a.data_ptr(), n, dq_block, _f32(code2).data_ptr(), q.data_ptr(),
          absmax2.data_ptr(), offset.data_ptr(), ws.data_ptr(), ws_bytes, _stream(dev))
    return q, absmax2, offset


@nf4_double_quantize.register_fake
def _(absmax, code2, dq_block):
    n = absmax.numel()
    return (absmax.new_empty(n, dtype=torch.uint8), absmax.new_empty(-(-n // dq_block)),
            absmax.new_empty(()))


# ------------------------------------------------------------ NF4 + LoRA
@_custom_op(f"{NS}::lora_project", mutates_args=())
def lora_project(z: Tensor, z2: Optional[Tensor], mode: int, zscale: float, lora: Tensor,
                 layout: int) -> Tensor:
    """out[M, r] = bf16(z . bf16(lora)^T) (methods/nf4_lora.py:49,86-90)."""
    what = "LoRA projection"
    dev = _require_gpu(z, z2, lora, what=what)
    z = _bf16(z, "activations", what)
    z2 = None if z2 is None else _bf16(z2, "activations", what)
    if z.dim() != 2 or (z2 is not None and z2.shape != z.shape):
        raise ValueError(f"{what}: expected a 2-D activation (and a second operand of the same shape)")
    m, d = z.shape
    lw = _f32(lora)
    r = lw.shape[0] if layout == 0 else lw.shape[1]
    if (lw.shape[1] if layout == 0 else lw.shape[0]) != d:
        raise ValueError(f"{what}: adapter width {tuple(lw.shape)} does not match activation width {d}")
    out = torch.empty((m, r), device=dev, dtype=torch.bfloat16)
    ws_bytes = _workspace("molt_lora_project_workspace", m, d, r)
    ws = torch.empty(max(ws_bytes, 16), device=dev, dtype=torch.uint8)
    _call("molt_lora_project", z.data_ptr(), _ptr(z2), d, mode, zscale, m, d, lw.data_ptr(), layout, r,
          out.data_ptr(), r, ws.data_ptr(), ws_bytes, _stream(dev))
    return out


@lora_project.register_fake
def _(z, z2, mode, zscale, lora, layout):
    r = lora.shape[0] if layout == 0 else lora.shape[1]
    return z.new_empty((z.shape[0], r), dtype=torch.bfloat16)


@_custom_op(f"{NS}::lora_project_pair", mutates_args=())
def lora_project_pair(z0: Tensor, z1: Tensor, zscale0: float, zscale1: float, lora0: Tensor,
                      lora1: Tensor) -> Tensor:
    """[bf16(bf16(s0 z0) . bf16(B0)) | bf16(bf16(s1 z1) . bf16(B1))], [M, 2 r]: the
    gate and up U of the gated MLP's backward (methods/nf4_lora.py:87-90, mode
    2, adapters [D, r]) written as the two column halves of one matrix, so that
    the gate/up input gradient and the shared dA pass read them in place."""
    what = "LoRA projection pair"
    dev = _require_gpu(z0, z1, lora0, lora1, what=what)
    z0 = _bf16(z0, "activations", what)
    z1 = _bf16(z1, "activations", what)
    if z0.dim() != 2 or z1.shape != z0.shape:
        raise ValueError(f"{what}: expected two 2-D activations of one shape")
    m, d = z0.shape
    l0, l1 = _f32(lora0), _f32(lora1)
    if l0.dim() != 2 or l0.shape[0] != d or l1.shape != l0.shape:
        raise ValueError(f"{what}: adapters {tuple(l0.shape)}, {tuple(l1.shape)} must both be [{d}, r]")
    # both adapters packed in one launch, then one projection launch for the pair
    # (bitwise lora_project_pair_packed)
    packs = direct.lora_pack_many([l0, l1], [None, None], [1, 1])
    return direct.lora_project_pair_packed(z0, z1, zscale0, zscale1, packs[0], packs[1], l0.shape[1])


@lora_project_pair.register_fake
def _(z0, z1, zscale0, zscale1, lora0, lora1):
    return z0.new_empty((z0.shape[0], 2 * lora0.shape[1]), dtype=torch.bfloat16)


@_custom_op(f"{NS}::lora_pack_many", mutates_args=())
def lora_pack_many(loras: list[Tensor], loras2: list[Optional[Tensor]], layouts: list[int]) -> list[Tensor]:
    """The projection's bf16 fragment-order operands of 1..8 fp32 adapters in
    one launch (molt_lora_pack_many), as uint8 tensors for
    ``lora_project_packed``. ``loras2[i]`` (or None) is stacked after
    ``loras[i]`` (rows for layout 0 = A [r, D], columns for layout 1 = B
    [D, r]), so [A_gate; A_up] needs no copy."""
    what = "LoRA pack"
    n = len(loras)
    if not (1 <= n <= 8) or len(loras2) != n or len(layouts) != n:
        raise ValueError(f"{what}: 1..8 adapters with one entry per argument list")
    dev = _require_gpu(*loras, *[t for t in loras2 if t is not None], what=what)
    descs = (_lib.LoraPackDesc * n)()
    keep, outs = [], []
    lib = _lib.load()
    for i in range(n):
        a = _f32(loras[i])
        b = None if loras2[i] is None else _f32(loras2[i])
        lay = int(layouts[i])
        if a.dim() != 2 or (b is not None and (b.dim() != 2 or (b.shape[1] if lay == 0 else b.shape[0]) !=
                                               (a.shape[1] if lay == 0 else a.shape[0]))):
            raise ValueError(f"{what}: adapters {tuple(a.shape)} and {None if b is None else tuple(b.shape)} "
                             f"do not stack in layout {lay}")
        d = a.shape[1] if lay == 0 else a.shape[0]
        split = a.shape[0] if lay == 0 else a.shape[1]
        r = split + (0 if b is None else (b.shape[0] if lay == 0 else b.shape[1]))
        out = torch.empty(int(lib.molt_lora_packed_bytes(d, r)), device=dev, dtype=torch.uint8)
        keep += [a, b]
        outs.append(out)
        descs[i] = _lib.LoraPackDesc(a.data_ptr(), _ptr(b), split, lay, r, d, out.data_ptr())
    _call("molt_lora_pack_many", n, descs, _stream(dev))
    del keep
    return outs


@lora_pack_many.register_fake
def _(loras, loras2, layouts):
    lib = _lib.load()
    outs = []
    for a, b, lay in zip(loras, loras2, layouts):
        d = a.shape[1] if lay == 0 else a.shape[0]
        r = (a.shape[0] if lay == 0 else a.shape[1]) + (0 if b is None else (b.shape[0] if lay == 0 else b.shape[1]))
        outs.append(a.new_empty((int(lib.molt_lora_packed_bytes(d, r)),), dtype=torch.uint8))
    return outs


@_custom_op(f"{NS}::lora_project_packed", mutates_args=())
def lora_project_packed(z: Tensor, z2: Optional[Tensor], mode: int, zscale: float, packed: Tensor,
                        r: int) -> Tensor:
    """``lora_project`` over an adapter packed by ``lora_pack_many`` (rank r,
    width z.shape[1]): no pack launch; bitwise the same output."""
    what = "LoRA projection"
    dev = _require_gpu(z, z2, packed, what=what)
    z = _bf16(z, "activations", what)
    z2 = None if z2 is None else _bf16(z2, "activations", what)
    if z.dim() != 2 or (z2 is not None and z2.shape != z.shape):
        raise ValueError(f"{what}: expected a 2-D activation (and a second operand of the same shape)")
    m, d = z.shape
    if packed.dtype != torch.uint8 or packed.numel() != int(_lib.load().molt_lora_packed_bytes(d, r)):
        raise ValueError(f"{what}: the packed adapter does not match width {d} and rank {r}")
    out = torch.empty((m, r), device=dev, dtype=torch.bfloat16)
    ws_bytes = _workspace("molt_lora_project_packed_workspace", m, d, r)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
    _call("molt_lora_project_packed", z.data_ptr(), _ptr(z2), d, mode, zscale, m, d, packed.data_ptr(), r,
          out.data_ptr(), r, _ptr(ws), ws_bytes, _stream(dev))
    return out


@lora_project_packed.register_fake
def _(z, z2, mode, zscale, packed, r):
    return z.new_empty((z.shape[0], r), dtype=torch.bfloat16)


@_custom_op(f"{NS}::lora_project_pair_packed", mutates_args=())
def lora_project_pair_packed(z0: Tensor, z1: Tensor, zscale0: float, zscale1: float, packed0: Tensor,
                             packed1: Tensor, r: int) -> Tensor:
    """``lora_project_pair`` over adapters packed by ``lora_pack_many`` (layout
    1, rank r each) as one launch (molt_lora_project_pair_packed): no pack
    launches, and the split over D counts both operands' row blocks. Each half
    is that operand's projection; where the pair runs with a different split
    count than a single projection, its fp32 sums run in another order."""
    what = "LoRA projection pair"
    dev = _require_gpu(z0, z1, packed0, packed1, what=what)
    z0 = _bf16(z0, "activations", what)
    z1 = _bf16(z1, "activations", what)
    if z0.dim() != 2 or z1.shape != z0.shape:
        raise ValueError(f"{what}: expected two 2-D activations of one shape")
    m, d = z0.shape
    nbytes = int(_lib.load().molt_lora_packed_bytes(d, r))
    if packed0.numel() != nbytes or packed1.numel() != nbytes:
        raise ValueError(f"{what}: the packed adapters do not match width {d} and rank {r}")
    out = torch.empty((m, 2 * r), device=dev, dtype=torch.bfloat16)
    ws_bytes = _workspace("molt_lora_project_pair_packed_workspace", m, d, r)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
    _call("molt_lora_project_pair_packed", z0.data_ptr(), z1.data_ptr(), d, 2, zscale0, zscale1, m, d,
          packed0.data_ptr(), packed1.data_ptr(), r, out.data_ptr(), 2 * r, _ptr(ws), ws_bytes, _stream(dev))
    return out


@lora_project_pair_packed.register_fake
def _(z0, z1, zscale0, zscale1, packed0, packed1, r):
    return z0.new_empty((z0.shape[0], 2 * r), dtype=torch.bfloat16)


_KEEP_WT = [os.environ.get("MOLT_KEEP_WEIGHT_TRANSPOSES", "1") != "0"]


def keep_weight_transposes(enabled: Optional[bool] = None) -> bool:
    """Policy of the fused gated MLP for large token batches: its forward GEMMs
    leave the bf16 transposed weights (N * K * 2 bytes per weight, held until
    the backward of the same call) for the input gradients, which then skip
    their own dequantise-and-transpose pass. On by default; the environment
    variable MOLT_KEEP_WEIGHT_TRANSPOSES=0 or ``keep_weight_transposes(False)``
    trades that time back for the memory. Returns the setting in force (after
    the change, if ``enabled`` is given)."""
    if enabled is not None:
        _KEEP_WT[0] = bool(enabled)
    return _KEEP_WT[0]


def _keeps_wt(m: int, rows: int, cols: int, weights: int) -> bool:
    """Whether a forward over m rows would hand deq(W)^T to the input gradient
    (molt_nf4_keeps_wt): both GEMMs stage the weights."""
    return bool(_workspace("molt_nf4_keeps_wt", m, rows, cols, weights))


def _empty_wt(dev) -> Tensor:
    return torch.empty(0, device=dev, dtype=torch.bfloat16)


@_custom_op(f"{NS}::nf4_lora_forward", mutates_args=())
def nf4_lora_forward(x: Tensor, packed: Tensor, scales: Tensor, code: Tensor, rows: int, cols: int,
                     order: int, block_size: int, t: Optional[Tensor], lora_b: Optional[Tensor],
                     scaling: float) -> Tensor:
    """Y = X deq(W)^T + T bf16(s B)^T (methods/nf4_lora.py:43-50)."""
    return _lora_forward(x, packed, scales, code, rows, cols, order, block_size, t, lora_b, scaling, False)[0]


@_custom_op(f"{NS}::nf4_lora_forward_keep_wt", mutates_args=())
def nf4_lora_forward_keep_wt(x: Tensor, packed: Tensor, scales: Tensor, code: Tensor, rows: int, cols: int,
                             order: int, block_size: int, t: Optional[Tensor], lora_b: Optional[Tensor],
                             scaling: float) -> tuple[Tensor, Tensor]:
    """(Y, deq(W)^T): nf4_lora_forward that also leaves the bf16 transposed
    weight [cols, rows] for the input gradient of the same weight
    (nf4_lora_backward_input(..., wt=)) when both GEMMs stage the weight, else
    an empty tensor in its place."""
    y, wt = _lora_forward(x, packed, scales, code, rows, cols, order, block_size, t, lora_b, scaling, True)
    return y, wt


def _lora_forward(x, packed, scales, code, rows, cols, order, block_size, t, lora_b, scaling, keep):
    what = "NF4-LoRA forward"
    dev = _require_gpu(x, packed, scales, code, t, lora_b, what=what)
    x = _bf16(x, "activations", what)
    if x.dim() != 2 or x.shape[1] != cols:
        raise ValueError(f"{what}: input width {tuple(x.shape)} does not match in_features {cols}")
    packed = _check_packed(packed, rows, cols, what)
    _check_stats(what, rows, cols, block_size, code, scales=scales)
    y = torch.empty((x.shape[0], rows), device=dev, dtype=torch.bfloat16)
    sc, cd = _f32(scales), _f32(code)
    w = _weight(packed, sc, cd, rows, cols, block_size, order)
    r = 0
    tt = bb = None
    if t is not None:
        tt = _bf16(t, "low-rank activations", what)
        _check_rows(what, "the low-rank activation", tt, x.shape[0])
        if lora_b is None:
            raise ValueError(f"{what}: a low-rank activation needs LoRA B")
        bb = _f32(lora_b)
        r = tt.shape[1]
        if bb.shape != (rows, r):
            raise ValueError(f"{what}: LoRA B shape {tuple(bb.shape)} != ({rows}, {r})")
    ws_bytes = _workspace("molt_nf4_lora_forward_workspace", x.shape[0], rows, cols, r)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
    if keep and _keeps_wt(x.shape[0], rows, cols, 1):
        wt = torch.empty((cols, rows), device=dev, dtype=torch.bfloat16)
        written = C.c_int32(0)
        _call("molt_nf4_lora_forward_keep_wt", x.data_ptr(), cols, x.shape[0], C.byref(w), _ptr(tt), max(r, 1),
              _ptr(bb), r, float(scaling), y.data_ptr(), rows, wt.data_ptr(), C.byref(written), _ptr(ws),
              ws_bytes, _stream(dev))
        return y, (wt if written.value else _empty_wt(dev))
    _call("molt_nf4_lora_forward", x.data_ptr(), cols, x.shape[0], C.byref(w), _ptr(tt), max(r, 1),
          _ptr(bb), r, float(scaling), y.data_ptr(), rows, _ptr(ws), ws_bytes, _stream(dev))
    return y, (_empty_wt(dev) if keep else None)


@nf4_lora_forward.register_fake
def _(x, packed, scales, code, rows, cols, order, block_size, t, lora_b, scaling):
    return x.new_empty((x.shape[0], rows), dtype=torch.bfloat16)


@nf4_lora_forward_keep_wt.register_fake
def _(x, packed, scales, code, rows, cols, order, block_size, t, lora_b, scaling):
    keep = _keeps_wt(x.shape[0], rows, cols, 1)
    return (x.new_empty((x.shape[0], rows), dtype=torch.bfloat16),
            x.new_empty((cols, rows) if keep else (0,), dtype=torch.bfloat16))


# ----------------------------------------------------------- stacked weights
def stack_adapters(loras_a: list[Tensor], loras_b: list[Tensor], lr: int) -> tuple[Tensor, Tensor]:
    """(A_stack fp32 [lr, K], B_blocks fp32 [N, lr]) for projections that
    share one input (molt_lora_stack_adapters): A_stack = [A_0; A_1; ..; zero
    rows], B_blocks block-diagonal with B_i [rows_i, r] in columns i r ..
    i r + r - 1 of its rows. One launch."""
    what = "adapter stack"
    n = len(loras_a)
    if not (1 <= n <= 8) or len(loras_b) != n:
        raise ValueError(f"{what}: 1..8 adapter pairs")
    dev = _require_gpu(*loras_a, *loras_b, what=what)
    a = [_f32(t) for t in loras_a]
    b = [_f32(t) for t in loras_b]
    r, k = a[0].shape
    for ai, bi in zip(a, b):
        if ai.shape != (r, k) or bi.dim() != 2 or bi.shape[1] != r:
            raise ValueError(f"{what}: adapters of one rank and width expected, got A {tuple(ai.shape)}, "
                             f"B {tuple(bi.shape)}")
    rows = [int(bi.shape[0]) for bi in b]
    a_stack = torch.empty((lr, k), device=dev, dtype=torch.float32)
    b_blocks = torch.empty((sum(rows), lr), device=dev, dtype=torch.float32)
    pa = (C.c_void_p * n)(*[t.data_ptr() for t in a])
    pb = (C.c_void_p * n)(*[t.data_ptr() for t in b])
    pr = (C.c_int64 * n)(*rows)
    _call("molt_lora_stack_adapters", n, pa, pb, pr, r, k, lr, a_stack.data_ptr(), b_blocks.data_ptr(),
          _stream(dev))
    del a, b
    return a_stack, b_blocks


def _stacked_weights(weights: list[tuple[Tensor, Tensor, int]], code: Tensor, cols: int, order: int,
                     block_size: int, what: str):
    """ctypes array of the stacked weights' descriptors (packed, resolved
    scales, rows each), and their total rows."""
    n = len(weights)
    if not (1 <= n <= 8):
        raise ValueError(f"{what}: 1..8 weights")
    descs = (_lib.NF4Weight * n)()
    keep = []
    cd = _f32(code)
    for i, (packed, scales, rows) in enumerate(weights):
        packed = _check_packed(packed, rows, cols, what)
        _check_stats(what, rows, cols, block_size, code, scales=scales)
        sc = _f32(scales)
        keep += [packed, sc]
        descs[i] = _weight(packed, sc, cd, rows, cols, block_size, order)
    keep.append(cd)
    return descs, sum(int(w[2]) for w in weights), keep


def nf4_stacked_forward(x: Tensor, weights: list[tuple[Tensor, Tensor, int]], code: Tensor, cols: int,
                        order: int, block_size: int, t: Optional[Tensor], b_blocks: Optional[Tensor],
                        scaling: float, keep_wt: bool) -> tuple[Tensor, Optional[Tensor]]:
    """(Y [M, N], deq(W)^T [cols, N] or None) over the weights stacked along
    their output rows, W = [W_0; W_1; ..] (molt_nf4_stacked_forward): one GEMM
    for projections that share X. T [M, lr] = X A_stack^T and B_blocks [N, lr]
    from ``stack_adapters`` (lr a multiple of 64), or None for no LoRA. Raises
    CapabilityError for a batch the staged GEMM does not take."""
    what = "stacked NF4-LoRA forward"
    dev = _require_gpu(x, code, t, b_blocks, *[w[0] for w in weights], what=what)
    x = _bf16(x, "activations", what)
    if x.dim() != 2 or x.shape[1] != cols:
        raise ValueError(f"{what}: input width {tuple(x.shape)} does not match in_features {cols}")
    descs, n, keep = _stacked_weights(weights, code, cols, order, block_size, what)
    m = x.shape[0]
    lr = 0
    if t is not None:
        t = _bf16(t, "low-rank activations", what)
        lr = t.shape[1]
        if t.shape[0] != m or b_blocks is None or tuple(b_blocks.shape) != (n, lr):
            raise ValueError(f"{what}: T {tuple(t.shape)} and B_blocks "
                             f"{None if b_blocks is None else tuple(b_blocks.shape)} do not match ({m}, {n})")
        b_blocks = _f32(b_blocks)
    y = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
    ws_bytes = _workspace("molt_nf4_lora_forward_workspace", m, n, cols, lr)
    ws = torch.empty(max(ws_bytes, 256), device=dev, dtype=torch.uint8)
    wt = torch.empty((cols, n), device=dev, dtype=torch.bfloat16) if keep_wt else None
    written = C.c_int32(0)
    lib = _lib.load()
    rc = lib.molt_nf4_stacked_forward(x.data_ptr(), cols, m, len(weights), descs, _ptr(t), max(lr, 1), lr,
                                      _ptr(b_blocks), max(lr, 1), float(scaling), y.data_ptr(), n, _ptr(wt),
                                      C.byref(written), ws.data_ptr(), ws_bytes, _stream(dev))
    _lib.check(rc)     # a batch the staged GEMM does not take: CapabilityError
    del keep
    return y, (wt if keep_wt and written.value else None)


def nf4_stacked_backward_input(dy: Tensor, weights: list[tuple[Tensor, Tensor, int]], code: Tensor, cols: int,
                               order: int, block_size: int, wt: Tensor, u: Optional[Tensor],
                               a_stack: Optional[Tensor], lora_scale: float) -> Tensor:
    """dX = dY deq(W) + U bf16(lora_scale A_stack) for the stacked weights,
    from the deq(W)^T their forward left (molt_nf4_stacked_backward_input)."""
    what = "stacked NF4-LoRA backward"
    dev = _require_gpu(dy, wt, u, a_stack, *[w[0] for w in weights], what=what)
    dy = _bf16(dy, "gradients", what)
    descs, n, keep = _stacked_weights(weights, code, cols, order, block_size, what)
    if dy.dim() != 2 or dy.shape[1] != n:
        raise ValueError(f"{what}: gradient width {tuple(dy.shape)} does not match the stacked outputs {n}")
    if wt is None or wt.dtype != torch.bfloat16 or tuple(wt.shape) != (cols, n) or not wt.is_contiguous():
        raise ValueError(f"{what}: the forward's contiguous BF16 ({cols}, {n}) transposed weight is required")
    m = dy.shape[0]
    r = 0
    if u is not None:
        u = _bf16(u, "LoRA gradients", what)
        r = u.shape[1]
        if u.shape[0] != m or a_stack is None or tuple(a_stack.shape) != (r, cols):
            raise ValueError(f"{what}: U {tuple(u.shape)} and A_stack do not match ({m}, {cols})")
        a_stack = _f32(a_stack)
    dx = torch.empty((m, cols), device=dev, dtype=torch.bfloat16)
    ws_bytes = _workspace("molt_nf4_lora_backward_workspace_wt", m, n, cols, 1)
    ws = torch.empty(max(ws_bytes, 256), device=dev, dtype=torch.uint8)
    lib = _lib.load()
    rc = lib.molt_nf4_stacked_backward_input(dy.data_ptr(), n, m, len(weights), descs, wt.data_ptr(), _ptr(u),
                                             max(r, 1), _ptr(a_stack), r, float(lora_scale), dx.data_ptr(), cols,
                                             ws.data_ptr(), ws_bytes, _stream(dev))
    _lib.check(rc)     # a batch the staged GEMM does not take: CapabilityError
    del keep
    return dx


@_custom_op(f"{NS}::nf4_gateup_forward", mutates_args=())
def nf4_gateup_forward(x: Tensor, packed_g: Tensor, scales_g: Tensor, packed_u: Tensor,
                       scales_u: Tensor, code: Tensor, rows: int, cols: int, order: int,
                       t: Optional[Tensor], lora_bg: Optional[Tensor], lora_bu: Optional[Tensor],
                       sg: float, su: float) -> tuple[Tensor, Tensor, Tensor]:
    """gate, up and h = bf16(bf16(silu(gate)) up) in one launch
    (methods/gated_replay.py:78-94,290-291)."""
    return _gateup_forward(x, packed_g, scales_g, packed_u, scales_u, code, rows, cols, order, t, lora_bg,
                           lora_bu, sg, su, False)[:3]


@_custom_op(f"{NS}::nf4_gateup_forward_keep_wt", mutates_args=())
def nf4_gateup_forward_keep_wt(x: Tensor, packed_g: Tensor, scales_g: Tensor, packed_u: Tensor,
                               scales_u: Tensor, code: Tensor, rows: int, cols: int, order: int,
                               t: Optional[Tensor], lora_bg: Optional[Tensor], lora_bu: Optional[Tensor],
                               sg: float, su: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(gate, up, h, deq(Wg)^T, deq(Wu)^T): nf4_gateup_forward that also
    leaves the bf16 transposed weights [cols, rows] for the paired input
    gradient (nf4_lora_backward_input_pair(..., wt0=, wt1=)) when both GEMMs
    stage the weights, else empty tensors in their place."""
    return _gateup_forward(x, packed_g, scales_g, packed_u, scales_u, code, rows, cols, order, t, lora_bg,
                           lora_bu, sg, su, True)


def _gateup_forward(x, packed_g, scales_g, packed_u, scales_u, code, rows, cols, order, t, lora_bg, lora_bu,
                    sg, su, keep):
    what = "NF4-LoRA gate/up forward"
    dev = _require_gpu(x, packed_g, scales_g, packed_u, scales_u, code, t, lora_bg, lora_bu, what=what)
    x = _bf16(x, "activations", what)
    if x.dim() != 2 or x.shape[1] != cols:
        raise ValueError(f"{what}: input width {tuple(x.shape)} does not match in_features {cols}")
    pg = _check_packed(packed_g, rows, cols, what)
    pu = _check_packed(packed_u, rows, cols, what)
    _check_stats(what, rows, cols, 64, code, scales=scales_g)
    _check_stats(what, rows, cols, 64, code, scales=scales_u)
    cd, sc_g, sc_u = _f32(code), _f32(scales_g), _f32(scales_u)
    wg = _weight(pg, sc_g, cd, rows, cols, 64, order)
    wu = _weight(pu, sc_u, cd, rows, cols, 64, order)
    m = x.shape[0]
    outs = [torch.empty((m, rows), device=dev, dtype=torch.bfloat16) for _ in range(3)]
    r = 0
    tt = bg = bu = None
    if t is not None:
        tt = _bf16(t, "low-rank activations", what)
        _check_rows(what, "the low-rank activation", tt, m)
        if lora_bg is None or lora_bu is None or tt.shape[1] % 2:
            raise ValueError(f"{what}: a low-rank activation needs [T_gate | T_up] and both LoRA B")
        r = tt.shape[1] // 2
        bg, bu = _f32(lora_bg), _f32(lora_bu)
        if bg.shape != (rows, r) or bu.shape != (rows, r):
            raise ValueError(f"{what}: LoRA B shapes {tuple(bg.shape)}, {tuple(bu.shape)} != ({rows}, {r})")
    ws_bytes = _workspace("molt_nf4_gateup_forward_workspace", m, rows, cols, r)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
    if keep and _keeps_wt(m, rows, cols, 2):
        wts = [torch.empty((cols, rows), device=dev, dtype=torch.bfloat16) for _ in range(2)]
        written = C.c_int32(0)
        _call("molt_nf4_gateup_forward_keep_wt", x.data_ptr(), cols, m, C.byref(wg), C.byref(wu), _ptr(tt),
              max(2 * r, 1), _ptr(bg), _ptr(bu), r, float(sg), float(su), outs[0].data_ptr(),
              outs[1].data_ptr(), outs[2].data_ptr(), rows, wts[0].data_ptr(), wts[1].data_ptr(),
              C.byref(written), _ptr(ws), ws_bytes, _stream(dev))
        if not written.value:
            wts = [_empty_wt(dev), _empty_wt(dev)]
        return outs[0], outs[1], outs[2], wts[0], wts[1]
    _call("molt_nf4_gateup_forward", x.data_ptr(), cols, m, C.byref(wg), C.byref(wu), _ptr(tt),
          max(2 * r, 1), _ptr(bg), _ptr(bu), r, float(sg), float(su), outs[0].data_ptr(),
          outs[1].data_ptr(), outs[2].data_ptr(), rows, _ptr(ws), ws_bytes, _stream(dev))
    if keep:
        return outs[0], outs[1], outs[2], _empty_wt(dev), _empty_wt(dev)
    return outs[0], outs[1], outs[2]


@nf4_gateup_forward.register_fake
def _(x, packed_g, scales_g, packed_u, scales_u, code, rows, cols, order, t, lora_bg, lora_bu, sg, su):
    return tuple(x.new_empty((x.shape[0], rows), dtype=torch.bfloat16) for _ in range(3))


@nf4_gateup_forward_keep_wt.register_fake
def _(x, packed_g, scales_g, packed_u, scales_u, code, rows, cols, order, t, lora_bg, lora_bu, sg, su):
    shape = (cols, rows) if _keeps_wt(x.shape[0], rows, cols, 2) else (0,)
    return tuple([x.new_empty((x.shape[0], rows), dtype=torch.bfloat16) for _ in range(3)] +
                 [x.new_empty(shape, dtype=torch.bfloat16) for _ in range(2)])


@_custom_op(f"{NS}::nf4_lora_backward_input", mutates_args=())
def nf4_lora_backward_input(dy: Tensor, packed: Tensor, scales: Tensor, code: Tensor, rows: int,
                            cols: int, order: int, block_size: int, u: Optional[Tensor],
                            lora_a: Optional[Tensor], lora_scale: float, wt: Optional[Tensor] = None) -> Tensor:
    """dX = dY deq(W) + U bf16(lora_scale A) (methods/nf4_lora.py:86-101;
    methods/nf4_backward.py:167-284). ``wt``: deq(W)^T from
    nf4_lora_forward_keep_wt of the same weight (an empty tensor or None =
    none); the result is bitwise the same."""
    what = "NF4-LoRA backward"
    dev = _require_gpu(dy, packed, scales, code, u, lora_a, what=what)
    dy = _bf16(dy, "gradients", what)
    if dy.dim() != 2 or dy.shape[1] != rows:
        raise ValueError("gradient width must match the NF4 output dimension")
    packed = _check_packed(packed, rows, cols, what)
    _check_stats(what, rows, cols, block_size, code, scales=scales)
    dx = torch.empty((dy.shape[0], cols), device=dev, dtype=torch.bfloat16)
    sc, cd = _f32(scales), _f32(code)
    w = _weight(packed, sc, cd, rows, cols, block_size, order)
    r = 0
    uu = aa = None
    if u is not None:
        uu = _bf16(u, "LoRA gradients", what)
        if lora_a is None:
            raise ValueError(f"{what}: a LoRA gradient needs LoRA A")
        aa = _f32(lora_a)
        r = uu.shape[1]
        if uu.shape[0] != dy.shape[0]:
            raise ValueError("LoRA gradient rows must match the output gradient")
        if aa.dim() != 2 or aa.shape != (r, cols):
            raise ValueError("LoRA gradient and A matrix dimensions are incompatible")
    wt = _wt_given(wt, rows, cols, what)
    if wt is not None:
        ws_bytes = _workspace("molt_nf4_lora_backward_workspace_wt", dy.shape[0], rows, cols, 1)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
        _call("molt_nf4_lora_backward_input_wt", dy.data_ptr(), rows, dy.shape[0], C.byref(w), wt.data_ptr(),
              _ptr(uu), max(r, 1), _ptr(aa), r, float(lora_scale), dx.data_ptr(), cols, _ptr(ws), ws_bytes,
              _stream(dev))
        return dx
    ws_bytes = _workspace("molt_nf4_lora_backward_workspace", dy.shape[0], rows, cols, 1)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
    _call("molt_nf4_lora_backward_input", dy.data_ptr(), rows, dy.shape[0], C.byref(w), _ptr(uu),
          max(r, 1), _ptr(aa), r, float(lora_scale), dx.data_ptr(), cols, _ptr(ws), ws_bytes, _stream(dev))
    return dx


def _wt_given(wt: Optional[Tensor], rows: int, cols: int, what: str) -> Optional[Tensor]:
    """A deq(W)^T handed over by a keep_wt forward, or None (None or empty)."""
    if wt is None or wt.numel() == 0:
        return None
    if wt.dtype != torch.bfloat16 or tuple(wt.shape) != (cols, rows) or not wt.is_contiguous():
        raise ValueError(f"{what}: the transposed weight must be contiguous BF16 ({cols}, {rows}), "
                         f"got {tuple(wt.shape)} {wt.dtype}")
    return wt


@nf4_lora_backward_input.register_fake
def _(dy, packed, scales, code, rows, cols, order, block_size, u, lora_a, lora_scale, wt=None):
    return dy.new_empty((dy.shape[0], cols), dtype=torch.bfloat16)


@_custom_op(f"{NS}::nf4_lora_backward_input_pair", mutates_args=())
def nf4_lora_backward_input_pair(dy0: Tensor, dy1: Tensor, packed0: Tensor, scales0: Tensor,
                                 packed1: Tensor, scales1: Tensor, code: Tensor, rows: int, cols: int,
                                 order: int, u0: Optional[Tensor], u1: Optional[Tensor],
                                 a0: Optional[Tensor], a1: Optional[Tensor], wt0: Optional[Tensor] = None,
                                 wt1: Optional[Tensor] = None) -> Tensor:
    """dX of the gate and up projections in one contraction
    (methods/gated_replay.py:167-186). ``wt0``/``wt1``: deq(W0)^T and
    deq(W1)^T from nf4_gateup_forward_keep_wt (empty or None = none; both or
    neither); the result is bitwise the same."""
    what = "NF4-LoRA paired backward"
    dev = _require_gpu(dy0, dy1, packed0, scales0, packed1, scales1, code, u0, u1, a0, a1, what=what)
    dy0 = _bf16(dy0, "gradients", what)
    dy1 = _bf16(dy1, "gradients", what)
    if dy0.shape != dy1.shape or dy0.dim() != 2 or dy0.shape[1] != rows:
        raise ValueError("gradient width must match the NF4 output dimension")
    p0 = _check_packed(packed0, rows, cols, what)
    p1 = _check_packed(packed1, rows, cols, what)
    _check_stats(what, rows, cols, 64, code, scales=scales0)
    _check_stats(what, rows, cols, 64, code, scales=scales1)
    cd, sc0, sc1 = _f32(code), _f32(scales0), _f32(scales1)
    w0 = _weight(p0, sc0, cd, rows, cols, 64, order)
    w1 = _weight(p1, sc1, cd, rows, cols, 64, order)
    m = dy0.shape[0]
    dx = torch.empty((m, cols), device=dev, dtype=torch.bfloat16)
    r = 0
    uu0 = uu1 = aa0 = aa1 = None
    if u0 is not None:
        if u1 is None or a0 is None or a1 is None:
            raise ValueError(f"{what}: LoRA terms need both gradients and both A matrices")
        uu0, uu1 = _bf16_rows(u0, "LoRA gradients", what), _bf16_rows(u1, "LoRA gradients", what)
        if uu0.stride(0) != uu1.stride(0):   # one row stride for both (e.g. column halves of one matrix)
            uu0, uu1 = uu0.contiguous(), uu1.contiguous()
        _check_rows(what, "the LoRA gradient", uu0, m)
        aa0, aa1 = _f32(a0), _f32(a1)
        r = uu0.shape[1]
        if uu1.shape != uu0.shape or aa0.shape != (r, cols) or aa1.shape != (r, cols):
            raise ValueError("LoRA gradient and A matrix dimensions are incompatible")
    wt0, wt1 = _wt_given(wt0, rows, cols, what), _wt_given(wt1, rows, cols, what)
    if (wt0 is None) != (wt1 is None):
        raise ValueError(f"{what}: give both transposed weights or neither")
    if wt0 is not None:
        ws_bytes = _workspace("molt_nf4_lora_backward_workspace_wt", m, rows, cols, 2)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
        _call("molt_nf4_lora_backward_input_pair_wt", dy0.data_ptr(), dy1.data_ptr(), rows, m, C.byref(w0),
              C.byref(w1), wt0.data_ptr(), wt1.data_ptr(), _ptr(uu0), _ptr(uu1),
              max(uu0.stride(0) if r else 1, 1), _ptr(aa0), _ptr(aa1), r, dx.data_ptr(), cols, _ptr(ws), ws_bytes,
              _stream(dev))
        return dx
    ws_bytes = _workspace("molt_nf4_lora_backward_workspace", m, rows, cols, 2)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
    _call("molt_nf4_lora_backward_input_pair", dy0.data_ptr(), dy1.data_ptr(), rows, m, C.byref(w0),
          C.byref(w1), _ptr(uu0), _ptr(uu1), max(uu0.stride(0) if r else 1, 1), _ptr(aa0), _ptr(aa1), r,
          dx.data_ptr(), cols,
          _ptr(ws), ws_bytes, _stream(dev))
    return dx


@nf4_lora_backward_input_pair.register_fake
def _(dy0, dy1, packed0, scales0, packed1, scales1, code, rows, cols, order, u0, u1, a0, a1, wt0=None, wt1=None):
    return dy0.new_empty((dy0.shape[0], cols), dtype=torch.bfloat16)


@_custom_op(f"{NS}::nf4_swiglu_backward", mutates_args=())
def nf4_swiglu_backward(dy: Tensor, packed: Tensor, scales: Tensor, code: Tensor, rows: int, cols: int,
                        order: int, u: Optional[Tensor], lora_a: Optional[Tensor], gate: Tensor,
                        up: Tensor, wt: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
    """(dgate, dup) from dY through the down projection and SwiGLU
    (methods/gated_replay.py:376-387); dh is never stored. ``wt``: deq(Wd)^T
    from nf4_lora_forward_keep_wt of the down weight (empty or None = none);
    the result is bitwise the same."""
    what = "NF4-LoRA SwiGLU backward"
    dev = _require_gpu(dy, packed, scales, code, u, lora_a, gate, up, what=what)
    dy = _bf16(dy, "gradients", what)
    gate = _bf16(gate, "gate", what)
    up = _bf16(up, "up", what)
    if dy.dim() != 2 or dy.shape[1] != rows:
        raise ValueError("gradient width must match the NF4 output dimension")
    if gate.shape != (dy.shape[0], cols) or up.shape != gate.shape:
        raise ValueError(f"{what}: gate/up shape must be ({dy.shape[0]}, {cols})")
    packed = _check_packed(packed, rows, cols, what)
    _check_stats(what, rows, cols, 64, code, scales=scales)
    sc, cd = _f32(scales), _f32(code)
    w = _weight(packed, sc, cd, rows, cols, 64, order)
    dg = torch.empty_like(gate)
    du = torch.empty_like(up)
    r = 0
    uu = aa = None
    if u is not None:
        if lora_a is None:
            raise ValueError(f"{what}: a LoRA gradient needs LoRA A")
        uu, aa = _bf16(u, "LoRA gradients", what), _f32(lora_a)
        _check_rows(what, "the LoRA gradient", uu, dy.shape[0])
        r = uu.shape[1]
        if aa.shape != (r, cols):
            raise ValueError("LoRA gradient and A matrix dimensions are incompatible")
    wt = _wt_given(wt, rows, cols, what)
    if wt is not None:
        ws_bytes = _workspace("molt_nf4_lora_backward_workspace_wt", dy.shape[0], rows, cols, 1)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
        _call("molt_nf4_swiglu_backward_wt", dy.data_ptr(), rows, dy.shape[0], C.byref(w), wt.data_ptr(),
              _ptr(uu), max(r, 1), _ptr(aa), r, gate.data_ptr(), up.data_ptr(), cols, dg.data_ptr(),
              du.data_ptr(), _ptr(ws), ws_bytes, _stream(dev))
        return dg, du
    ws_bytes = _workspace("molt_nf4_lora_backward_workspace", dy.shape[0], rows, cols, 1)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
    _call("molt_nf4_swiglu_backward", dy.data_ptr(), rows, dy.shape[0], C.byref(w), _ptr(uu), max(r, 1),
          _ptr(aa), r, gate.data_ptr(), up.data_ptr(), cols, dg.data_ptr(), du.data_ptr(), _ptr(ws), ws_bytes,
          _stream(dev))
    return dg, du


@nf4_swiglu_backward.register_fake
def _(dy, packed, scales, code, rows, cols, order, u, lora_a, gate, up, wt=None):
    return torch.empty_like(gate), torch.empty_like(up)


@_custom_op(f"{NS}::lora_grad", mutates_args=())
def lora_grad(l: Tensor, l2: Optional[Tensor], mode: int, rmat: Tensor, scale: float,
              layout: int) -> Tensor:
    """scale * L^T R in fp32: dB = s dY^T T (layout 0, [P, Q]) and dA = U^T X
    (layout 1, [Q, P]) (methods/nf4_lora.py:102-103)."""
    what = "LoRA gradient"
    dev = _require_gpu(l, l2, rmat, what=what)
    l = _bf16(l, "activations", what)
    l2 = None if l2 is None else _bf16(l2, "activations", what)
    rmat = _bf16_rows(rmat, "low-rank operand", what)
    if l2 is not None and l2.shape != l.shape:
        raise ValueError(f"{what}: the second operand {tuple(l2.shape)} must match {tuple(l.shape)}")
    if l.dim() != 2 or rmat.dim() != 2 or l.shape[0] != rmat.shape[0]:
        raise ValueError(f"{what}: row counts differ ({tuple(l.shape)} vs {tuple(rmat.shape)})")
    m, p = l.shape
    q = rmat.shape[1]
    out = torch.empty((p, q) if layout == 0 else (q, p), device=dev, dtype=torch.float32)
    ws_bytes = _workspace("molt_lora_grad_workspace", m, p, q)
    ws = torch.empty(max(ws_bytes, 4), device=dev, dtype=torch.uint8)
    _call("molt_lora_grad", l.data_ptr(), _ptr(l2), p, mode, rmat.data_ptr(), max(rmat.stride(0), q), m, p, q,
          float(scale), out.data_ptr(), layout, ws.data_ptr(), ws_bytes, _stream(dev))
    return out


@lora_grad.register_fake
def _(l, l2, mode, rmat, scale, layout):
    p, q = l.shape[1], rmat.shape[1]
    return l.new_empty((p, q) if layout == 0 else (q, p), dtype=torch.float32)


@_custom_op(f"{NS}::lora_grad_many", mutates_args=())
def lora_grad_many(ls: list[Tensor], l2s: list[Optional[Tensor]], modes: list[int], rmats: list[Tensor],
                   scales: list[float], layouts: list[int], norm_inv: Optional[Tensor] = None,
                   norm_weight: Optional[Tensor] = None, norm_offset: float = 0.0) -> list[Tensor]:
    """Several (1..8) ``lora_grad`` (modes 0, 1) results and at most one
    ``lora_grad_rmsnorm`` result (mode 2: ``ls[i]`` is the norm's input x,
    with ``norm_inv``, ``norm_weight`` and ``norm_offset``) with one split-sum
    launch (molt_lora_grad_many): the plain aligned ones share one launch, the
    others take a launch each. Each output is bitwise that of its own call."""
    what = "LoRA gradients"
    n = len(ls)
    if not (1 <= n <= 8) or not (len(l2s) == len(modes) == len(rmats) == len(scales) == len(layouts) == n):
        raise ValueError(f"{what}: 1..8 gradients with one entry per argument list")
    n_norm = sum(1 for md in modes if int(md) == 2)
    if n_norm > 1 or (n_norm == 1) != (norm_inv is not None and norm_weight is not None):
        raise ValueError(f"{what}: at most one RMSNorm-replay gradient, with its inv_rms and weight")
    dev = _require_gpu(*ls, *[t for t in l2s if t is not None], *rmats, norm_inv, norm_weight, what=what)
    keep, outs = [], []
    descs = (_lib.LoraGradDesc * n)()
    for i in range(n):
        mode = int(modes[i])
        # a plain left operand may be a column slice of a wider matrix (its row stride is passed)
        l = _bf16_rows(ls[i], "activations", what) if mode == 0 else _bf16(ls[i], "activations", what)
        l2 = _bf16(l2s[i], "activations", what) if mode == 1 else None
        rmat = _bf16_rows(rmats[i], "low-rank operand", what)
        if mode == 1 and (l2 is None or l2.shape != l.shape):
            raise ValueError(f"{what}: the SwiGLU replay needs an up operand of shape {tuple(l.shape)}")
        if l.dim() != 2 or rmat.dim() != 2 or l.shape[0] != rmat.shape[0]:
            raise ValueError(f"{what}: row counts differ ({tuple(l.shape)} vs {tuple(rmat.shape)})")
        m, p = l.shape
        q = rmat.shape[1]
        inv = w = None
        w_dtype, offset = 0, 0.0
        if mode == 2:
            inv, w, offset = norm_inv, norm_weight.detach().contiguous(), float(norm_offset)
            if inv.dtype != torch.float32 or inv.shape != (m,):
                raise ValueError(f"{what}: inv_rms must be fp32 [{m}]")
            if w.numel() != p:
                raise ValueError(f"{what}: norm weight has {w.numel()} elements for {p} features")
            inv = inv.contiguous()
            w_dtype = _rn_dtype(w, "weight")
        out = torch.empty((p, q) if layouts[i] == 0 else (q, p), device=dev, dtype=torch.float32)
        keep += [l, l2, rmat, inv, w]
        outs.append(out)
        descs[i] = _lib.LoraGradDesc(l.data_ptr(), _ptr(l2), max(l.stride(0), p), mode, rmat.data_ptr(),
                                     max(rmat.stride(0), q), m, p, q, float(scales[i]), out.data_ptr(),
                                     int(layouts[i]), _ptr(inv), _ptr(w), w_dtype, offset)
    ws_bytes = int(_lib.load().molt_lora_grad_many_workspace(n, descs))
    ws = torch.empty(max(ws_bytes, 256), device=dev, dtype=torch.uint8)
    _call("molt_lora_grad_many", n, descs, ws.data_ptr(), ws_bytes, _stream(dev))
    del keep
    return outs


@lora_grad_many.register_fake
def _(ls, l2s, modes, rmats, scales, layouts, norm_inv=None, norm_weight=None, norm_offset=0.0):
    return [l.new_empty((l.shape[1], r.shape[1]) if lay == 0 else (r.shape[1], l.shape[1]), dtype=torch.float32)
            for l, r, lay in zip(ls, rmats, layouts)]


@_custom_op(f"{NS}::lora_grad_rmsnorm", mutates_args=())
def lora_grad_rmsnorm(x: Tensor, inv_rms: Tensor, norm_weight: Tensor, offset: float, rmat: Tensor,
                      scale: float, layout: int) -> Tensor:
    """lora_grad with L = the frozen RMSNorm's bf16 output, formed from its
    input x (bf16 [M, P]), per-row inv_rms (rmsnorm_inv) and weight as it is
    staged, bitwise as over the materialised output
    (methods/gated_replay.py:146-151,167-184)."""
    what = "LoRA gradient over the RMSNorm replay"
    dev = _require_gpu(x, inv_rms, norm_weight, rmat, what=what)
    rmat = _bf16(rmat, "low-rank operand", what)
    if x.dtype != torch.bfloat16 or x.dim() != 2 or not x.is_contiguous():
        raise ValueError(f"{what}: x must be a contiguous bf16 matrix")
    m, p = x.shape
    q = rmat.shape[1] if rmat.dim() == 2 else -1
    if rmat.dim() != 2 or rmat.shape[0] != m:
        raise ValueError(f"{what}: row counts differ ({tuple(x.shape)} vs {tuple(rmat.shape)})")
    if inv_rms.dtype != torch.float32 or inv_rms.shape != (m,):
        raise ValueError(f"{what}: inv_rms must be fp32 [{m}]")
    w = norm_weight.detach().contiguous()
    if w.numel() != p:
        raise ValueError(f"{what}: norm weight has {w.numel()} elements for {p} features")
    out = torch.empty((p, q) if layout == 0 else (q, p), device=dev, dtype=torch.float32)
    ws_bytes = _workspace("molt_lora_grad_workspace", m, p, q)
    ws = torch.empty(max(ws_bytes, 4), device=dev, dtype=torch.uint8)
    _call("molt_lora_grad_rmsnorm", x.data_ptr(), p, inv_rms.contiguous().data_ptr(), w.data_ptr(),
          _rn_dtype(w, "weight"), float(offset), rmat.data_ptr(), q, m, p, q, float(scale), out.data_ptr(), layout,
          ws.data_ptr(), ws_bytes, _stream(dev))
    return out


@lora_grad_rmsnorm.register_fake
def _(x, inv_rms, norm_weight, offset, rmat, scale, layout):
    p, q = x.shape[1], rmat.shape[1]
    return x.new_empty((p, q) if layout == 0 else (q, p), dtype=torch.float32)


def norm_replay_fusable(x: Tensor) -> bool:
    """Whether lora_grad_rmsnorm takes x as it is: a bf16 matrix, contiguous,
    16-byte aligned, a multiple of 8 features."""
    return (x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous() and x.shape[1] % 8 == 0
            and x.data_ptr() % 16 == 0)


# ------------------------------------------------------------------ GEMV
@_custom_op(f"{NS}::nf4_gemv", mutates_args=())
def nf4_gemv(x: Tensor, packed: Tensor, scales: Optional[Tensor], absmax_q: Optional[Tensor],
             absmax2: Optional[Tensor], code2: Optional[Tensor], offset: float, dq_block: int,
             code: Tensor, rows: int, cols: int, order: int, t: Optional[Tensor],
             lora_b: Optional[Tensor], scaling: float) -> Tensor:
    """Skinny-M (<= 16 tokens) NF4 GEMV with the LoRA add-on (decode path of
    training/qlora.py:1332-1358)."""
    what = "NF4 GEMV"
    dev = _require_gpu(x, packed, scales, absmax_q, absmax2, code2, code, t, lora_b, what=what)
    x = _bf16(x, "activations", what)
    if x.dim() != 2 or x.shape[1] != cols or not 1 <= x.shape[0] <= 16:
        raise ValueError(f"{what}: needs 1..16 rows of width {cols}, got {tuple(x.shape)}")
    packed = _check_packed(packed, rows, cols, what)
    _check_stats(what, rows, cols, 64, code, scales=scales, absmax_q=absmax_q, absmax2=absmax2, code2=code2,
                 dq_block=dq_block)
    m = x.shape[0]
    nested = absmax_q is not None
    sc, cd = None if nested else _f32(scales), _f32(code)
    q, a2, c2 = (absmax_q.contiguous(), _f32(absmax2), _f32(code2)) if nested else (None, None, None)
    w = _weight(packed, sc, cd, rows, cols, 64, order, q, a2, c2, offset, dq_block)
    y = torch.empty((m, rows), device=dev, dtype=torch.bfloat16)
    r = 0
    tt = bb = None
    if t is not None:
        if lora_b is None:
            raise ValueError(f"{what}: a low-rank activation needs LoRA B")
        tt, bb = _bf16(t, "low-rank activations", what), _f32(lora_b)
        _check_rows(what, "the low-rank activation", tt, m)
        r = tt.shape[1]
        if bb.shape != (rows, r):
            raise ValueError(f"{what}: LoRA B shape {tuple(bb.shape)} != ({rows}, {r})")
    lib = _lib.load()
    ws_bytes = int(lib.molt_nf4_gemv_workspace(m, rows, cols))
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
    _call("molt_nf4_gemv", x.data_ptr(), cols, m, C.byref(w), _ptr(tt), max(r, 1), _ptr(bb), r,
          float(scaling), y.data_ptr(), rows, _ptr(ws), ws_bytes, _stream(dev))
    return y


@nf4_gemv.register_fake
def _(x, packed, scales, absmax_q, absmax2, code2, offset, dq_block, code, rows, cols, order, t, lora_b,
      scaling):
    return x.new_empty((x.shape[0], rows), dtype=torch.bfloat16)


# --------------------------------------------------------------- SwiGLU
def _sw_dtype(t: Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    if t.dtype == torch.float32:
        return _lib.DTYPE_F32
    raise CapabilityError(f"fused SiLU multiply supports bf16 and fp32 (got {t.dtype})")


@_custom_op(f"{NS}::silu_mul_forward", mutates_args=())
def silu_mul_forward(gate: Tensor, up: Tensor, round_silu: bool) -> Tensor:
    """h = silu(g) * u (kernels/gated_activation.py:29-36)."""
    dev = _require_gpu(gate, up, what="fused SiLU multiply")
    g, u = gate.contiguous(), up.contiguous()
    out = torch.empty_like(g)
    _call("molt_silu_mul_forward", g.data_ptr(), u.data_ptr(), out.data_ptr(), g.numel(), _sw_dtype(g),
          int(round_silu), _stream(dev))
    return out


@silu_mul_forward.register_fake
def _(gate, up, round_silu):
    return torch.empty_like(gate)


@_custom_op(f"{NS}::silu_mul_backward", mutates_args=())
def silu_mul_backward(grad: Tensor, gate: Tensor, up: Tensor) -> tuple[Tensor, Tensor]:
    """(dgate, dup) of h = silu(g) * u (kernels/gated_activation.py:38-51)."""
    dev = _require_gpu(grad, gate, up, what="fused SiLU multiply")
    d, g, u = grad.contiguous(), gate.contiguous(), up.contiguous()
    dg, du = torch.empty_like(g), torch.empty_like(u)
    _call("molt_silu_mul_backward", d.data_ptr(), g.data_ptr(), u.data_ptr(), dg.data_ptr(), du.data_ptr(),
          g.numel(), _sw_dtype(g), _stream(dev))
    return dg, du


@silu_mul_backward.register_fake
def _(grad, gate, up):
    return torch.empty_like(gate), torch.empty_like(up)


# --------------------------------------------------------------------------
# Frozen RMSNorm (kernels/frozen_rmsnorm.py:9-37, methods/gated_replay.py:22-30)
# --------------------------------------------------------------------------
def _rn_dtype(t: Tensor, what: str) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    if t.dtype == torch.float32:
        return _lib.DTYPE_F32
    raise CapabilityError(f"frozen RMSNorm supports bf16 and fp32 {what} (got {t.dtype})")


def _rn_check(x: Tensor, weight: Tensor) -> int:
    if x.dim() == 0 or weight.dim() != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError(f"frozen RMSNorm: weight {tuple(weight.shape)} does not match hidden {tuple(x.shape)}")
    return int(x.shape[-1])


@_custom_op(f"{NS}::rmsnorm_forward", mutates_args=())
def rmsnorm_forward(x: Tensor, weight: Tensor, eps: float, offset: float) -> Tensor:
    """bf16(fp32(x) * rsqrt(mean(fp32(x)^2) + eps) * (fp32(weight) + offset))
    over the last dimension (kernels/frozen_rmsnorm.py:16-23)."""
    dev = _require_gpu(x, weight, what="frozen RMSNorm")
    h = _rn_check(x, weight)
    xc, w = x.contiguous(), weight.detach().contiguous()
    out = torch.empty(x.shape, dtype=torch.bfloat16, device=dev)
    if out.numel() == 0:
        return out
    rows = xc.numel() // h
    _call("molt_rmsnorm_forward", xc.data_ptr(), _rn_dtype(xc, "hidden"), h, rows, h, w.data_ptr(),
          _rn_dtype(w, "weight"), float(eps), float(offset), out.data_ptr(), h, None, _stream(dev))
    return out


@rmsnorm_forward.register_fake
def _(x, weight, eps, offset):
    return torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)


@_custom_op(f"{NS}::rmsnorm_inv", mutates_args=())
def rmsnorm_inv(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """fp32 rsqrt(mean(fp32(x)^2) + eps) of every row, bitwise the value
    rmsnorm_forward(x, weight, ...) scales the row by (same kernel, same
    reduction)."""
    dev = _require_gpu(x, weight, what="frozen RMSNorm")
    h = _rn_check(x, weight)
    xc, w = x.contiguous(), weight.detach().contiguous()
    rows = xc.numel() // h
    inv = torch.empty(rows, dtype=torch.float32, device=dev)
    if rows == 0:
        return inv
    _call("molt_rmsnorm_forward", xc.data_ptr(), _rn_dtype(xc, "hidden"), h, rows, h, w.data_ptr(),
          _rn_dtype(w, "weight"), float(eps), 0.0, None, h, inv.data_ptr(), _stream(dev))
    return inv


@rmsnorm_inv.register_fake
def _(x, weight, eps):
    return torch.empty(x.numel() // x.shape[-1], dtype=torch.float32, device=x.device)


@_custom_op(f"{NS}::rmsnorm_backward", mutates_args=())
def rmsnorm_backward(grad: Tensor, x: Tensor, weight: Tensor, eps: float, offset: float) -> Tensor:
    """Input gradient of the frozen RMSNorm in x's dtype (kernels/frozen_rmsnorm.py:25-37)."""
    dev = _require_gpu(grad, x, weight, what="frozen RMSNorm")
    h = _rn_check(x, weight)
    if grad.shape != x.shape:
        raise ValueError(f"frozen RMSNorm: grad {tuple(grad.shape)} does not match hidden {tuple(x.shape)}")
    dy = grad.to(torch.bfloat16).contiguous()
    xc, w = x.contiguous(), weight.detach().contiguous()
    dx = torch.empty_like(xc)
    if dx.numel() == 0:
        return dx
    rows = xc.numel() // h
    _call("molt_rmsnorm_backward", dy.data_ptr(), h, xc.data_ptr(), _rn_dtype(xc, "hidden"), h, rows, h,
          w.data_ptr(), _rn_dtype(w, "weight"), float(eps), float(offset), dx.data_ptr(), h, _stream(dev))
    return dx


@rmsnorm_backward.register_fake
def _(grad, x, weight, eps, offset):
    return torch.empty_like(x)


# --------------------------------------------------------------------------
# Frozen-head cross-entropy (kernels/frozen_linear_cross_entropy.py:26-139)
# --------------------------------------------------------------------------
@_custom_op(f"{NS}::cross_entropy_rows", mutates_args=("logits",))
def cross_entropy_rows(logits: Tensor, targets: Tensor, total: float, with_grad: bool) -> Tensor:
    """Per-row loss ``(lse - l_y) / total`` (0 for targets outside [0, vocab));
    with ``with_grad`` the logits are overwritten in place by
    ``(softmax - onehot(y)) / total`` in their own dtype."""
    dev = _require_gpu(logits, targets, what="cross-entropy")
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("cross-entropy: logits must be a row-major [rows, vocab] matrix")
    if targets.dtype != torch.long or targets.shape != (logits.shape[0],):
        raise ValueError("cross-entropy: targets must be int64 [rows]")
    dt = _lib.DTYPE_BF16 if logits.dtype == torch.bfloat16 else _lib.DTYPE_F32
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise CapabilityError(f"cross-entropy supports bf16 and fp32 logits (got {logits.dtype})")
    rows, vocab = logits.shape
    loss = torch.empty(rows, device=dev, dtype=torch.float32)
    tg = targets.contiguous()
    _call("molt_cross_entropy_rows", logits.data_ptr(), dt, logits.stride(0), rows, vocab, tg.data_ptr(),
          float(total), loss.data_ptr(), logits.data_ptr() if with_grad else None, logits.stride(0), _stream(dev))
    return loss


@cross_entropy_rows.register_fake
def _(logits, targets, total, with_grad):
    return logits.new_empty((logits.shape[0],), dtype=torch.float32)


@_custom_op(f"{NS}::cross_entropy_rows_exact", mutates_args=("logits",))
def cross_entropy_rows_exact(logits: Tensor, targets: Tensor, total: float, grad_scale: Optional[Tensor],
                             with_grad: bool) -> Tensor:
    """Per-row loss and (with ``with_grad``, in place) gradient under
    F.cross_entropy's rule: rows whose target lies outside [0, vocab) (the
    ignored index -100) get a zero loss and a zero gradient, and the gradient
    is scaled by the device scalar ``grad_scale`` (kernels/partitioned_loss.py:18-103).
    Targets that are neither valid nor ignored are the caller's to reject."""
    dev = _require_gpu(logits, targets, grad_scale, what="cross-entropy")
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("cross-entropy: logits must be a row-major [rows, vocab] matrix")
    if targets.dtype != torch.long or targets.shape != (logits.shape[0],):
        raise ValueError("cross-entropy: targets must be int64 [rows]")
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise CapabilityError(f"cross-entropy supports bf16 and fp32 logits (got {logits.dtype})")
    dt = _lib.DTYPE_BF16 if logits.dtype == torch.bfloat16 else _lib.DTYPE_F32
    gs = None if grad_scale is None else grad_scale.detach().reshape(-1)[:1].to(torch.float32).contiguous()
    rows, vocab = logits.shape
    loss = torch.empty(rows, device=dev, dtype=torch.float32)
    tg = targets.contiguous()
    _call("molt_cross_entropy_rows_exact", logits.data_ptr(), dt, logits.stride(0), rows, vocab, tg.data_ptr(),
          float(total), _ptr(gs), loss.data_ptr(), logits.data_ptr() if with_grad else None, logits.stride(0),
          _stream(dev))
    return loss


@cross_entropy_rows_exact.register_fake
def _(logits, targets, total, grad_scale, with_grad):
    return logits.new_empty((logits.shape[0],), dtype=torch.float32)
