"""CPU oracle for the NF4 QLoRA linear and gated-MLP hot path (TEST INFRASTRUCTURE).

This module is the checker, never the product. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The shipped path (``molt_amd``) never calls into it and fails loudly
when its HIP library is missing.

It restates, in numpy, the algorithms of the reference (PraveenNimilka/MOLT)
on the path, each function citing the reference file:line it follows
(paths relative to the reference's ``src/molt_stream/``).

Pinning (what independently checks each function; see ``tests/test_oracle.py``):

* ``NF4_CODE`` - the 16 literals of ``streaming/nf4.py:10-18``; pinned against
  QLoRA's normal-quantile construction recomputed with scipy.
* ``quantize_blocks`` - pinned by the reference's own CPU test
  (``tests/test_molt_stream_nf4.py:9-15``: storage bytes and RMS error on
  ``torch.randn(64, 64)`` seed 1), exact round trip of every code times
  sampled scales, tie-breaking at exact fp32 midpoints, sign preservation,
  the error bound, and a per-element brute force on tiny inputs.
* ``pack_nibbles`` / ``unpack_nibbles`` - pinned by a per-element Python loop
  on tiny inputs for both nibble orders.
* ``bf16_rne`` - pinned against torch's own fp32->bf16 conversion.
* ``dequantize`` - pinned by the round-trip and torch-conversion checks above.
* ``absmax_offset`` - pinned against ``math.fsum`` (1 fp32 ulp).
* ``double_quantize`` / ``resolve_scales`` - pinned by blocks whose values
  decode exactly (centred value 0 or the block maximum) or to a closed form,
  with a different absmax2 per block; by the error bound
  ``|resolved - absmax| <= absmax2 * max_gap(code2) / 2``; and, for the
  rounding order, by torch CPU fp32 ``mul`` then ``add_`` (the two ops of
  methods/nf4_backward.py:157-160) on inputs where a fused multiply-add
  rounds differently.
* ``linspace_f32`` / ``dynamic_map`` - bitsandbytes' ``create_dynamic_map``
  (bitsandbytes 0.50.2, a dependency absent from the reference tree and from
  this image). Pinned bit for bit against the published construction run as
  torch fp32 ops (``torch.linspace`` without a dtype is fp32; the Python-float
  decade scale multiplies in fp32), with the fp64-scale variant shown to
  differ; also against torch's fp32 ``linspace``, the closed form of each
  entry (2 ulp) and the entry count per decade.
* ``lora_linear_*``, ``swiglu_*``, ``gated_mlp_*`` - fp64 textbook algebra;
  the backward formulas are pinned against torch autograd of the forward
  expression in fp64, and SwiGLU against ``F.silu(g) * u``
  (``tests/kernels/test_gated_activation.py:10-26``).
* ``lora_linear_forward_bf16_points`` - the reference's autocast rounding
  points, pinned against the same forward run as torch CPU bf16 ops.
* ``lora_linear_backward_bf16_points`` / ``gated_mlp_reference_bf16`` - the
  reference's own bf16 step (rounding points of methods/nf4_lora.py:83-109 and
  methods/gated_replay.py:290-299,372-388), pinned against torch autograd under
  CPU bf16 autocast of the same graph (>= 99.9 % of elements equal). Used only
  to report how far the reference path itself lands from the fp64 oracle.
* ``rmsnorm_forward`` / ``rmsnorm_backward`` - fp64 algebra. The forward is
  pinned by closed forms (a constant row maps to ``sign * (w + offset)`` at
  eps = 0, scale invariance, unit RMS of the normalised row); the backward by
  central differences of the forward in fp64 and by its two invariants
  (zero gradient along x at eps = 0, and the closed form of the reference's
  own test, ``tests/kernels/test_frozen_rmsnorm.py:6-53``).
* ``cross_entropy_rows`` - pinned against torch's ``F.cross_entropy`` and its
  autograd gradient in fp64 for valid targets, by central differences of the
  summed loss, and by the invariants of the invalid-target rows (zero loss,
  a softmax gradient that sums to 1/total).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

# streaming/nf4.py:10-18 - MOLT's NormalFloat-4 literals (fp32).
NF4_CODE = np.array(
    [
        -1.0, -0.6961928, -0.52507305, -0.3949175,
        -0.28444138, -0.18477343, -0.09105004, 0.0,
        0.0795803, 0.1609302, 0.2461123, 0.33791524,
        0.44070983, 0.562617, 0.72295684, 1.0,
    ],
    dtype=np.float32,
)

FP32_TINY = np.float32(np.finfo(np.float32).tiny)

NIBBLE_LOW_FIRST = 0   # streaming/nf4.py:62  element 2i in the low nibble
NIBBLE_HIGH_FIRST = 1  # methods/nf4_backward.py:97-98  element 2i in the high nibble


# --------------------------------------------------------------------------
# bf16 helpers
# --------------------------------------------------------------------------
def bf16_rne_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern, round-to-nearest-even; NaN -> 0x7FC0."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    bits = f.view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    out = rounded.astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        out[nan] = 0x7FC0
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 (or fp64, first rounded to fp32) values to bf16, returned as fp32."""
    return bf16_bits_to_f32(bf16_rne_bits(np.asarray(x, dtype=np.float32)))


# --------------------------------------------------------------------------
# NF4 codec
# --------------------------------------------------------------------------
def quantize_blocks(values: np.ndarray, block_size: int, code: np.ndarray = NF4_CODE):
    """Blockwise NF4 codes and fp32 absmax, following streaming/nf4.py:50-61.

    Flattens, zero-pads to a whole block, absmax per block clamped to the
    smallest normal fp32, divides (fp32) and takes the first index of the
    minimum ``|normalized - code|``. Returns (indices uint8 [padded], absmax fp32).
    """
    if values.size == 0 or block_size < 16 or block_size % 2:
        raise ValueError("invalid tensor or NF4 block size")
    flat = np.asarray(values, dtype=np.float32).reshape(-1)
    pad = (-flat.size) % block_size
    if pad:
        flat = np.concatenate([flat, np.zeros(pad, np.float32)])
    blocks = flat.reshape(-1, block_size)
    absmax = np.maximum(np.abs(blocks).max(axis=1), FP32_TINY).astype(np.float32)
    code = np.asarray(code, dtype=np.float32)
    idx = np.empty(blocks.shape, dtype=np.uint8)
    chunk = max(1, (1 << 22) // block_size)
    for s in range(0, blocks.shape[0], chunk):
        normalized = (blocks[s:s + chunk] / absmax[s:s + chunk, None]).astype(np.float32)
        dist = np.abs(normalized[..., None] - code).astype(np.float32)
        idx[s:s + chunk] = np.argmin(dist, axis=-1).astype(np.uint8)
    return idx.reshape(-1), absmax


def pack_nibbles(idx: np.ndarray, order: int) -> np.ndarray:
    """Pack codes two per byte: streaming/nf4.py:62 (low first) or
    methods/nf4_backward.py:97-98 (high first, bitsandbytes)."""
    idx = np.asarray(idx, dtype=np.uint8).reshape(-1)
    if idx.size % 2:
        idx = np.concatenate([idx, np.zeros(1, np.uint8)])
    even, odd = idx[0::2], idx[1::2]
    if order == NIBBLE_LOW_FIRST:
        return (even | (odd << 4)).astype(np.uint8)
    return ((even << 4) | odd).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray, order: int, n: int) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.uint8).reshape(-1)
    low, high = packed & 0x0F, packed >> 4
    first, second = (low, high) if order == NIBBLE_LOW_FIRST else (high, low)
    return np.stack([first, second], axis=-1).reshape(-1)[:n]


def dequantize_f32(idx: np.ndarray, scales: np.ndarray, block_size: int,
                   code: np.ndarray = NF4_CODE) -> np.ndarray:
    """fp32 ``code[idx] * scale`` per element (streaming/nf4.py:33-34)."""
    idx = np.asarray(idx).reshape(-1)
    code = np.asarray(code, dtype=np.float32)
    block = np.arange(idx.size) // block_size
    return (code[idx] * np.asarray(scales, dtype=np.float32)[block]).astype(np.float32)


def dequantize_bf16_bits(idx, scales, block_size, code=NF4_CODE) -> np.ndarray:
    """bf16 bit patterns of ``bf16(fp32(code[idx] * scale))``
    (streaming/nf4.py:33-35 ``.to(bfloat16)``; methods/nf4_backward.py:99-105)."""
    return bf16_rne_bits(dequantize_f32(idx, scales, block_size, code))


# --------------------------------------------------------------------------
# Double quantisation of absmax (bitsandbytes compress_statistics=True)
# --------------------------------------------------------------------------
def linspace_f32(start: float, end: float, steps: int) -> np.ndarray:
    """fp32 ``torch.linspace(start, end, steps)`` as its CPU kernel computes it:
    ``step = fl32((end - start) / (steps - 1))``; the first half is
    ``fma(step, i, start)`` and the second ``end - step * (steps - 1 - i)``,
    each rounded once to fp32 (``step * i`` is exact in fp64 here, so the fp64
    expression below is that single rounding)."""
    s, e = np.float32(start), np.float32(end)
    if steps == 1:
        return np.array([s], np.float32)
    step = np.float32((e - s) / np.float32(steps - 1))
    idx = np.arange(steps, dtype=np.float64)
    head = np.float64(s) + np.float64(step) * idx
    tail = np.float64(e) - np.float64(step) * (steps - 1 - idx)
    return np.where(idx < steps // 2, head, tail).astype(np.float32)


def dynamic_map(signed: bool = True, max_exponent_bits: int = 7, total_bits: int = 8) -> np.ndarray:
    """Restatement of bitsandbytes' ``create_dynamic_map`` (bitsandbytes 0.50.2,
    not vendored in the reference; version pinned in uv.lock:46-47): for each
    decade i the midpoints of an fp32 ``linspace(0.1, 1, 2**i + 1)``, scaled by
    ``fl32(10**(i - 6))`` in fp32, with both signs, plus 0 and 1, sorted.

    Pinned (tests/test_oracle.py) bit for bit against the published
    construction run as torch fp32 ops (fp32 ``torch.linspace``, fp32
    midpoints, the Python-float decade scale applied in fp32); an fp64-scale
    variant differs from it. Also against torch's own fp32 linspace, the closed
    form ``10**(i-6) * (b_j + b_{j+1}) / 2`` with ``b_j = 0.1 + 0.9 j / 2**i``
    to 2 ulp per entry, and the entry count per decade. The kernels read the
    table as data, so it only decides which table this build's quantiser
    writes."""
    data: list[float] = []
    non_sign_bits = total_bits - 1
    additional = 2 ** (non_sign_bits - max_exponent_bits) - 1
    decades = list(range(max_exponent_bits))
    counts = [(2 ** (i + non_sign_bits - max_exponent_bits) + 1) if signed
              else (2 ** (i + non_sign_bits - max_exponent_bits + 1) + 1) for i in decades]
    if additional > 0:
        decades.append(max_exponent_bits - 1)
        counts.append(additional + 1)
    for i, items in zip(decades, counts):
        bounds = linspace_f32(0.1, 1.0, items)
        means = ((bounds[:-1] + bounds[1:]) / np.float32(2.0)).astype(np.float32)
        mag = np.float32(10.0 ** (-(max_exponent_bits - 1) + i))
        vals = (mag * means).astype(np.float32)
        data += vals.tolist()
        if signed:
            data += (-vals).tolist()
    data += [0.0, 1.0]
    data += [0.0] * (2 ** total_bits - len(data))
    return np.sort(np.array(data, dtype=np.float32))


DQ_BLOCK = 256


DQ_CHUNK = 4096


def absmax_offset(absmax: np.ndarray) -> np.float32:
    """Mean of the block absmax values (bitsandbytes' ``absmax.mean()``) with
    the arithmetic fixed so host and device agree bit for bit: fp64 partial
    sums over chunks of 4096 values (within a chunk, 256 runs of 16 values
    each summed left to right, then a halving tree over the 256 runs), chunk
    sums added left to right, divided by n in fp64, rounded once to fp32.
    Pinned against ``math.fsum`` (|error| <= 1 fp32 ulp)."""
    a = np.asarray(absmax, dtype=np.float32).astype(np.float64).reshape(-1)
    n = a.size
    chunks = -(-n // DQ_CHUNK)
    padded = np.zeros(chunks * DQ_CHUNK, np.float64)
    padded[:n] = a
    runs = padded.reshape(chunks, 256, 16)
    s = np.zeros((chunks, 256), np.float64)
    for i in range(16):
        s = s + runs[:, :, i]
    stride = 128
    while stride >= 1:
        s[:, :stride] = s[:, :stride] + s[:, stride:2 * stride]
        stride //= 2
    total = 0.0
    for c in range(chunks):
        total = total + float(s[c, 0])
    return np.float32(total / n)


def double_quantize(absmax: np.ndarray, code2: np.ndarray | None = None, block: int = DQ_BLOCK):
    """Nested absmax: offset = mean, then blockwise 8-bit quantisation of
    ``absmax - offset`` against ``code2`` (first index of the nearest value).
    Returns (q uint8 [n], absmax2 fp32 [ceil(n/block)], offset fp32, code2)."""
    code2 = dynamic_map() if code2 is None else np.asarray(code2, np.float32)
    absmax = np.asarray(absmax, dtype=np.float32)
    offset = absmax_offset(absmax)
    centred = (absmax - offset).astype(np.float32)
    n = centred.size
    nb = -(-n // block)
    padded = np.concatenate([centred, np.zeros(nb * block - n, np.float32)]).reshape(nb, block)
    absmax2 = np.maximum(np.abs(padded).max(axis=1), FP32_TINY).astype(np.float32)
    q = np.empty(padded.shape, np.uint8)
    for s in range(0, nb, 4096):
        normalized = (padded[s:s + 4096] / absmax2[s:s + 4096, None]).astype(np.float32)
        dist = np.abs(normalized[..., None] - code2).astype(np.float32)
        q[s:s + 4096] = np.argmin(dist, axis=-1).astype(np.uint8)
    return q.reshape(-1)[:n], absmax2, offset, code2


def resolve_scales(q: np.ndarray, absmax2: np.ndarray, code2: np.ndarray,
                   offset: np.float32, block: int = DQ_BLOCK) -> np.ndarray:
    """``fl32(fl32(code2[q] * absmax2[j]) + offset)`` in the order of
    methods/nf4_backward.py:157-160 (dequantize_blockwise, then add offset)."""
    q = np.asarray(q).reshape(-1)
    j = np.arange(q.size) // block
    prod = (np.asarray(code2, np.float32)[q] * np.asarray(absmax2, np.float32)[j]).astype(np.float32)
    return (prod + np.float32(offset)).astype(np.float32)


@dataclass
class OracleNF4:
    """A quantised matrix as the oracle sees it (either layout)."""
    packed: np.ndarray        # uint8 [ceil(n/2)]
    shape: tuple
    block_size: int
    order: int
    code: np.ndarray          # fp32 [16]
    absmax: np.ndarray        # fp32 [nblocks] - the raw per-block absmax
    scales: np.ndarray        # fp32 [nblocks] - what dequant multiplies by
    nested: bool = False
    q: np.ndarray | None = None
    absmax2: np.ndarray | None = None
    code2: np.ndarray | None = None
    offset: np.float32 | None = None

    @property
    def elements(self) -> int:
        return int(np.prod(self.shape))

    def indices(self) -> np.ndarray:
        return unpack_nibbles(self.packed, self.order, self.elements)

    def dequant_bf16_bits(self) -> np.ndarray:
        return dequantize_bf16_bits(self.indices(), self.scales, self.block_size,
                                    self.code).reshape(self.shape)

    def dequant_bf16(self) -> np.ndarray:
        return bf16_bits_to_f32(self.dequant_bf16_bits())

    def dequant_f32(self) -> np.ndarray:
        return dequantize_f32(self.indices(), self.scales, self.block_size,
                              self.code).reshape(self.shape)


def quantize_cleanroom(values: np.ndarray, block_size: int = 64) -> OracleNF4:
    """MOLT ``NF4Tensor.quantize`` (streaming/nf4.py:46-68): low nibble first,
    one fp32 absmax per block, no double quantisation."""
    idx, absmax = quantize_blocks(values, block_size)
    return OracleNF4(pack_nibbles(idx, NIBBLE_LOW_FIRST), tuple(values.shape), block_size,
                     NIBBLE_LOW_FIRST, NF4_CODE.copy(), absmax, absmax)


def quantize_bnb_layout(values: np.ndarray, block_size: int = 64, nested: bool = True,
                        code: np.ndarray = NF4_CODE) -> OracleNF4:
    """bitsandbytes layout (``quantize_4bit(blocksize=64, compress_statistics=True,
    quant_type='nf4')`` as consumed at methods/nf4_backward.py:97-105,145-164):
    high nibble first, optional nested absmax. Code decisions follow
    streaming/nf4.py:57-61 (fp32 divide, first-index argmin); bitsandbytes'
    own decision tree is absent here, so that part is parity unpinned."""
    idx, absmax = quantize_blocks(values, block_size, code)
    packed = pack_nibbles(idx, NIBBLE_HIGH_FIRST)
    if not nested:
        return OracleNF4(packed, tuple(values.shape), block_size, NIBBLE_HIGH_FIRST,
                         np.asarray(code, np.float32).copy(), absmax, absmax)
    q, absmax2, offset, code2 = double_quantize(absmax)
    scales = resolve_scales(q, absmax2, code2, offset)
    return OracleNF4(packed, tuple(values.shape), block_size, NIBBLE_HIGH_FIRST,
                     np.asarray(code, np.float32).copy(), absmax, scales, True, q,
                     absmax2, code2, offset)


def storage_bytes(t: OracleNF4) -> int:
    """streaming/nf4.py:70-72 (clean-room), plus the nested statistics."""
    if not t.nested:
        return t.packed.size + t.scales.size * 4
    return t.packed.size + t.q.size + t.absmax2.size * 4 + 4


# --------------------------------------------------------------------------
# NF4 + LoRA linear (fp64 algebra over bf16-valued inputs)
# --------------------------------------------------------------------------
def _f64(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64)


def lora_linear_forward(x, w, a, b, s):
    """``Y = X W^T + s (X A^T) B^T`` (streaming/engine.py:27-31;
    methods/nf4_lora.py:43-50). fp64."""
    x, w, a, b = map(_f64, (x, w, a, b))
    return x @ w.T + s * ((x @ a.T) @ b.T)


def lora_linear_backward(x, w, a, b, s, dy):
    """``dX = dY W + s (dY B) A``, ``dA = s (dY B)^T X``, ``dB = s dY^T (X A^T)``
    (streaming/engine.py:41-44; methods/nf4_lora.py:86-103). fp64."""
    x, w, a, b, dy = map(_f64, (x, w, a, b, dy))
    t = x @ a.T
    u = s * (dy @ b)
    return dy @ w + u @ a, u.T @ x, s * (dy.T @ t)


def lora_linear_forward_bf16_points(x, w, a, b, s):
    """Forward with MOLT's bf16 rounding points under autocast
    (methods/nf4_lora.py:43-50): base, low_rank, the LoRA GEMM, the scaled
    term and the sum are each rounded to bf16. Inner products are fp64."""
    x, w = _f64(x), _f64(w)
    a16, b16 = bf16_round(a).astype(np.float64), bf16_round(b).astype(np.float64)
    base = bf16_round(x @ w.T)
    low = bf16_round(x @ a16.T).astype(np.float64)
    lora = bf16_round(low @ b16.T)
    term = bf16_round(lora.astype(np.float32) * np.float32(s))
    return bf16_round(base.astype(np.float32) + term.astype(np.float32))


def lora_linear_backward_bf16_points(x, w, a, b, s, dy):
    """Backward with MOLT's bf16 rounding points under autocast
    (methods/nf4_lora.py:83-109, the same equations as
    methods/gated_replay.py:236-253): ``low = bf16(X A^T)``,
    ``scaled = bf16(dY s)`` (scale before the product), ``through = bf16(scaled B)``,
    ``base = bf16(dY W)``, ``dX = bf16(base + bf16(through A))``,
    ``dB = bf16(scaled^T low)``, ``dA = bf16(through^T X)``; dA and dB are then
    widened to fp32 (``.to(lora_a.dtype)``), so they carry a bf16 rounding.
    Inner products are fp64 (the library GEMMs accumulate in fp32)."""
    x, w, dy = _f64(x), _f64(w), _f64(dy)
    a16, b16 = bf16_round(a).astype(np.float64), bf16_round(b).astype(np.float64)
    low = bf16_round(x @ a16.T).astype(np.float64)
    scaled = bf16_round(dy * s).astype(np.float64)
    through = bf16_round(scaled @ b16).astype(np.float64)
    base = bf16_round(dy @ w)
    dx = bf16_round(base + bf16_round(through @ a16))
    return dx.astype(np.float64), bf16_round(through.T @ x).astype(np.float64), \
        bf16_round(scaled.T @ low).astype(np.float64)


def gated_mlp_reference_bf16(x, wg, wu, wd, ag, bg, au, bu, ad, bd, s, dy):
    """The reference's own bf16 gated-MLP step, every autocast rounding point
    kept, for reporting how far MOLT's path itself lands from the fp64 oracle.
    gate and up come from NF4-LoRA nodes (methods/nf4_lora.py:43-50); the
    replay node forms ``bf16(bf16(silu(g)) * u)`` (methods/gated_replay.py:290-291,
    372-374), runs the down projection's bf16 backward, then
    ``du = bf16(dh * bf16(silu(g)))`` and ``dg = silu_backward(bf16(dh * u), g)``
    rounded to bf16 (:385-387); autograd adds the gate and up input gradients in
    bf16. Returns (Y, dX, (dAg, dBg, dAu, dBu, dAd, dBd))."""
    rnd = lambda v: bf16_round(v).astype(np.float64)  # noqa: E731
    g = rnd(lora_linear_forward_bf16_points(x, wg, ag, bg, s))
    u = rnd(lora_linear_forward_bf16_points(x, wu, au, bu, s))
    act = rnd(g * _sigmoid(g))
    h = rnd(act * u)
    y = rnd(lora_linear_forward_bf16_points(h, wd, ad, bd, s))
    dh, dad, dbd = lora_linear_backward_bf16_points(h, wd, ad, bd, s, dy)
    du = rnd(dh * act)
    sg = _sigmoid(g)
    dg = rnd(rnd(dh * u) * sg * (1.0 + g * (1.0 - sg)))
    dxg, dag, dbg = lora_linear_backward_bf16_points(x, wg, ag, bg, s, dg)
    dxu, dau, dbu = lora_linear_backward_bf16_points(x, wu, au, bu, s, du)
    return y, rnd(dxg + dxu), (dag, dbg, dau, dbu, dad, dbd)


# --------------------------------------------------------------------------
# SwiGLU (kernels/gated_activation.py:29-51; methods/gated_replay.py:290-299,373-388)
# --------------------------------------------------------------------------
def _sigmoid(g):
    return 1.0 / (1.0 + np.exp(-g))


def swiglu_forward(g, u):
    """``h = g * sigmoid(g) * u`` (kernels/gated_activation.py:33-36)."""
    g, u = _f64(g), _f64(u)
    return g * _sigmoid(g) * u


def swiglu_backward(g, u, dh):
    """``dg = dh u s (1 + g (1 - s))``, ``du = dh g s`` (kernels/gated_activation.py:44-51)."""
    g, u, dh = _f64(g), _f64(u), _f64(dh)
    sg = _sigmoid(g)
    return dh * u * sg * (1.0 + g * (1.0 - sg)), dh * g * sg


# --------------------------------------------------------------------------
# Gated MLP with NF4+LoRA projections (methods/gated_replay.py:50-208,256-407)
# --------------------------------------------------------------------------
def gated_mlp_forward(x, wg, wu, wd, ag, bg, au, bu, ad, bd, s, bf16_storage=True):
    """Returns (y, saved) with ``g = LoRA(x; Wg)``, ``u = LoRA(x; Wu)``,
    ``h = silu(g) u`` and ``y = LoRA(h; Wd)``. When ``bf16_storage`` the
    stored activations g, u, h are rounded to bf16 as the reference stores
    them under autocast (methods/gated_replay.py:290-299)."""
    rnd = (lambda v: bf16_round(v).astype(np.float64)) if bf16_storage else _f64
    g = rnd(lora_linear_forward(x, wg, ag, bg, s))
    u = rnd(lora_linear_forward(x, wu, au, bu, s))
    h = rnd(swiglu_forward(g, u))
    y = lora_linear_forward(h, wd, ad, bd, s)
    return y, {"g": g, "u": u, "h": h}


def gated_mlp_backward(x, wg, wu, wd, ag, bg, au, bu, ad, bd, s, dy, saved, bf16_storage=True):
    """Gradient algebra of methods/gated_replay.py:373-388 extended to the
    gate/up projections (methods/gated_replay.py:155-186). Returns
    dX and (dAg, dBg, dAu, dBu, dAd, dBd)."""
    rnd = (lambda v: bf16_round(v).astype(np.float64)) if bf16_storage else _f64
    g, u, h = saved["g"], saved["u"], saved["h"]
    dh, dad, dbd = lora_linear_backward(h, wd, ad, bd, s, dy)
    dh = rnd(dh)
    dg, du = swiglu_backward(g, u, dh)
    dg, du = rnd(dg), rnd(du)
    dxg, dag, dbg = lora_linear_backward(x, wg, ag, bg, s, dg)
    dxu, dau, dbu = lora_linear_backward(x, wu, au, bu, s, du)
    return dxg + dxu, (dag, dbg, dau, dbu, dad, dbd)


# --------------------------------------------------------------------------
# Frozen RMSNorm (kernels/frozen_rmsnorm.py:9-37; methods/gated_replay.py:13-30)
# --------------------------------------------------------------------------
def rmsnorm_forward(x, w, eps, offset):
    """``x * rsqrt(mean(x^2) + eps) * (w + offset)`` over the last axis
    (kernels/frozen_rmsnorm.py:16-23; methods/gated_replay.py:22-30). fp64,
    before the bf16 rounding of the output."""
    x, w = _f64(x), _f64(w)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * inv * (w + offset)


def rmsnorm_backward(x, w, eps, offset, dy):
    """Input gradient of the frozen-weight RMSNorm (kernels/frozen_rmsnorm.py:25-37):
    ``inv * (g - n * mean(g * n))``, ``n = x * inv``, ``g = dy * (w + offset)``. fp64."""
    x, w, dy = _f64(x), _f64(w), _f64(dy)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    n = x * inv
    g = dy * (w + offset)
    return inv * (g - n * np.mean(g * n, axis=-1, keepdims=True))


# --------------------------------------------------------------------------
# Frozen-head cross-entropy (kernels/frozen_linear_cross_entropy.py:26-139)
# --------------------------------------------------------------------------
def cross_entropy_rows(logits, targets, total):
    """Per-row loss ``(lse - l_y) / total`` and gradient
    ``(softmax - onehot(y)) / total``; a target outside [0, vocab) gives a zero
    loss and the plain softmax gradient, as the fused kernel's ``valid_target``
    mask does (kernels/frozen_linear_cross_entropy.py:97-139). fp64."""
    z = _f64(logits)
    t = np.asarray(targets, dtype=np.int64)
    m = z.max(axis=1, keepdims=True)
    e = np.exp(z - m)
    d = e.sum(axis=1, keepdims=True)
    lse = (m + np.log(d))[:, 0]
    valid = (t >= 0) & (t < z.shape[1])
    rows = np.arange(z.shape[0])
    ly = np.where(valid, z[rows, np.where(valid, t, 0)], 0.0)
    loss = np.where(valid, (lse - ly) / total, 0.0)
    grad = e / d
    grad[rows[valid], t[valid]] -= 1.0
    return loss, grad / total


# --------------------------------------------------------------------------
# Comparisons
# --------------------------------------------------------------------------
def rel_fro(actual, expected) -> float:
    """Relative Frobenius error ||a - e|| / ||e|| in fp64."""
    a, e = _f64(actual), _f64(expected)
    denom = np.linalg.norm(e)
    return float(np.linalg.norm(a - e) / (denom if denom > 0 else 1.0))
