"""Pins for the CPU oracle (no GPU). Each check is independent of the formula
it checks: a published construction, torch's own implementation, the
reference's own CPU tests, exact arithmetic, or per-element brute force."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as O


# --------------------------------------------------------------- codebook
def _qlora_normal_map(offset: float = 0.9677083) -> np.ndarray:
    """NF4 levels from the QLoRA construction: normal quantiles, 8 positive and
    7 negative, plus zero, normalised by the largest."""
    from scipy.stats import norm

    v1 = norm.ppf(np.linspace(offset, 0.5, 9)[:-1])
    v3 = -norm.ppf(np.linspace(offset, 0.5, 8)[:-1])
    values = np.sort(np.concatenate([v1, [0.0], v3]))
    return values / values.max()


def test_codebook_matches_qlora_normal_quantiles():
    ref = _qlora_normal_map()
    assert O.NF4_CODE.shape == (16,)
    np.testing.assert_allclose(O.NF4_CODE.astype(np.float64), ref, rtol=0, atol=2e-7)
    assert O.NF4_CODE[7] == 0.0 and O.NF4_CODE[0] == -1.0 and O.NF4_CODE[15] == 1.0
    assert np.all(np.diff(O.NF4_CODE) > 0)


def test_package_codebook_is_the_oracle_codebook():
    import molt_amd

    assert np.array_equal(molt_amd.NF4_CODEBOOK.numpy().view(np.uint32), O.NF4_CODE.view(np.uint32))


# ------------------------------------------------------------ bf16 rounding
def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.normal(0, 1, 20000).astype(np.float32),
        rng.normal(0, 1e-30, 2000).astype(np.float32),
        (rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32)).view(np.float32),
    ])
    x = x[np.isfinite(x)]
    ours = O.bf16_rne_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)


# ----------------------------------------------- reference's own CPU test
def test_reference_storage_and_rms_error():
    """tests/test_molt_stream_nf4.py:9-15 restated on the oracle."""
    torch.manual_seed(1)
    value = torch.randn(64, 64).numpy()
    t = O.quantize_cleanroom(value, block_size=64)
    restored = t.dequant_f32()
    assert O.storage_bytes(t) == value.size // 2 + value.size // 64 * 4
    assert float(np.sqrt(np.mean((restored - value) ** 2))) < 0.15


# --------------------------------------------------------------- quantise
def _brute_codes(block: np.ndarray, code: np.ndarray) -> tuple[list[int], np.float32]:
    absmax = np.float32(0.0)
    for v in block:
        absmax = max(absmax, np.float32(abs(np.float32(v))))
    absmax = max(absmax, O.FP32_TINY)
    out = []
    for v in block:
        nv = np.float32(np.float32(v) / absmax)
        best, bi = None, 0
        for i, c in enumerate(code):
            d = np.float32(abs(np.float32(nv - c)))
            if best is None or d < best:
                best, bi = d, i
        out.append(bi)
    return out, absmax


@pytest.mark.parametrize("n,block", [(40, 16), (64, 64), (130, 64), (50, 32)])
def test_quantize_matches_per_element_brute_force(n, block):
    rng = np.random.default_rng(n + block)
    x = rng.normal(0, 1, n).astype(np.float32)
    idx, absmax = O.quantize_blocks(x, block)
    padded = np.concatenate([x, np.zeros((-n) % block, np.float32)])
    for b in range(padded.size // block):
        codes, am = _brute_codes(padded[b * block:(b + 1) * block], O.NF4_CODE)
        assert absmax[b] == am
        assert list(idx[b * block:(b + 1) * block]) == codes


def test_exact_codes_round_trip_and_midpoint_ties():
    # every code times a set of power-of-two and odd scales survives exactly
    for s in (np.float32(1.0), np.float32(0.5), np.float32(3.0), np.float32(1e-3)):
        x = (O.NF4_CODE * s).astype(np.float32)
        idx, absmax = O.quantize_blocks(np.concatenate([x, x]), 32)
        assert np.array_equal(idx[:16], np.arange(16))
        assert np.array_equal(O.dequantize_f32(idx, absmax, 32)[:16], x)
    # at an exact fp32 tie the lower code wins (first index of the minimum)
    lo, hi = O.NF4_CODE[9], O.NF4_CODE[10]
    for m in (np.float32((np.float64(lo) + np.float64(hi)) / 2),
              np.nextafter(np.float32((np.float64(lo) + np.float64(hi)) / 2), np.float32(1))):
        block = np.array([1.0, m] + [0.0] * 14, np.float32)
        d_lo, d_hi = np.float32(abs(m - lo)), np.float32(abs(m - hi))
        idx, _ = O.quantize_blocks(block, 16)
        assert idx[1] == (9 if d_lo <= d_hi else 10)


def test_quantize_invariants():
    rng = np.random.default_rng(11)
    x = rng.normal(0, 0.02, 64 * 50).astype(np.float32)
    idx, absmax = O.quantize_blocks(x, 64)
    deq = O.dequantize_f32(idx, absmax, 64)
    gaps = np.diff(O.NF4_CODE.astype(np.float64)).max()
    blk = np.repeat(absmax, 64)
    assert np.all(np.abs(deq - x) <= gaps / 2 * blk * (1 + 1e-6))
    assert np.all(np.sign(deq[np.abs(x) > blk * 0.05]) == np.sign(x[np.abs(x) > blk * 0.05]))
    # the block maximum maps to +-1
    for b in range(50):
        j = np.argmax(np.abs(x[b * 64:(b + 1) * 64]))
        assert idx[b * 64 + j] in (0, 15)


@pytest.mark.parametrize("order", [O.NIBBLE_LOW_FIRST, O.NIBBLE_HIGH_FIRST])
def test_pack_unpack_against_python_loop(order):
    rng = np.random.default_rng(order)
    idx = rng.integers(0, 16, 37).astype(np.uint8)
    packed = O.pack_nibbles(idx, order)
    for i in range(37):
        byte = int(packed[i // 2])
        first = (byte & 15) if order == O.NIBBLE_LOW_FIRST else (byte >> 4)
        second = (byte >> 4) if order == O.NIBBLE_LOW_FIRST else (byte & 15)
        assert idx[i] == (first if i % 2 == 0 else second)
    assert np.array_equal(O.unpack_nibbles(packed, order, 37), idx)


def test_dequant_bf16_is_rne_of_fp32_product():
    rng = np.random.default_rng(3)
    idx = rng.integers(0, 16, 4096).astype(np.uint8)
    scales = np.abs(rng.normal(0, 0.05, 64)).astype(np.float32)
    prod = torch.from_numpy(O.NF4_CODE)[torch.from_numpy(idx.astype(np.int64))] * \
        torch.from_numpy(scales).repeat_interleave(64)
    ref = prod.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.dequantize_bf16_bits(idx, scales, 64), ref)


# ------------------------------------------------------ double quantise
def test_offset_is_the_mean_to_one_ulp():
    rng = np.random.default_rng(7)
    for n in (1, 255, 4096, 4097, 100003):
        a = (np.abs(rng.normal(0, 0.02, n)) + 1e-5).astype(np.float32)
        off = O.absmax_offset(a)
        exact = math.fsum(a.astype(np.float64)) / n
        assert abs(float(off) - exact) <= float(np.spacing(np.float32(exact)))


def test_double_quant_error_bound():
    rng = np.random.default_rng(9)
    absmax = (np.abs(rng.normal(0, 0.02, 3000)) + 1e-4).astype(np.float32)
    q, absmax2, offset, code2 = O.double_quantize(absmax)
    scales = O.resolve_scales(q, absmax2, code2, offset)
    gap = np.diff(code2.astype(np.float64)).max()
    bound = np.repeat(absmax2, 256)[:absmax.size] * gap / 2 + 4 * np.spacing(absmax)
    assert np.all(np.abs(scales.astype(np.float64) - absmax) <= bound)


def test_double_quant_representable_values_decode_exactly():
    """Blocks built from ``v`` (centred value 0, code 0.0), ``v + K_b d`` (centred
    value = the block's absmax2, code 1.0) and ``v - K_b d`` (equal counts, so
    the mean is exactly v) with dyadic v, d: the first two kinds decode to
    themselves exactly, the third to ``fl32(fl32(code2[0] K_b d) + v)``. K_b
    differs per block, so an absmax2 taken from the wrong block fails."""
    v, d = np.float32(0.015625), np.float32(2.0 ** -12)
    code2 = O.dynamic_map()
    blocks = []
    for b in range(6):
        k = np.float32(b + 3)
        blk = np.array([v] * 128 + [v + k * d] * 64 + [v - k * d] * 64, np.float32)
        blocks.append(np.random.default_rng(b).permutation(blk))
    a = np.concatenate(blocks)
    q, absmax2, offset, _ = O.double_quantize(a, code2)
    assert offset == v
    assert np.array_equal(absmax2, (np.arange(6, dtype=np.float32) + 3) * d)
    scales = O.resolve_scales(q, absmax2, code2, offset)
    low = a < v
    assert np.array_equal(scales[~low], a[~low])
    kd = np.repeat(absmax2, 256)[low]
    expect = (np.float32(code2[0]) * kd).astype(np.float32) + v
    assert np.array_equal(scales[low], expect.astype(np.float32))


def test_resolve_scales_two_roundings_match_torch():
    """``dequantize_blockwise(...).float()`` then ``.add_(offset)`` as two fp32
    ops (methods/nf4_backward.py:157-160), restated with torch CPU tensors. The
    inputs include cases where one fused multiply-add would round differently,
    and the test checks that such cases are present."""
    rng = np.random.default_rng(17)
    code2 = O.dynamic_map()
    n = 1 << 16
    q = rng.integers(0, 256, n).astype(np.uint8)
    absmax2 = (np.abs(rng.normal(0, 0.01, n // 256)) + 1e-4).astype(np.float32)
    offset = np.float32(0.0137)
    ours = O.resolve_scales(q, absmax2, code2, offset)
    prod = torch.from_numpy(code2)[torch.from_numpy(q.astype(np.int64))] * \
        torch.from_numpy(absmax2).repeat_interleave(256)
    prod.add_(float(offset))
    assert np.array_equal(ours, prod.numpy())
    fused = (code2[q].astype(np.float64) * np.repeat(absmax2, 256).astype(np.float64)
             + np.float64(offset)).astype(np.float32)
    assert np.count_nonzero(fused != ours) > 0


def test_dynamic_map_linspace_is_torch_fp32():
    for steps in (2, 3, 5, 9, 17, 33, 65, 129):
        ref = torch.linspace(0.1, 1.0, steps, dtype=torch.float32).numpy()
        assert np.array_equal(O.linspace_f32(0.1, 1.0, steps), ref), steps


def test_dynamic_map_closed_form():
    """Entry j of decade i is ``10**(i-6) * (b_j + b_{j+1}) / 2``,
    ``b_j = 0.1 + 0.9 j / 2**i``, within 2 fp32 ulp; decade i holds 2**i
    positive and 2**i negative entries; 0 and 1 are present; 256 entries."""
    m = O.dynamic_map()
    assert m.shape == (256,) and m.dtype == np.float32
    expect = []
    for i in range(7):
        j = np.arange(2 ** i, dtype=np.float64)
        b0, b1 = 0.1 + 0.9 * j / 2 ** i, 0.1 + 0.9 * (j + 1) / 2 ** i
        expect.append(10.0 ** (i - 6) * (b0 + b1) / 2)
    pos = np.concatenate(expect)
    closed = np.sort(np.concatenate([pos, -pos, [0.0, 1.0]]))
    ulp = np.spacing(np.abs(closed).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(m.astype(np.float64) - closed) <= 2 * ulp)
    for i in range(7):
        lo, hi = 10.0 ** (i - 6) * 0.1, 10.0 ** (i - 6)
        assert np.count_nonzero((m > lo) & (m < hi)) == 2 ** i
        assert np.count_nonzero((m < -lo) & (m > -hi)) == 2 ** i
    assert m[-1] == 1.0 and np.count_nonzero(m == 0.0) == 1 and np.all(np.diff(m) > 0)


def _dynamic_map_torch(scale_in_fp64: bool = False) -> np.ndarray:
    """The published ``create_dynamic_map`` construction (bitsandbytes 0.50.2,
    signed, 7 exponent bits, 8 bits) written as torch ops on fp32 tensors: per
    decade an fp32 ``torch.linspace(0.1, 1, 2**i + 1)``, fp32 midpoints, then the
    decade scale ``10**(i-6)`` as a Python float times the fp32 tensor (torch
    rounds the scalar to fp32 and multiplies in fp32), both signs, 0 and 1,
    sorted. ``scale_in_fp64`` is the plausible mistake of scaling in fp64 and
    rounding once afterwards."""
    data = []
    for i in range(7):
        bounds = torch.linspace(0.1, 1, 2 ** i + 1)
        assert bounds.dtype == torch.float32
        means = (bounds[:-1] + bounds[1:]) / 2.0
        if scale_in_fp64:
            vals = (10 ** (i - 6) * means.double()).float()
        else:
            vals = 10 ** (i - 6) * means
        assert vals.dtype == torch.float32
        data += vals.tolist() + (-vals).tolist()
    data += [0.0, 1.0]
    return torch.tensor(data, dtype=torch.float32).sort().values.numpy()


def test_dynamic_map_bitwise_equals_torch_fp32_construction():
    """Bit-for-bit pin of the nested statistics' code table (``state2.code``,
    read by methods/nf4_backward.py:157-160): the oracle's numpy restatement
    (its own linspace, fp32 scalar scale) equals the construction run as torch
    fp32 ops, and the fp64-scale variant, which moves entries by an ulp, does not."""
    ours = O.dynamic_map()
    assert np.array_equal(ours.view(np.uint32), _dynamic_map_torch().view(np.uint32))
    variant = _dynamic_map_torch(scale_in_fp64=True)
    assert np.count_nonzero(variant.view(np.uint32) != ours.view(np.uint32)) > 0


def test_product_dynamic_map_is_the_oracle_table():
    import molt_amd

    assert np.array_equal(molt_amd.dynamic_map().numpy(), O.dynamic_map())


# ----------------------------------------------------- GEMM-level algebra
def _autograd_lora(x, w, a, b, s, dy):
    xt, at, bt = (torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (x, a, b))
    wt = torch.tensor(w, dtype=torch.float64)
    y = xt @ wt.T + s * ((xt @ at.T) @ bt.T)
    y.backward(torch.tensor(dy, dtype=torch.float64))
    return y.detach().numpy(), xt.grad.numpy(), at.grad.numpy(), bt.grad.numpy()


def test_lora_linear_algebra_matches_autograd():
    rng = np.random.default_rng(21)
    m, k, n, r, s = 9, 13, 11, 3, 0.3
    x, w = rng.normal(size=(m, k)), rng.normal(size=(n, k))
    a, b, dy = rng.normal(size=(r, k)), rng.normal(size=(n, r)), rng.normal(size=(m, n))
    y, dx, da, db = _autograd_lora(x, w, a, b, s, dy)
    np.testing.assert_allclose(O.lora_linear_forward(x, w, a, b, s), y, rtol=1e-12, atol=1e-12)
    gx, ga, gb = O.lora_linear_backward(x, w, a, b, s, dy)
    np.testing.assert_allclose(gx, dx, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ga, da, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gb, db, rtol=1e-12, atol=1e-12)


def test_swiglu_matches_torch_silu():
    """kernels/gated_activation.py fp32 closed form vs F.silu autograd; also the
    reference CPU test's tolerance (tests/kernels/test_gated_activation.py:10-26)."""
    rng = np.random.default_rng(3401)
    g, u, dh = (rng.normal(size=(3, 5, 17)) for _ in range(3))
    gt = torch.tensor(g, requires_grad=True)
    ut = torch.tensor(u, requires_grad=True)
    h = torch.nn.functional.silu(gt) * ut
    h.backward(torch.tensor(dh))
    np.testing.assert_allclose(O.swiglu_forward(g, u), h.detach().numpy(), rtol=1e-12, atol=1e-12)
    dg, du = O.swiglu_backward(g, u, dh)
    np.testing.assert_allclose(dg, gt.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(du, ut.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_gated_mlp_algebra_matches_autograd():
    rng = np.random.default_rng(1221)
    m, hd, idim, r, s = 7, 10, 12, 3, 2.0
    x = rng.normal(size=(m, hd))
    wg, wu, wd = rng.normal(size=(idim, hd)), rng.normal(size=(idim, hd)), rng.normal(size=(hd, idim))
    ag, au, ad = rng.normal(size=(r, hd)), rng.normal(size=(r, hd)), rng.normal(size=(r, idim))
    bg, bu, bd = rng.normal(size=(idim, r)), rng.normal(size=(idim, r)), rng.normal(size=(hd, r))
    dy = rng.normal(size=(m, hd))
    T = lambda v, g=True: torch.tensor(v, dtype=torch.float64, requires_grad=g)  # noqa: E731
    xt, agt, aut, adt, bgt, but, bdt = T(x), T(ag), T(au), T(ad), T(bg), T(bu), T(bd)
    wgt, wut, wdt = T(wg, False), T(wu, False), T(wd, False)
    lin = lambda z, w, a, b: z @ w.T + s * ((z @ a.T) @ b.T)  # noqa: E731
    g, u = lin(xt, wgt, agt, bgt), lin(xt, wut, aut, but)
    y = lin(torch.nn.functional.silu(g) * u, wdt, adt, bdt)
    y.backward(torch.tensor(dy))
    yo, saved = O.gated_mlp_forward(x, wg, wu, wd, ag, bg, au, bu, ad, bd, s, bf16_storage=False)
    np.testing.assert_allclose(yo, y.detach().numpy(), rtol=1e-11, atol=1e-11)
    dx, grads = O.gated_mlp_backward(x, wg, wu, wd, ag, bg, au, bu, ad, bd, s, dy, saved, bf16_storage=False)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-10, atol=1e-10)
    for got, ref in zip(grads, (agt, bgt, aut, but, adt, bdt)):
        np.testing.assert_allclose(got, ref.grad.numpy(), rtol=1e-10, atol=1e-10)


def test_rel_fro_detects_a_dropped_lora_term():
    rng = np.random.default_rng(2)
    x, w = rng.normal(size=(32, 64)), rng.normal(size=(48, 64)) * 0.02
    a, b = rng.normal(size=(8, 64)) / 8, rng.normal(size=(48, 8)) * 0.1
    full = O.lora_linear_forward(x, w, a, b, 2.0)
    assert O.rel_fro(x @ w.T, full) > 5e-3


def test_bf16_points_forward_matches_torch_bf16_ops():
    """The reference's autocast forward (methods/nf4_lora.py:43-50) run as torch
    CPU bf16 ops: ``base = bf16(X W^T)``, ``low = F.linear(x, A)``,
    ``base + F.linear(low, B) * s``, every op returning bf16. The restatement
    uses fp64 inner products, torch accumulates in fp32, so a few elements may
    round to the neighbouring bf16 value; a dropped rounding point or term moves
    far more."""
    g = torch.Generator().manual_seed(23)
    m, k, n, r, s = 64, 256, 96, 16, 2.0
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    a = torch.randn(r, k, generator=g) / 16
    b = torch.randn(n, r, generator=g) * 0.01
    base = (x.float() @ w.float().T).to(torch.bfloat16)
    low = torch.nn.functional.linear(x, a.to(torch.bfloat16))
    ref = base + torch.nn.functional.linear(low, b.to(torch.bfloat16)) * s
    assert ref.dtype == torch.bfloat16
    ours = O.lora_linear_forward_bf16_points(x.float().numpy(), w.float().numpy(), a.numpy(), b.numpy(), s)
    ref = ref.float().numpy()
    assert np.mean(ours == ref) >= 0.995
    ulp = np.spacing(O.bf16_round(np.abs(ref))) * 2 ** 16
    assert np.all(np.abs(ours - ref) <= 2 * ulp)
    no_round = O.lora_linear_forward(x.float().numpy(), w.float().numpy(), a.numpy(), b.numpy(), s)
    assert np.mean(O.bf16_round(no_round) == ref) < 0.9


def _autocast_gated_mlp(x, wg, wu, wd, ag, bg, au, bu, ad, bd, s, dy):
    """The reference's gated-MLP step as a torch autograd graph on the CPU under
    bf16 autocast: gate and up as ``F.linear(x, W) + F.linear(F.linear(x, A), B) * s``
    (methods/nf4_lora.py:43-50; the NF4 base as the bf16 dequantised weight),
    ``h = F.silu(g) * u`` and the down projection likewise
    (methods/gated_replay.py:290-299). Autograd's own backward (Mul, SiLU, Linear
    and the autocast casts of the fp32 masters) supplies the rounding points the
    reference's manual backward reproduces (:341-388); the gate and up input
    gradients are summed in bf16, as autograd sums the two nodes' outputs."""
    from torch.nn import functional as F

    leaves = [t.clone().requires_grad_() for t in (ag, bg, au, bu, ad, bd)]
    xg, xu = x.clone().requires_grad_(), x.clone().requires_grad_()

    def proj(z, w, a, b):
        return F.linear(z, w) + F.linear(F.linear(z, a), b) * s

    with torch.autocast("cpu", dtype=torch.bfloat16):
        g = proj(xg, wg, leaves[0], leaves[1])
        u = proj(xu, wu, leaves[2], leaves[3])
        gd, ud = g.detach().requires_grad_(), u.detach().requires_grad_()
        y = proj(F.silu(gd) * ud, wd, leaves[4], leaves[5])
    assert y.dtype == torch.bfloat16
    y.backward(dy)
    g.backward(gd.grad)
    u.backward(ud.grad)
    return y, xg.grad + xu.grad, [leaf.grad for leaf in leaves]


def test_reference_bf16_gated_mlp_matches_torch_autocast_autograd():
    """``lora_linear_backward_bf16_points`` and ``gated_mlp_reference_bf16`` (the
    reference's own bf16 rounding points, used by the GPU tests to report the
    reference path's error beside the HIP path's) against torch's autocast +
    autograd on the CPU: at least 99.9 % of every output's elements equal (the
    restatement's inner products are fp64, torch's fp32). Dropping the bf16
    rounding of dA/dB (the reference widens bf16 products to fp32) fails it."""
    g = torch.Generator().manual_seed(5)
    m, hid, inter, r, s = 64, 128, 256, 16, 2.0
    x = torch.randn(m, hid, generator=g).bfloat16()
    dy = torch.randn(m, hid, generator=g).bfloat16()
    wg, wu = ((torch.randn(inter, hid, generator=g) * 0.05).bfloat16() for _ in range(2))
    wd = (torch.randn(hid, inter, generator=g) * 0.05).bfloat16()
    ag, au = (torch.randn(r, hid, generator=g) / hid ** 0.5 for _ in range(2))
    ad = torch.randn(r, inter, generator=g) / inter ** 0.5
    bg, bu = (torch.randn(inter, r, generator=g) * 0.05 for _ in range(2))
    bd = torch.randn(hid, r, generator=g) * 0.05
    ty, tdx, tgrads = _autocast_gated_mlp(x, wg, wu, wd, ag, bg, au, bu, ad, bd, s, dy)
    f = lambda t: t.detach().float().numpy().astype(np.float64)  # noqa: E731
    args = [f(t) for t in (x, wg, wu, wd, ag, bg, au, bu, ad, bd)]
    oy, odx, ograds = O.gated_mlp_reference_bf16(*args, s, f(dy))
    for name, ours, ref in [("Y", oy, ty), ("dX", odx, tdx)] + list(
            zip(("dAg", "dBg", "dAu", "dBu", "dAd", "dBd"), ograds, tgrads)):
        assert np.mean(ours == f(ref)) >= 0.999, name
    # dA of the down projection without the reference's bf16 rounding
    xo, wdo, ado, bdo = args[0], args[3], args[8], args[9]
    gg = O.bf16_round(O.lora_linear_forward_bf16_points(xo, args[1], args[4], args[5], s)).astype(np.float64)
    uu = O.bf16_round(O.lora_linear_forward_bf16_points(xo, args[2], args[6], args[7], s)).astype(np.float64)
    hh = O.bf16_round(O.bf16_round(gg / (1 + np.exp(-gg))) * uu).astype(np.float64)
    _, dad_unrounded, _ = O.lora_linear_backward(hh, wdo, O.bf16_round(ado), O.bf16_round(bdo), s, f(dy))
    assert np.mean(dad_unrounded == f(tgrads[4])) < 0.5


# --------------------------------------------------------------- RMSNorm
def test_rmsnorm_forward_closed_forms():
    rng = np.random.default_rng(5)
    w = rng.standard_normal(48)
    # a constant row normalises to sign(c) * (w + offset) at eps = 0
    for c in (3.25, -0.5):
        x = np.full((2, 48), c)
        for off in (0.0, 1.0):
            np.testing.assert_allclose(O.rmsnorm_forward(x, w, 0.0, off), np.broadcast_to(np.sign(c) * (w + off), x.shape),
                                       rtol=1e-14, atol=1e-14)
    x = rng.standard_normal((5, 48))
    # scale invariance at eps = 0, and unit RMS of the normalised row
    np.testing.assert_allclose(O.rmsnorm_forward(7.5 * x, w, 0.0, 0.0), O.rmsnorm_forward(x, w, 0.0, 0.0),
                               rtol=1e-13, atol=1e-13)
    n = O.rmsnorm_forward(x, np.zeros(48), 0.0, 1.0)
    np.testing.assert_allclose(np.mean(n * n, axis=-1), 1.0, rtol=1e-13)
    # eps enters under the root: a zero row stays zero, a tiny row is damped
    assert np.all(O.rmsnorm_forward(np.zeros((1, 48)), w, 1e-6, 0.0) == 0.0)
    tiny = np.full((1, 48), 1e-4)
    np.testing.assert_allclose(O.rmsnorm_forward(tiny, np.ones(48), 1e-6, 0.0),
                               1e-4 / math.sqrt(1e-8 + 1e-6), rtol=1e-12)


def test_rmsnorm_backward_matches_central_differences():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 16))
    w = rng.standard_normal(16)
    dy = rng.standard_normal((3, 16))
    for eps, off in ((1e-6, 0.0), (0.3, 1.0)):
        got = O.rmsnorm_backward(x, w, eps, off, dy)
        num = np.zeros_like(x)
        h = 1e-6
        for i in range(x.shape[0]):
            for j in range(x.shape[1]):
                xp, xm = x.copy(), x.copy()
                xp[i, j] += h
                xm[i, j] -= h
                num[i, j] = np.sum(dy * (O.rmsnorm_forward(xp, w, eps, off) - O.rmsnorm_forward(xm, w, eps, off))) / (2 * h)
        np.testing.assert_allclose(got, num, rtol=1e-6, atol=1e-8)
    # at eps = 0 the map is scale invariant, so the gradient is orthogonal to x
    g0 = O.rmsnorm_backward(x, w, 0.0, 0.0, dy)
    np.testing.assert_allclose(np.sum(g0 * x, axis=-1), 0.0, atol=1e-12)


def test_rmsnorm_oracle_matches_reference_test_algebra():
    """The closed form of the reference's own test (tests/kernels/test_frozen_rmsnorm.py:6-53),
    evaluated by torch autograd in fp64."""
    torch.manual_seed(23)
    w = torch.randn(64, dtype=torch.float64)
    x = torch.randn(8, 64, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(8, 64, dtype=torch.float64)
    for off in (0.0, 1.0):
        ref = x * torch.rsqrt(x.square().mean(-1, keepdim=True) + 1e-6) * (w + off)
        (gx,) = torch.autograd.grad(ref, x, dy)
        np.testing.assert_allclose(O.rmsnorm_forward(x.detach().numpy(), w.numpy(), 1e-6, off),
                                   ref.detach().numpy(), rtol=1e-13, atol=1e-13)
        np.testing.assert_allclose(O.rmsnorm_backward(x.detach().numpy(), w.numpy(), 1e-6, off, dy.numpy()),
                                   gx.numpy(), rtol=1e-12, atol=1e-12)


# --------------------------------------------------------------- cross-entropy
def test_cross_entropy_rows_matches_torch_and_differences():
    from torch.nn import functional as F

    rng = np.random.default_rng(8)
    z = rng.standard_normal((6, 37)) * 3.0
    t = rng.integers(0, 37, 6)
    loss, grad = O.cross_entropy_rows(z, t, 6.0)
    zt = torch.tensor(z, requires_grad=True)
    ref = F.cross_entropy(zt, torch.tensor(t), reduction="mean")
    (gref,) = torch.autograd.grad(ref, zt)
    np.testing.assert_allclose(loss.sum(), ref.item(), rtol=1e-13)
    np.testing.assert_allclose(grad, gref.numpy(), rtol=1e-12, atol=1e-15)
    # central differences of the summed loss
    h = 1e-6
    for i, j in ((0, 0), (3, int(t[3])), (5, 36)):
        zp, zm = z.copy(), z.copy()
        zp[i, j] += h
        zm[i, j] -= h
        num = (O.cross_entropy_rows(zp, t, 6.0)[0].sum() - O.cross_entropy_rows(zm, t, 6.0)[0].sum()) / (2 * h)
        np.testing.assert_allclose(grad[i, j], num, rtol=1e-6, atol=2e-9)


def test_cross_entropy_rows_invalid_targets():
    rng = np.random.default_rng(9)
    z = rng.standard_normal((3, 10))
    t = np.array([-100, 10, 4])
    loss, grad = O.cross_entropy_rows(z, t, 3.0)
    assert loss[0] == 0.0 and loss[1] == 0.0 and loss[2] > 0.0
    np.testing.assert_allclose(grad[:2].sum(axis=1), 1.0 / 3.0, rtol=1e-14)
    np.testing.assert_allclose(grad[2].sum(), 0.0, atol=1e-15)
    assert np.all(grad[:2] > 0)
