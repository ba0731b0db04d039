"""NF4-LoRA linear (scheduled forward/backward, packed input gradients) on the
GPU vs the fp64 oracle over the same bf16 operands. Shapes, seeds and scales
follow the reference's tests/kernels/test_nf4_lora.py:14-143."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as O
from tests._util import TOL, assert_close_fro, bf16_values, np_f32, oracle_weight

import molt_amd
from molt_amd.errors import CapabilityError
from molt_amd.methods import (packed_nf4_backward_input, packed_nf4_lora_backward_input, scheduled_nf4_lora)

pytestmark = pytest.mark.gpu


def _problem(width, out_width, rank, tokens, seed, weight_std=1.0, nested=True):
    torch.manual_seed(seed)
    x = torch.randn(1, tokens, width, device="cuda", dtype=torch.bfloat16)
    dense = torch.randn(out_width, width, device="cuda", dtype=torch.bfloat16) * weight_std
    packed, qs = molt_amd.quantize_4bit(dense, blocksize=64, compress_statistics=nested)
    a = torch.randn(rank, width, device="cuda", dtype=torch.float32)
    b = torch.randn(out_width, rank, device="cuda", dtype=torch.float32)
    dy = torch.randn(1, tokens, out_width, device="cuda", dtype=torch.bfloat16)
    return x, packed, qs, a, b, dy


def _oracle(x, packed, qs, a, b, dy, s):
    w = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    xo = bf16_values(x).reshape(-1, w.shape[1])
    ao, bo = bf16_values(a), bf16_values(b)
    dyo = bf16_values(dy).reshape(-1, w.shape[0])
    y = O.lora_linear_forward(xo, w, ao, bo, s)
    dx, da, db = O.lora_linear_backward(xo, w, ao, bo, s, dyo)
    return y, dx, da, db


def _run(x, packed, qs, a, b, dy, s, cached=None):
    xr = x.detach().clone().requires_grad_()
    ar = a.detach().clone().requires_grad_()
    br = b.detach().clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = scheduled_nf4_lora(xr, packed, ar, br, qs, s, cached)
    y.backward(dy)
    return y, xr.grad, ar.grad, br.grad


@pytest.mark.parametrize("width,out_width", [(64, 96), (1536, 256), (1536, 1536), (1536, 8960), (8960, 1536)])
@pytest.mark.parametrize("scale", [0.125, 0.3, 2.0])
def test_scheduled_nf4_lora_matches_oracle(width, out_width, scale):
    print(f"scheduled_nf4_lora {width}->{out_width} scale={scale}", flush=True)
    x, packed, qs, a, b, dy = _problem(width, out_width, 8, 256, 941)
    y, dx, da, db = _run(x, packed, qs, a, b, dy, scale)
    ry, rdx, rda, rdb = _oracle(x, packed, qs, a, b, dy, scale)
    assert y.dtype == torch.bfloat16 and dx.dtype == torch.bfloat16
    assert da.dtype == torch.float32 and db.dtype == torch.float32
    assert_close_fro(np_f32(y).reshape(ry.shape), ry, what="Y")
    assert_close_fro(np_f32(dx).reshape(rdx.shape), rdx, what="dX")
    assert_close_fro(np_f32(da), rda, what="dA")
    assert_close_fro(np_f32(db), rdb, what="dB")


@pytest.mark.parametrize("width,out_width,rank,tokens", [(70, 65, 7, 5), (65, 70, 3, 33), (4096, 1024, 64, 130),
                                                         (896, 4864, 16, 1024), (128, 64, 1, 1)])
def test_scheduled_nf4_lora_tails_and_ranks(width, out_width, rank, tokens):
    print(f"tails {width}->{out_width} r={rank} M={tokens}", flush=True)
    x, packed, qs, a, b, dy = _problem(width, out_width, rank, tokens, 942, weight_std=0.02)
    y, dx, da, db = _run(x, packed, qs, a, b, dy, 2.0)
    ry, rdx, rda, rdb = _oracle(x, packed, qs, a, b, dy, 2.0)
    assert_close_fro(np_f32(y).reshape(ry.shape), ry, what="Y")
    assert_close_fro(np_f32(dx).reshape(rdx.shape), rdx, what="dX")
    assert_close_fro(np_f32(da), rda, what="dA")
    assert_close_fro(np_f32(db), rdb, what="dB")


@pytest.mark.parametrize("width,out_width", [(1536, 256), (1536, 8960), (8960, 1536)])
def test_scheduled_error_beside_the_reference_bf16_path(width, out_width):
    """The HIP linear's relative Frobenius error against the fp64 oracle, printed
    beside the error of the reference's own autocast step on the same operands
    (``lora_linear_forward_bf16_points`` / ``lora_linear_backward_bf16_points``,
    methods/nf4_lora.py:43-50,83-109). The HIP path may not be worse than 1.5x
    the reference's error on Y, dX, dA or dB."""
    s = 2.0
    x, packed, qs, a, b, dy = _problem(width, out_width, 16, 512, 946, weight_std=0.02)
    got = _run(x, packed, qs, a, b, dy, s)
    ref = _oracle(x, packed, qs, a, b, dy, s)
    w = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    xo = bf16_values(x).reshape(-1, width)
    dyo = bf16_values(dy).reshape(-1, out_width)
    ao, bo = np_f32(a).astype(np.float64), np_f32(b).astype(np.float64)
    emul = (O.lora_linear_forward_bf16_points(xo, w, ao, bo, s),) + O.lora_linear_backward_bf16_points(
        xo, w, ao, bo, s, dyo)
    print(f"scheduled {width}->{out_width} r=16 M=512: relative Frobenius error vs fp64 (HIP / reference bf16)",
          flush=True)
    for name, g, e, o in zip(("Y", "dX", "dA", "dB"), got, emul, ref):
        eh, ee = O.rel_fro(np_f32(g).reshape(o.shape), o), O.rel_fro(e, o)
        print(f"  {name:3s} {eh:10.3e} {ee:10.3e}", flush=True)
        assert eh <= TOL and eh <= 1.5 * ee, f"{name}: HIP {eh:.3e}, reference bf16 {ee:.3e}"


def test_cached_backward_weight_is_bitwise_equal_to_per_call_decode():
    """tests/kernels/test_nf4_lora.py:48-79."""
    x, packed, qs, a, b, dy = _problem(1536, 1536, 8, 256, 944)
    decoded = molt_amd.dequantize_4bit(packed, qs).to(torch.bfloat16)
    left = _run(x, packed, qs, a, b, dy, 2.0)
    right = _run(x, packed, qs, a, b, dy, 2.0, decoded)
    for lt, rt in zip(left, right):
        assert torch.equal(lt, rt)


def test_repeat_runs_are_bitwise_deterministic():
    x, packed, qs, a, b, dy = _problem(1536, 8960, 16, 512, 945, weight_std=0.02)
    first = _run(x, packed, qs, a, b, dy, 2.0)
    second = _run(x, packed, qs, a, b, dy, 2.0)
    for lt, rt in zip(first, second):
        assert torch.equal(lt, rt)


def test_packed_nf4_backward_handles_dimension_tails():
    """tests/kernels/test_nf4_lora.py:106-121 against the oracle."""
    torch.manual_seed(942)
    dense = torch.randn(70, 65, device="cuda", dtype=torch.bfloat16)
    packed, qs = molt_amd.quantize_4bit(dense, blocksize=64, compress_statistics=True)
    grad = torch.randn(5, 70, device="cuda", dtype=torch.bfloat16)
    actual = packed_nf4_backward_input(grad, packed, qs)
    w = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    assert_close_fro(np_f32(actual), bf16_values(grad) @ w, what="dX")


def test_fused_packed_nf4_lora_backward_handles_rank_and_dimension_tails():
    """tests/kernels/test_nf4_lora.py:124-143 against the oracle (no rank limit)."""
    torch.manual_seed(943)
    dense = torch.randn(70, 65, device="cuda", dtype=torch.bfloat16)
    packed, qs = molt_amd.quantize_4bit(dense, blocksize=64, compress_statistics=True)
    w = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    for rank in (7, 40):
        grad = torch.randn(5, 70, device="cuda", dtype=torch.bfloat16)
        lora_grad = torch.randn(5, rank, device="cuda", dtype=torch.bfloat16)
        lora_a = torch.randn(rank, 65, device="cuda", dtype=torch.float32)
        actual = packed_nf4_lora_backward_input(grad, packed, qs, lora_grad, lora_a, 0.125)
        ref = bf16_values(grad) @ w + 0.125 * (bf16_values(lora_grad) @ bf16_values(lora_a))
        assert_close_fro(np_f32(actual), ref, what=f"dX r={rank}")


def test_cleanroom_layout_through_scheduled_path():
    """Low-nibble-first fp32-scale weights (streaming/nf4.py) through the same GEMMs."""
    torch.manual_seed(5)
    dense = torch.randn(96, 128, device="cuda", dtype=torch.float32) * 0.02
    packed, qs = molt_amd.quantize_4bit(dense, blocksize=64, compress_statistics=False, nibble_order=0)
    x = torch.randn(40, 128, device="cuda", dtype=torch.bfloat16)
    a = torch.randn(4, 128, device="cuda") / 11
    b = torch.randn(96, 4, device="cuda") * 0.01
    dy = torch.randn(40, 96, device="cuda", dtype=torch.bfloat16)
    y, dx, da, db = _run(x, packed, qs, a, b, dy, 2.0)
    ry, rdx, rda, rdb = _oracle(x, packed, qs, a, b, dy, 2.0)
    assert_close_fro(np_f32(y), ry, what="Y")
    assert_close_fro(np_f32(dx), rdx, what="dX")
    assert_close_fro(np_f32(da), rda, what="dA")
    assert_close_fro(np_f32(db), rdb, what="dB")


def test_preconditions_raise_like_the_reference():
    x, packed, qs, a, b, dy = _problem(64, 96, 8, 4, 1)
    with pytest.raises(CapabilityError, match="FP32 adapter masters"):
        scheduled_nf4_lora(x, packed, a.to(torch.bfloat16), b, qs, 1.0)
    trainable = torch.nn.Parameter(packed.float(), requires_grad=True)
    with pytest.raises(CapabilityError, match="frozen"):
        scheduled_nf4_lora(x, trainable, a, b, qs, 1.0)
    with pytest.raises(CapabilityError, match="cached NF4 backward weight"):
        scheduled_nf4_lora(x, packed, a, b, qs, 1.0, torch.zeros(3, 3, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="gradient width"):
        packed_nf4_backward_input(torch.randn(2, 5, device="cuda", dtype=torch.bfloat16), packed, qs)
    with pytest.raises(CapabilityError, match="BF16"):
        packed_nf4_backward_input(torch.randn(2, 96, device="cuda"), packed, qs)


def test_custom_ops_pass_opcheck():
    from molt_amd import ops

    x, packed, qs, a, b, dy = _problem(128, 64, 4, 16, 3, weight_std=0.02)
    scales = molt_amd.resolved_nf4_scales(qs)
    flat = x.reshape(-1, 128)
    t = ops.lora_project(flat, None, 0, 1.0, a, 0)
    torch.library.opcheck(ops.lora_project, (flat, None, 0, 1.0, a, 0))
    torch.library.opcheck(ops.nf4_lora_forward, (flat, packed.reshape(-1), scales, qs.code, 64, 128, 1, 64, t, b, 2.0))
    torch.library.opcheck(ops.lora_grad, (flat, None, 0, t, 1.0, 1))
    torch.library.opcheck(ops.nf4_dequantize, (packed.reshape(-1), scales, qs.code, 64, 128, 64, 1, torch.bfloat16))
    assert TOL == 5e-3


def test_ops_refuse_host_statistics_and_short_operands():
    """Host-side refusals before any launch: statistics on the CPU, too few
    block scales, and low-rank operands whose rows do not match the tokens."""
    from molt_amd import ops

    x, packed, qs, a, b, dy = _problem(128, 64, 4, 16, 4, weight_std=0.02)
    flat = x.reshape(-1, 128)
    scales = molt_amd.resolved_nf4_scales(qs)
    t = ops.lora_project(flat, None, 0, 1.0, a, 0)
    p = packed.reshape(-1)
    with pytest.raises(CapabilityError, match="CUDA"):
        ops.nf4_lora_forward(flat, p, scales.cpu(), qs.code, 64, 128, 1, 64, t, b, 2.0)
    with pytest.raises(ValueError, match="block scales"):
        ops.nf4_lora_forward(flat, p, scales[:-1], qs.code, 64, 128, 1, 64, t, b, 2.0)
    with pytest.raises(ValueError, match="rows"):
        ops.nf4_lora_forward(flat, p, scales, qs.code, 64, 128, 1, 64, t[:-1], b, 2.0)
    with pytest.raises(CapabilityError, match="CUDA"):
        ops.nf4_gateup_forward(flat, p, scales, p, scales, qs.code, 64, 128, 1,
                               torch.cat([t, t], 1), b.cpu(), b, 2.0, 2.0)
    with pytest.raises(ValueError, match="rows"):
        ops.nf4_lora_backward_input(dy.reshape(-1, 64), p, scales, qs.code, 64, 128, 1, 64,
                                    t[:3], a, 1.0)
    s2 = qs.state2
    with pytest.raises(CapabilityError, match="CUDA"):
        ops.nf4_gemv(flat[:1], p, None, qs.absmax.cpu(), s2.absmax, s2.code, float(qs.offset), 256, qs.code,
                     64, 128, 1, None, None, 1.0)
    with pytest.raises(ValueError, match="second-level"):
        ops.nf4_gemv(flat[:1], p, None, qs.absmax, s2.absmax[:0], s2.code, float(qs.offset), 256, qs.code,
                     64, 128, 1, None, None, 1.0)
    with pytest.raises(ValueError, match="rows"):
        ops.nf4_gemv(flat[:2], p, None, qs.absmax, s2.absmax, s2.code, float(qs.offset), 256, qs.code,
                     64, 128, 1, t[:1], b, 1.0)
