"""Frozen RMSNorm (forward, backward) and the gated MLP's RMSNorm-replay recipe
on the GPU vs the fp64 oracle, plus the reference's own RMSNorm tests
(tests/kernels/test_frozen_rmsnorm.py:6-53) restated on the GPU."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch
from torch import nn

from oracle import nf4_oracle as O
from tests._util import assert_close_fro, bf16_values, np_f32, oracle_weight, seeded, uniform

import molt_amd
from molt_amd import _lib, ops
from molt_amd.errors import CapabilityError
from molt_amd.kernels import FrozenRMSNormBF16
from molt_amd.kernels.frozen_rmsnorm import _FrozenRMSNormFunction
from molt_amd.methods import enable_fused_gated_nf4_lora, enable_rmsnorm_replay, fused_gated_nf4_lora_mlp
from molt_amd.methods.gated_replay import _ResidualRecipeGatedNF4LoRA, _RMSNormReplayRecipe
from molt_amd.modules import GatedMLP, NF4Linear, NF4LoRALinear

pytestmark = pytest.mark.gpu


def _values(t: torch.Tensor) -> np.ndarray:
    return np_f32(t).astype(np.float64)


def _within_one_bf16_ulp(got: np.ndarray, ref: np.ndarray) -> None:
    """|got - ref| <= one bf16 ulp of ref (2^-7 |ref|, plus the subnormal floor)."""
    bound = np.abs(ref) * 2.0 ** -7 + 1e-38
    bad = np.abs(got - ref) > bound
    assert not bad.any(), f"{bad.sum()} elements beyond one bf16 ulp (first at {np.argwhere(bad)[0]})"


@pytest.mark.parametrize("m,h,x_dtype,w_dtype,offset", [
    (8, 64, torch.bfloat16, torch.float32, 0.0),
    (257, 4096, torch.bfloat16, torch.bfloat16, 0.0),
    (33, 896, torch.float32, torch.float32, 1.0),
    (5, 70, torch.bfloat16, torch.float32, 1.0),     # H % 8 != 0: one element per access
    (1, 8192, torch.float32, torch.bfloat16, 0.0),
])
def test_rmsnorm_forward_matches_oracle(m, h, x_dtype, w_dtype, offset):
    print(f"rmsnorm fwd M={m} H={h} x={x_dtype} w={w_dtype} off={offset}", flush=True)
    x = seeded((m, h), 1, std=1.7, dtype=x_dtype)
    w = seeded((h,), 2, std=0.3, dtype=w_dtype)
    y = ops.rmsnorm_forward(x, w, 1e-6, offset)
    assert y.dtype == torch.bfloat16 and y.shape == x.shape
    ref = O.rmsnorm_forward(_values(x), _values(w), 1e-6, offset)
    got = _values(y)
    _within_one_bf16_ulp(got, ref)
    exact = np.mean(O.bf16_round(ref.astype(np.float32)).astype(np.float64) == got)
    assert exact >= 0.99, f"only {exact:.4f} of outputs equal bf16(oracle)"


@pytest.mark.parametrize("m,h,x_dtype,w_dtype,offset", [
    (8, 64, torch.bfloat16, torch.float32, 0.0),
    (257, 4096, torch.bfloat16, torch.bfloat16, 1.0),
    (33, 896, torch.float32, torch.float32, 0.0),
    (5, 70, torch.float32, torch.bfloat16, 1.0),
])
def test_rmsnorm_backward_matches_oracle(m, h, x_dtype, w_dtype, offset):
    print(f"rmsnorm bwd M={m} H={h} x={x_dtype} w={w_dtype} off={offset}", flush=True)
    x = seeded((m, h), 3, std=0.8, dtype=x_dtype)
    w = seeded((h,), 4, std=0.5, dtype=w_dtype)
    dy = seeded((m, h), 5)
    dx = ops.rmsnorm_backward(dy, x, w, 1e-5, offset)
    assert dx.dtype == x_dtype and dx.shape == x.shape
    ref = O.rmsnorm_backward(_values(x), _values(w), 1e-5, offset, _values(dy))
    if x_dtype == torch.float32:
        assert_close_fro(_values(dx), ref, tol=1e-5, what="dx fp32")
    else:
        assert_close_fro(_values(dx), ref, what="dx bf16")


def test_rmsnorm_strided_rows_through_the_abi():
    """Row strides larger than H (a view into a wider buffer), called through the C ABI."""
    m, h, ld = 12, 512, 520
    buf = seeded((m, ld), 6)
    w = seeded((h,), 7, dtype=torch.float32)
    out = torch.full((m, ld), 7.0, dtype=torch.bfloat16, device="cuda")
    ops._call("molt_rmsnorm_forward", buf.data_ptr(), _lib.DTYPE_BF16, ld, m, h, w.data_ptr(), _lib.DTYPE_F32,
              1e-6, 0.0, out.data_ptr(), ld, None, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    dense = ops.rmsnorm_forward(buf[:, :h].contiguous(), w, 1e-6, 0.0)
    assert torch.equal(out[:, :h], dense)
    assert torch.all(out[:, h:] == 7.0), "wrote past H"
    inv = torch.empty(m, dtype=torch.float32, device="cuda")
    ops._call("molt_rmsnorm_forward", buf.data_ptr(), _lib.DTYPE_BF16, ld, m, h, w.data_ptr(), _lib.DTYPE_F32,
              1e-6, 0.0, out.data_ptr(), ld, inv.data_ptr(), torch.cuda.current_stream().cuda_stream)
    xo = _values(buf[:, :h])
    np.testing.assert_allclose(np_f32(inv), 1.0 / np.sqrt(np.mean(xo * xo, axis=-1) + 1e-6), rtol=2e-6)


def test_rmsnorm_edge_cases_and_errors():
    w = torch.ones(16, device="cuda")
    assert ops.rmsnorm_forward(torch.empty(0, 16, dtype=torch.bfloat16, device="cuda"), w, 1e-6, 0.0).shape == (0, 16)
    z = ops.rmsnorm_forward(torch.zeros(3, 16, dtype=torch.bfloat16, device="cuda"), w, 1e-6, 0.0)
    assert torch.all(z == 0)
    with pytest.raises(ValueError):
        ops.rmsnorm_forward(torch.zeros(3, 16, dtype=torch.bfloat16, device="cuda"), torch.ones(8, device="cuda"),
                            1e-6, 0.0)
    with pytest.raises(CapabilityError):
        ops.rmsnorm_forward(torch.zeros(3, 16, dtype=torch.float16, device="cuda"), w, 1e-6, 0.0)
    with pytest.raises(CapabilityError):
        ops.rmsnorm_forward(torch.zeros(3, 16, dtype=torch.bfloat16), w.cpu(), 1e-6, 0.0)
    with pytest.raises(ValueError, match="frozen weight"):
        _FrozenRMSNormFunction.apply(torch.zeros(3, 16, dtype=torch.bfloat16, device="cuda"),
                                     w.clone().requires_grad_(), 1e-6, 0.0)
    lib = _lib.load()
    rc = lib.molt_rmsnorm_forward(None, 7, 16, 3, 16, None, 1, C.c_float(1e-6), C.c_float(0.0), None, 16, None, None)
    assert rc == 1 and b"dtype" in lib.molt_amd_last_error()


# ------------------------------------- the reference's own tests, on the GPU
def test_frozen_rmsnorm_preserves_bf16_contract_and_reference_gradient():
    """tests/kernels/test_frozen_rmsnorm.py:6-23."""
    torch.manual_seed(23)
    weight = torch.randn(64, dtype=torch.float32)
    candidate_input = torch.randn(8, 64, dtype=torch.bfloat16).cuda().requires_grad_(True)
    reference_input = candidate_input.detach().float().cpu().requires_grad_(True)
    gradient = torch.randn(8, 64, dtype=torch.bfloat16)

    candidate = _FrozenRMSNormFunction.apply(candidate_input, weight.cuda(), 1e-6, 0.0)
    reference_inverse = torch.rsqrt(reference_input.square().mean(-1, keepdim=True) + 1e-6)
    reference = reference_input * reference_inverse * weight
    candidate.backward(gradient.cuda())
    reference.backward(gradient.float())

    assert candidate.dtype == torch.bfloat16
    torch.testing.assert_close(candidate.float().cpu(), reference, rtol=8e-3, atol=8e-3)
    torch.testing.assert_close(candidate_input.grad.float().cpu(), reference_input.grad, rtol=1.5e-2, atol=1.5e-2)


def test_gemma_weight_offset_preserves_reference_gradient():
    """tests/kernels/test_frozen_rmsnorm.py:26-42."""
    torch.manual_seed(24)
    weight = torch.randn(32, dtype=torch.float32)
    candidate_input = torch.randn(4, 32, dtype=torch.bfloat16).cuda().requires_grad_(True)
    reference_input = candidate_input.detach().float().cpu().requires_grad_(True)
    gradient = torch.randn(4, 32, dtype=torch.bfloat16)

    candidate = _FrozenRMSNormFunction.apply(candidate_input, weight.cuda(), 1e-6, 1.0)
    inverse = torch.rsqrt(reference_input.square().mean(-1, keepdim=True) + 1e-6)
    reference = reference_input * inverse * (1.0 + weight)
    candidate.backward(gradient.cuda())
    reference.backward(gradient.float())

    torch.testing.assert_close(candidate.float().cpu(), reference, rtol=8e-3, atol=8e-3)
    torch.testing.assert_close(candidate_input.grad.float().cpu(), reference_input.grad, rtol=1.5e-2, atol=1.5e-2)


def test_frozen_rmsnorm_converts_fp32_residual_to_bf16_without_losing_fp32_gradient():
    """tests/kernels/test_frozen_rmsnorm.py:45-53."""
    torch.manual_seed(25)
    weight = torch.randn(32, dtype=torch.float32).cuda()
    hidden = torch.randn(3, 32, dtype=torch.float32).cuda().requires_grad_(True)
    output = _FrozenRMSNormFunction.apply(hidden, weight, 1e-6, 0.0)

    assert output.dtype == torch.bfloat16
    output.float().sum().backward()
    assert hidden.grad is not None
    assert hidden.grad.dtype == torch.float32


# ------------------------------------------------ residual-recipe gated MLP
def _proj(out_f, in_f, r, seed):
    w = seeded((out_f, in_f), seed, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    a = uniform((r, in_f), seed + 1, 1.0 / np.sqrt(in_f))
    b = seeded((out_f, r), seed + 2, std=0.01, dtype=torch.float32)
    return packed, qs, a, b


class _PlainRMSNorm(nn.Module):
    def __init__(self, weight: torch.Tensor, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(weight, requires_grad=False)
        self.variance_epsilon = eps


@pytest.mark.parametrize("hidden,inter,r,m,offset", [(128, 256, 8, 64, 0.0), (256, 448, 16, 200, 1.0)])
def test_residual_recipe_matches_fused_mlp_and_oracle(hidden, inter, r, m, offset):
    print(f"residual recipe H={hidden} I={inter} r={r} M={m} off={offset}", flush=True)
    s, eps = 2.0, 1e-6
    projs = [_proj(inter, hidden, r, 10), _proj(inter, hidden, r, 20), _proj(hidden, inter, r, 30)]
    (pg, qg, ag, bg), (pu, qu, au, bu), (pd, qd, ad, bd) = projs
    norm_w = seeded((hidden,), 50, std=0.2)
    source = seeded((m, hidden), 51, std=1.5).requires_grad_()
    dy = seeded((m, hidden), 52)

    leaves = [t.clone().requires_grad_() for t in (ag, bg, au, bu, ad, bd)]
    normalized = _FrozenRMSNormFunction.apply(source, norm_w, eps, offset)
    y = _ResidualRecipeGatedNF4LoRA.apply(source, normalized, pg, leaves[0], leaves[1], pu, leaves[2], leaves[3],
                                          pd, leaves[4], leaves[5], qg, qu, qd, s, s, s, norm_w, eps, offset)
    y.backward(dy)

    # the same MLP on a detached copy of the normalised input, through the fused node
    x2 = normalized.detach().clone().requires_grad_()
    leaves2 = [t.clone().requires_grad_() for t in (ag, bg, au, bu, ad, bd)]
    y2 = fused_gated_nf4_lora_mlp(x2, pg, leaves2[0], leaves2[1], pu, leaves2[2], leaves2[3], pd, leaves2[4],
                                  leaves2[5], qg, qu, qd, s, s, s)
    y2.backward(dy)
    assert torch.equal(y, y2)
    for a, b in zip(leaves, leaves2):
        assert torch.equal(a.grad, b.grad)
    # the replayed input is bitwise the norm's forward output
    replay = _RMSNormReplayRecipe(source.detach(), norm_w, eps, offset).materialize()
    assert torch.equal(replay, normalized.detach())

    # end to end against the fp64 oracle: residual -> norm -> MLP -> norm backward
    xs = bf16_values(source)
    wn = bf16_values(norm_w)
    xn = O.bf16_round(O.rmsnorm_forward(xs, wn, eps, offset).astype(np.float32)).astype(np.float64)
    ws = [oracle_weight(p, q).dequant_bf16().astype(np.float64) for p, q, _, _ in projs]
    av = [bf16_values(t) for t in (ag, bg, au, bu, ad, bd)]
    ry, saved = O.gated_mlp_forward(xn, ws[0], ws[1], ws[2], av[0], av[1], av[2], av[3], av[4], av[5], s)
    rdx, rgrads = O.gated_mlp_backward(xn, ws[0], ws[1], ws[2], av[0], av[1], av[2], av[3], av[4], av[5], s,
                                       bf16_values(dy), saved)
    rds = O.rmsnorm_backward(xs, wn, eps, offset, O.bf16_round(rdx.astype(np.float32)).astype(np.float64))
    assert_close_fro(np_f32(y), ry, what="Y")
    assert_close_fro(np_f32(source.grad), rds, what="d_source")
    for leaf, ref, name in zip(leaves, rgrads, ("dA_gate", "dB_gate", "dA_up", "dB_up", "dA_down", "dB_down")):
        assert_close_fro(np_f32(leaf.grad), ref, what=name)


@pytest.mark.parametrize("m,h,q,w_dtype,offset", [
    (200, 256, 32, torch.bfloat16, 0.0),
    (77, 1536, 16, torch.float32, 1.0),
    (1, 64, 8, torch.bfloat16, 0.0),
    (8192, 4096, 128, torch.bfloat16, 0.0),   # cfg4: the gate/up adapters' dA
])
def test_norm_replay_gradient_is_bitwise_the_materialised_one(m, h, q, w_dtype, offset):
    """The gate/up dA over the RMSNorm output formed as it is staged
    (molt_lora_grad_rmsnorm) equals lora_grad over the materialised output,
    and rmsnorm_inv is the scale the forward kernel applies."""
    print(f"norm-replay dA m={m} h={h} q={q} w={w_dtype} off={offset}", flush=True)
    eps = 1e-5
    x = seeded((m, h), 81, std=1.3)
    w = seeded((h,), 82, std=0.3).to(w_dtype)
    u = seeded((m, q), 83)
    inv = ops.rmsnorm_inv(x, w, eps)
    n = ops.rmsnorm_forward(x, w, eps, offset)
    assert torch.equal(n, ((x.float() * inv[:, None]) * (w.float() + offset)).to(torch.bfloat16))
    for scale, layout in ((1.0, 1), (0.5, 0)):
        got = ops.lora_grad_rmsnorm(x, inv, w, offset, u, scale, layout)
        ref = ops.lora_grad(n, None, 0, u, scale, layout)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"layout {layout}: max |diff| {(got - ref).abs().max().item()}"


def test_norm_replay_gradient_of_no_tokens_is_zero():
    x = torch.empty(0, 64, dtype=torch.bfloat16, device="cuda")
    u = torch.empty(0, 8, dtype=torch.bfloat16, device="cuda")
    w = torch.ones(64, dtype=torch.bfloat16, device="cuda")
    inv = ops.rmsnorm_inv(x, w, 1e-6)
    assert inv.shape == (0,)
    g = ops.lora_grad_rmsnorm(x, inv, w, 0.0, u, 1.0, 1)
    assert torch.equal(g, torch.zeros(8, 64, device="cuda"))


def test_residual_recipe_with_fp32_source_materialises_and_matches_fused_mlp():
    """An fp32 residual takes the materialising replay; results stay bitwise
    those of the fused node on the norm's output."""
    hidden, inter, r, m, s, eps = 128, 256, 8, 96, 2.0, 1e-6
    projs = [_proj(inter, hidden, r, 10), _proj(inter, hidden, r, 20), _proj(hidden, inter, r, 30)]
    (pg, qg, ag, bg), (pu, qu, au, bu), (pd, qd, ad, bd) = projs
    norm_w = seeded((hidden,), 50, std=0.2)
    source = seeded((m, hidden), 51, std=1.5, dtype=torch.float32).requires_grad_()
    dy = seeded((m, hidden), 52)
    leaves = [t.clone().requires_grad_() for t in (ag, bg, au, bu, ad, bd)]
    normalized = _FrozenRMSNormFunction.apply(source, norm_w, eps, 0.0)
    y = _ResidualRecipeGatedNF4LoRA.apply(source, normalized, pg, leaves[0], leaves[1], pu, leaves[2], leaves[3],
                                          pd, leaves[4], leaves[5], qg, qu, qd, s, s, s, norm_w, eps, 0.0)
    y.backward(dy)
    x2 = normalized.detach().clone().requires_grad_()
    leaves2 = [t.clone().requires_grad_() for t in (ag, bg, au, bu, ad, bd)]
    y2 = fused_gated_nf4_lora_mlp(x2, pg, leaves2[0], leaves2[1], pu, leaves2[2], leaves2[3], pd, leaves2[4],
                                  leaves2[5], qg, qu, qd, s, s, s)
    y2.backward(dy)
    assert torch.equal(y, y2)
    for a, b in zip(leaves, leaves2):
        assert torch.equal(a.grad, b.grad)
    assert source.grad.dtype == torch.float32 and torch.isfinite(source.grad).all()


class _DecoderTail(nn.Module):
    """residual + mlp(post_attention_layernorm(residual)), as a decoder layer's second half."""

    def __init__(self, norm: nn.Module, mlp: nn.Module) -> None:
        super().__init__()
        self.post_attention_layernorm = norm
        self.mlp = mlp

    def forward(self, residual: torch.Tensor) -> torch.Tensor:
        return residual + self.mlp(self.post_attention_layernorm(residual))


def _tail(hidden, inter, r, offset):
    torch.manual_seed(77)
    projs = []
    for out_f, in_f, seed in ((inter, hidden, 60), (inter, hidden, 61), (hidden, inter, 62)):
        base = NF4Linear.from_dense(seeded((out_f, in_f), seed, std=0.02, dtype=torch.float32))
        lin = NF4LoRALinear(base, r, 2.0 * r)
        nn.init.normal_(lin.lora_B["default"].weight, std=0.01)
        projs.append(lin)
    norm = FrozenRMSNormBF16(_PlainRMSNorm(seeded((hidden,), 63, std=0.2), 1e-6), weight_offset=offset)
    return _DecoderTail(norm, GatedMLP(*projs))


def test_enable_rmsnorm_replay_routes_the_mlp_through_the_recipe():
    hidden, inter, r, m = 128, 256, 8, 96
    plain, wired = _tail(hidden, inter, r, 1.0), _tail(hidden, inter, r, 1.0)
    assert enable_fused_gated_nf4_lora(plain) == 1
    assert enable_fused_gated_nf4_lora(wired) == 1
    assert enable_rmsnorm_replay(wired) == 1
    outs, grads = [], []
    for layer in (plain, wired):
        residual = seeded((m, hidden), 64).requires_grad_()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            mlp_out = layer.mlp(layer.post_attention_layernorm(residual))
            out = residual + mlp_out
        names = type(mlp_out.grad_fn).__name__
        assert ("ResidualRecipe" in names) == (layer is wired), names
        out.backward(seeded((m, hidden), 65))
        outs.append(out.detach())
        grads.append([residual.grad] + [p.grad for n, p in layer.named_parameters() if p.requires_grad])
    assert torch.equal(outs[0], outs[1])
    for a, b in zip(grads[0], grads[1]):
        assert torch.equal(a, b)
    assert wired.mlp._molt_norm_replay_recipe is None, "the recipe must not outlive its forward"
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        wired(seeded((4, hidden), 66))
    assert wired.mlp._molt_norm_replay_recipe is None
