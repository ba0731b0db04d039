"""Gated NF4-LoRA MLP (fused gate/up/down node and the reference's asymmetric
replay API) and the SwiGLU elementwise op on the GPU vs the fp64 oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from oracle import nf4_oracle as O
from tests._util import assert_close_fro, bf16_values, np_f32, oracle_weight, seeded, uniform

import molt_amd
from molt_amd.kernels import fused_silu_multiply
from molt_amd.methods import asymmetric_gated_nf4_lora, fused_gated_nf4_lora_mlp, scheduled_nf4_lora

pytestmark = pytest.mark.gpu


def _proj(out_f, in_f, r, seed, std=0.02):
    w = seeded((out_f, in_f), seed, std=std, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    a = uniform((r, in_f), seed + 1, 1.0 / np.sqrt(in_f))
    b = seeded((out_f, r), seed + 2, std=0.01, dtype=torch.float32)
    return packed, qs, a, b


def _oracle_mlp(x, projs, s, dy):
    ws = [oracle_weight(p, q).dequant_bf16().astype(np.float64) for p, q, _, _ in projs]
    ad = [bf16_values(a) for _, _, a, _ in projs]
    bd = [bf16_values(b) for _, _, _, b in projs]
    xo = bf16_values(x).reshape(-1, ws[0].shape[1])
    dyo = bf16_values(dy).reshape(-1, ws[2].shape[0])
    y, saved = O.gated_mlp_forward(xo, ws[0], ws[1], ws[2], ad[0], bd[0], ad[1], bd[1], ad[2], bd[2], s)
    dx, grads = O.gated_mlp_backward(xo, ws[0], ws[1], ws[2], ad[0], bd[0], ad[1], bd[1], ad[2], bd[2], s, dyo,
                                     saved)
    return y, dx, grads


@pytest.mark.parametrize("hidden,inter,r,m", [(64, 96, 8, 32), (128, 256, 8, 32), (896, 4864, 16, 1024),
                                              (256, 448, 64, 200)])
def test_fused_gated_mlp_matches_oracle(hidden, inter, r, m):
    print(f"fused gated MLP H={hidden} I={inter} r={r} M={m}", flush=True)
    s = 2.0
    projs = [_proj(inter, hidden, r, 10), _proj(inter, hidden, r, 20), _proj(hidden, inter, r, 30)]
    x = seeded((m, hidden), 40).requires_grad_()
    dy = seeded((m, hidden), 41)
    leaves = []
    for _, _, a, b in projs:
        leaves += [a.clone().requires_grad_(), b.clone().requires_grad_()]
    (pg, qg, _, _), (pu, qu, _, _), (pd, qd, _, _) = projs
    y = fused_gated_nf4_lora_mlp(x, pg, leaves[0], leaves[1], pu, leaves[2], leaves[3], pd, leaves[4], leaves[5],
                                 qg, qu, qd, s, s, s)
    y.backward(dy)
    ry, rdx, rgrads = _oracle_mlp(x, projs, s, dy)
    assert_close_fro(np_f32(y), ry, what="Y")
    assert_close_fro(np_f32(x.grad), rdx, what="dX")
    names = ("dA_gate", "dB_gate", "dA_up", "dB_up", "dA_down", "dB_down")
    for leaf, ref, name in zip(leaves, rgrads, names):
        assert leaf.grad.dtype == torch.float32
        assert_close_fro(np_f32(leaf.grad), ref, what=name)


@pytest.mark.parametrize("hidden,inter,r,m", [(896, 4864, 16, 1024), (256, 448, 64, 200)])
def test_fused_gated_mlp_error_beside_the_reference_bf16_path(hidden, inter, r, m):
    """The HIP path's relative Frobenius error against the fp64 oracle, printed
    beside the error of the reference's own bf16 step on the same operands
    (``gated_mlp_reference_bf16``: every autocast rounding point of
    methods/nf4_lora.py:43-50,83-109 and methods/gated_replay.py:290-299,372-388).
    The HIP path keeps fp32 through each contraction and its epilogue, so it may
    not be worse than 1.5x the reference's error on any output or gradient."""
    s = 2.0
    projs = [_proj(inter, hidden, r, 90), _proj(inter, hidden, r, 91), _proj(hidden, inter, r, 92)]
    x = seeded((m, hidden), 93).requires_grad_()
    dy = seeded((m, hidden), 94)
    leaves = []
    for _, _, a, b in projs:
        leaves += [a.clone().requires_grad_(), b.clone().requires_grad_()]
    (pg, qg, _, _), (pu, qu, _, _), (pd, qd, _, _) = projs
    y = fused_gated_nf4_lora_mlp(x, pg, leaves[0], leaves[1], pu, leaves[2], leaves[3], pd, leaves[4], leaves[5],
                                 qg, qu, qd, s, s, s)
    y.backward(dy)
    ry, rdx, rgrads = _oracle_mlp(x, projs, s, dy)
    ws = [oracle_weight(p, q).dequant_bf16().astype(np.float64) for p, q, _, _ in projs]
    ab = [np_f32(t).astype(np.float64) for _, _, a, b in projs for t in (a, b)]
    ey, edx, egrads = O.gated_mlp_reference_bf16(bf16_values(x), *ws, *ab, s, bf16_values(dy))
    names = ("Y", "dX", "dA_gate", "dB_gate", "dA_up", "dB_up", "dA_down", "dB_down")
    hip = [np_f32(y), np_f32(x.grad)] + [np_f32(leaf.grad) for leaf in leaves]
    emul = [ey, edx] + list(egrads)
    ref = [ry, rdx] + list(rgrads)
    print(f"gated MLP H={hidden} I={inter} r={r} M={m}: relative Frobenius error vs fp64 oracle", flush=True)
    print(f"  {'':8s} {'HIP':>10s} {'reference bf16':>15s}", flush=True)
    for name, h, e, o in zip(names, hip, emul, ref):
        eh, ee = O.rel_fro(h, o), O.rel_fro(e, o)
        print(f"  {name:8s} {eh:10.3e} {ee:15.3e}", flush=True)
        assert eh <= 5e-3, f"{name}: HIP error {eh:.3e} > 5e-3"
        assert eh <= 1.5 * ee, f"{name}: HIP error {eh:.3e} > 1.5 x the reference path's {ee:.3e}"


@pytest.mark.parametrize("hidden,inter,r,m", [(128, 256, 8, 32), (256, 448, 64, 200)])
def test_fused_gated_mlp_saved_h_equals_replay(hidden, inter, r, m):
    # Keeping h from the forward must give bit-identical gradients to replaying it.
    s = 2.0
    projs = [_proj(inter, hidden, r, 50), _proj(inter, hidden, r, 60), _proj(hidden, inter, r, 70)]
    (pg, qg, _, _), (pu, qu, _, _), (pd, qd, _, _) = projs
    dy = seeded((m, hidden), 81)
    runs = []
    for save in (True, False):
        x = seeded((m, hidden), 80).requires_grad_()
        leaves = []
        for _, _, a, b in projs:
            leaves += [a.clone().requires_grad_(), b.clone().requires_grad_()]
        y = fused_gated_nf4_lora_mlp(x, pg, leaves[0], leaves[1], pu, leaves[2], leaves[3], pd, leaves[4],
                                     leaves[5], qg, qu, qd, s, s, s, save_gated=save)
        y.backward(dy)
        runs.append([y.detach(), x.grad] + [leaf.grad for leaf in leaves])
    for a, b in zip(*runs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("hidden,intermediate", [(64, 96), (128, 256)])
@pytest.mark.parametrize("rematerialize_up,offload_up,offload_gate",
                         [(False, False, False), (True, False, False), (False, True, False),
                          (False, False, True), (False, True, True)])
def test_asymmetric_gated_replay_matches_oracle(hidden, intermediate, rematerialize_up, offload_up, offload_gate):
    """tests/kernels/test_gated_replay.py:11-114 against the oracle."""
    s = 2.0
    projs = [_proj(intermediate, hidden, 8, 1), _proj(intermediate, hidden, 8, 2), _proj(hidden, intermediate, 8, 3)]
    (pg, qg, ag, bg), (pu, qu, au, bu), (pd, qd, ad, bd) = projs
    x = seeded((1, 32, hidden), 1221).requires_grad_()
    leaves = [t.clone().requires_grad_() for t in (ag, bg, au, bu, ad, bd)]
    with torch.autocast("cuda", dtype=torch.bfloat16):
        gate = scheduled_nf4_lora(x, pg, leaves[0], leaves[1], qg, s)
        up = scheduled_nf4_lora(x, pu, leaves[2], leaves[3], qu, s)
        y = asymmetric_gated_nf4_lora(
            x, gate, up, pu, leaves[2], leaves[3], pd, leaves[4], leaves[5], qu, qd, s, s,
            rematerialize_up, offload_up,
            torch.empty_like(up, device="cpu", pin_memory=True) if offload_up else None,
            offload_gate, torch.empty_like(gate, device="cpu", pin_memory=True) if offload_gate else None)
    dy = seeded((1, 32, hidden), 1222)
    y.backward(dy)
    ry, rdx, rgrads = _oracle_mlp(x, projs, s, dy)
    assert_close_fro(np_f32(y).reshape(ry.shape), ry, what="Y")
    assert_close_fro(np_f32(x.grad).reshape(rdx.shape), rdx, what="dX")
    for leaf, ref, name in zip(leaves, rgrads, ("dAg", "dBg", "dAu", "dBu", "dAd", "dBd")):
        assert_close_fro(np_f32(leaf.grad), ref, what=name)


def test_asymmetric_replay_rejects_conflicting_modes():
    projs = [_proj(96, 64, 8, 1), _proj(96, 64, 8, 2), _proj(64, 96, 8, 3)]
    (_, _, _, _), (pu, qu, au, bu), (pd, qd, ad, bd) = projs
    x = seeded((4, 64), 1)
    gate, up = seeded((4, 96), 2), seeded((4, 96), 3)
    with pytest.raises(molt_amd.CapabilityError, match="replayed and offloaded"):
        asymmetric_gated_nf4_lora(x, gate, up, pu, au, bu, pd, ad, bd, qu, qd, 2.0, 2.0, True, True,
                                  torch.empty_like(up, device="cpu", pin_memory=True))
    with pytest.raises(molt_amd.CapabilityError, match="host buffer"):
        asymmetric_gated_nf4_lora(x, gate, up, pu, au, bu, pd, ad, bd, qu, qd, 2.0, 2.0, False, True, None)


def test_fused_silu_multiply_matches_bf16_reference():
    """tests/kernels/test_gated_activation.py:28-42."""
    torch.manual_seed(3402)
    left_gate = torch.randn(2, 31, 4864, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    left_up = torch.randn_like(left_gate, requires_grad=True)
    right_gate = left_gate.detach().clone().requires_grad_()
    right_up = left_up.detach().clone().requires_grad_()
    gradient = torch.randn_like(left_gate)
    reference = F.silu(left_gate.float()) * left_up.float()
    candidate = fused_silu_multiply(right_gate, right_up)
    reference.backward(gradient.float())
    candidate.backward(gradient)
    torch.testing.assert_close(candidate.float(), reference, rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(right_gate.grad.float(), left_gate.grad.float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(right_up.grad.float(), left_up.grad.float(), rtol=2e-2, atol=2e-2)


def test_fused_silu_multiply_fp32_matches_oracle():
    g = seeded((3, 5, 17), 3401, dtype=torch.float32).requires_grad_()
    u = seeded((3, 5, 17), 3402, dtype=torch.float32).requires_grad_()
    dh = seeded((3, 5, 17), 3403, dtype=torch.float32)
    h = fused_silu_multiply(g, u)
    h.backward(dh)
    go, uo, dho = np_f32(g).astype(np.float64), np_f32(u).astype(np.float64), np_f32(dh).astype(np.float64)
    np.testing.assert_allclose(np_f32(h), O.swiglu_forward(go, uo), rtol=1e-5, atol=1e-5)
    dg, du = O.swiglu_backward(go, uo, dho)
    np.testing.assert_allclose(np_f32(g.grad), dg, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(np_f32(u.grad), du, rtol=1e-5, atol=1e-5)


def test_fused_silu_multiply_rejects_mismatched_inputs():
    with pytest.raises(ValueError, match="identical"):
        fused_silu_multiply(torch.randn(2, 3, device="cuda"), torch.randn(2, 4, device="cuda"))
