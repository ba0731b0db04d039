"""The headline workload at its full size (cfg4: H=4096, I=14336, r=64,
M=8192 tokens) through the fused gated MLP, checked by properties that do not
need the whole oracle: sampled rows of Y and dX against the fp64 oracle (a row
of Y and of dX depends only on the same row of X and dY), bitwise repeatability
of every output and gradient, and empty token batches."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as O
from tests._util import assert_close_fro, bf16_values, np_f32, oracle_weight, seeded, uniform

import molt_amd
from molt_amd.methods import fused_gated_nf4_lora_mlp, scheduled_nf4_lora

pytestmark = pytest.mark.gpu

H, I, R, M = 4096, 14336, 64, 8192


def _proj(out_f, in_f, seed):
    w = seeded((out_f, in_f), seed, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    del w
    a = uniform((R, in_f), seed + 1, 1.0 / np.sqrt(in_f)).requires_grad_()
    b = seeded((out_f, R), seed + 2, std=0.01, dtype=torch.float32).requires_grad_()
    return packed, qs, a, b


def _run(projs, x, dy, s):
    (pg, qg, ag, bg), (pu, qu, au, bu), (pd, qd, ad, bd) = projs
    for t in (x, ag, bg, au, bu, ad, bd):
        t.grad = None
    y = fused_gated_nf4_lora_mlp(x, pg, ag, bg, pu, au, bu, pd, ad, bd, qg, qu, qd, s, s, s)
    y.backward(dy)
    torch.cuda.synchronize()
    return [y.detach().clone(), x.grad.clone()] + [t.grad.clone() for t in (ag, bg, au, bu, ad, bd)]


def test_cfg4_sampled_rows_match_oracle_and_runs_repeat_bitwise():
    print("cfg4 full size: quantising three 14336 x 4096 weights", flush=True)
    s = 2.0
    projs = [_proj(I, H, 100), _proj(I, H, 200), _proj(H, I, 300)]
    x = seeded((M, H), 400).requires_grad_()
    dy = seeded((M, H), 401)
    first = _run(projs, x, dy, s)
    second = _run(projs, x, dy, s)
    for a, b in zip(first, second):
        assert torch.equal(a, b), "full-size runs differ"
    print("cfg4 full size: oracle on sampled rows", flush=True)
    rows = np.array([0, 1, 255, 256, 4095, 4096, 8190, 8191])
    ws = [oracle_weight(p, q).dequant_bf16().astype(np.float64) for p, q, _, _ in projs]
    av = []
    for _, _, a, b in projs:
        av += [bf16_values(a), bf16_values(b)]
    xo = bf16_values(x)[rows]
    dyo = bf16_values(dy)[rows]
    ry, saved = O.gated_mlp_forward(xo, ws[0], ws[1], ws[2], *av, s)
    rdx, _ = O.gated_mlp_backward(xo, ws[0], ws[1], ws[2], *av, s, dyo, saved)
    ey_hip = assert_close_fro(np_f32(first[0])[rows], ry, what="Y rows")
    edx_hip = assert_close_fro(np_f32(first[1])[rows], rdx, what="dX rows")
    # the reference's own bf16 step on the same rows (a row of Y and dX depends
    # only on its own rows of X and dY), reported beside the HIP error
    masters = [np_f32(t).astype(np.float64) for _, _, a, b in projs for t in (a, b)]
    ey, edx, _ = O.gated_mlp_reference_bf16(xo, ws[0], ws[1], ws[2], *masters, s, dyo)
    ey_ref, edx_ref = O.rel_fro(ey, ry), O.rel_fro(edx, rdx)
    print(f"cfg4 sampled rows, relative Frobenius error vs fp64: Y HIP {ey_hip:.3e} reference-bf16 {ey_ref:.3e}; "
          f"dX HIP {edx_hip:.3e} reference-bf16 {edx_ref:.3e}", flush=True)
    assert ey_hip <= 1.5 * ey_ref and edx_hip <= 1.5 * edx_ref
    for g in first[2:]:
        assert torch.isfinite(g).all() and g.abs().sum() > 0


def _fp64(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to(torch.float64)


def _rel(actual: torch.Tensor, expected: torch.Tensor) -> float:
    a, e = _fp64(actual), _fp64(expected)
    return float(torch.linalg.vector_norm(a - e) / torch.linalg.vector_norm(e).clamp_min(1e-300))


def test_cfg4_full_size_adapter_gradients_and_intermediates():
    """All 8192 rows at cfg4: the six adapter gradients against fp64 GPU matmuls
    of the node's own bf16 operands (dB = s dY^T T, dA = U^T Z; 1e-5), and the
    intermediates g, u, h, dg, du, Y and dX against fp32 GEMMs over the
    bit-exact dequantised weights (5e-3)."""
    from molt_amd import ops
    from molt_amd.methods.gated_replay import _fused_backward, _fused_forward

    torch.backends.cuda.matmul.allow_tf32 = False
    print("cfg4 full size: adapter gradients", flush=True)
    s = 2.0
    projs = [_proj(I, H, 110), _proj(I, H, 210), _proj(H, I, 310)]
    (pg, qg, ag, bg), (pu, qu, au, bu), (pd, qd, ad, bd) = projs
    x = seeded((M, H), 410)
    dy = seeded((M, H), 411)
    with torch.no_grad():
        # the training path: transposed weights and packed B handed from the forward to the backward
        y, gate, up, h, t_gu, t_d, dims, wts, bpacks = _fused_forward(x, pg, ag, bg, pu, au, bu, pd, ad, bd, qg,
                                                                      qu, qd, s, s, s, keep_wt=True, grad=True)
        assert wts is not None and all(w.numel() > 0 for w in wts), "cfg4 stages and keeps every weight"
        dx, dag, dbg, dau, dbu, dad, dbd = _fused_backward(dy, x, gate, up, h, t_gu, t_d, pg, ag, bg, pu, au, bu,
                                                           pd, ad, bd, (qg, qu, qd), (s, s, s), dims, wts=wts,
                                                           bpacks=bpacks)
        del wts, bpacks
        sc = molt_amd.resolved_nf4_scales
        u_d = ops.lora_project(dy, None, 2, s, bd, 1)
        dg, du = ops.nf4_swiglu_backward(dy, pd.reshape(-1), sc(qd), qd.code, H, I, 1, u_d, ad, gate, up)
        u_g = ops.lora_project(dg, None, 2, s, bg, 1)
        u_u = ops.lora_project(du, None, 2, s, bu, 1)
        r = R
        checks = {
            "dA_gate": (dag, _fp64(u_g).T @ _fp64(x)),
            "dA_up": (dau, _fp64(u_u).T @ _fp64(x)),
            "dA_down": (dad, _fp64(u_d).T @ _fp64(h)),
            "dB_gate": (dbg, s * (_fp64(dg).T @ _fp64(t_gu[:, :r]))),
            "dB_up": (dbu, s * (_fp64(du).T @ _fp64(t_gu[:, r:]))),
            "dB_down": (dbd, s * (_fp64(dy).T @ _fp64(t_d))),
        }
        for name, (got, ref) in checks.items():
            err = _rel(got, ref)
            print(f"  {name}: rel {err:.2e}", flush=True)
            assert err <= 1e-5, f"{name}: relative error {err:.3e} > 1e-5"
        print("cfg4 full size: intermediates vs fp32 GEMMs", flush=True)
        wg, wu, wd = (molt_amd.dequantize_4bit(p, q, torch.bfloat16).float() for p, q in ((pg, qg), (pu, qu), (pd, qd)))
        xf, dyf = x.float(), dy.float()
        bf = lambda t: t.to(torch.bfloat16).float()  # noqa: E731

        def lin(z, w, a, b):
            return z @ w.T + s * (bf(z @ bf(a).T) @ bf(b).T)

        g_ref = lin(xf, wg, ag, bg)
        assert _rel(gate.float(), g_ref) <= 5e-3
        u_ref = lin(xf, wu, au, bu)
        assert _rel(up.float(), u_ref) <= 5e-3
        del g_ref, u_ref
        gf, uf = gate.float(), up.float()
        h_ref = gf * torch.sigmoid(gf) * uf
        assert _rel(h.float(), h_ref) <= 5e-3
        del h_ref
        assert _rel(y.float(), lin(h.float(), wd, ad, bd)) <= 5e-3
        dh = dyf @ wd + bf(bf(s * dyf) @ bf(bd)) @ bf(ad)
        sg = torch.sigmoid(gf)
        assert _rel(dg.float(), dh * uf * sg * (1 + gf * (1 - sg))) <= 5e-3
        assert _rel(du.float(), dh * gf * sg) <= 5e-3
        del dh, sg
        dgf, duf = dg.float(), du.float()
        dx_ref = dgf @ wg + duf @ wu + bf(bf(s * dgf) @ bf(bg)) @ bf(ag) + bf(bf(s * duf) @ bf(bu)) @ bf(au)
        err = _rel(dx.float(), dx_ref)
        print(f"  dX all rows: rel {err:.2e}", flush=True)
        assert err <= 5e-3


def test_cfg2_full_size_forward_and_input_gradient():
    """cfg2 at its own workload: W 8960x1536 and 1536x8960, M = 4096 tokens,
    r = 16, forward Y and backward dX through scheduled_nf4_lora (the 256 x 256
    tile kernels at this size). 64 sampled rows against the fp64 oracle, every
    row against fp32 GEMMs over the bit-exact dequantised weight, and bitwise
    repeatability (tests/kernels/test_nf4_lora.py:14-45 shapes)."""
    torch.backends.cuda.matmul.allow_tf32 = False
    s, r, m = 2.0, 16, 4096
    rows = np.sort(np.random.default_rng(7).choice(m, 64, replace=False))
    for out_f, in_f in ((8960, 1536), (1536, 8960)):
        print(f"cfg2 {in_f}->{out_f} M={m}", flush=True)
        w = seeded((out_f, in_f), 600 + out_f, std=0.02, dtype=torch.float32)
        packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
        del w
        a = uniform((r, in_f), 601, 1.0 / np.sqrt(in_f))
        b = seeded((out_f, r), 602, std=0.01, dtype=torch.float32)
        x = seeded((m, in_f), 603)
        dy = seeded((m, out_f), 604)
        outs = []
        for _ in range(2):
            xr = x.clone().requires_grad_()
            with torch.autocast("cuda", dtype=torch.bfloat16):
                y = scheduled_nf4_lora(xr, packed, a, b, qs, s)
            y.backward(dy)
            outs.append((y.detach(), xr.grad))
        assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
        y, dx = outs[0]
        wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
        ao, bo = bf16_values(a), bf16_values(b)
        xo, dyo = bf16_values(x)[rows], bf16_values(dy)[rows]
        assert_close_fro(np_f32(y)[rows], O.lora_linear_forward(xo, wo, ao, bo, s), what="Y rows")
        rdx, _, _ = O.lora_linear_backward(xo, wo, ao, bo, s, dyo)
        assert_close_fro(np_f32(dx)[rows], rdx, what="dX rows")
        wf = molt_amd.dequantize_4bit(packed, qs, torch.bfloat16).float()
        bf = lambda t: t.to(torch.bfloat16).float()  # noqa: E731
        xf, dyf = x.float(), dy.float()
        y_ref = xf @ wf.T + s * (bf(xf @ bf(a).T) @ bf(b).T)
        dx_ref = dyf @ wf + bf(bf(s * dyf) @ bf(b)) @ bf(a)
        assert _rel(y.float(), y_ref) <= 5e-3
        assert _rel(dx.float(), dx_ref) <= 5e-3


def test_empty_token_batches():
    s = 2.0
    projs = [_proj(256, 128, 10), _proj(256, 128, 20), _proj(128, 256, 30)]
    (pg, qg, ag, bg), (pu, qu, au, bu), (pd, qd, ad, bd) = projs
    x = torch.empty((0, 128), device="cuda", dtype=torch.bfloat16, requires_grad=True)
    y = fused_gated_nf4_lora_mlp(x, pg, ag, bg, pu, au, bu, pd, ad, bd, qg, qu, qd, s, s, s)
    assert y.shape == (0, 128)
    y.backward(torch.empty_like(y))
    assert x.grad.shape == (0, 128)
    for t in (ag, bg, au, bu, ad, bd):
        assert t.grad is not None and torch.count_nonzero(t.grad) == 0
    with torch.autocast("cuda", dtype=torch.bfloat16):
        z = scheduled_nf4_lora(x, pg, ag, bg, qg, s)
    assert z.shape == (0, 256)


@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_cfg5_gemv_full_shapes_repeat_bitwise_and_match_oracle(n, k):
    """Every cfg5 decode shape at M in {1, 2, 16} with the r = 16 LoRA add-on:
    repeated calls are bitwise equal, and a sample of outputs matches the oracle."""
    from molt_amd import ops

    print(f"cfg5 gemv N={n} K={k}", flush=True)
    w = seeded((n, k), 500 + n + k, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    del w
    s2 = qs.state2
    a = uniform((16, k), 501, 1.0 / np.sqrt(k))
    b = seeded((n, 16), 502, std=0.01, dtype=torch.float32)
    ow = oracle_weight(packed, qs).dequant_f32().astype(np.float64)
    for m in (1, 2, 16):
        x = seeded((m, k), 503 + m)
        t = ops.lora_project(x, None, 0, 1.0, a, 0)

        def run():
            return ops.nf4_gemv(x, packed.reshape(-1), None, qs.absmax, s2.absmax, s2.code, float(qs.offset),
                                int(s2.blocksize), qs.code, n, k, 1, t, b, 2.0)

        y1, y2 = run(), run()
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), f"M={m}: repeated GEMV calls differ"
        ref = bf16_values(x) @ ow.T + 2.0 * (bf16_values(t) @ bf16_values(b).T)
        assert_close_fro(np_f32(y1), ref, what=f"GEMV M={m}")
