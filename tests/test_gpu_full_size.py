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
    assert_close_fro(np_f32(first[0])[rows], ry, what="Y rows")
    assert_close_fro(np_f32(first[1])[rows], rdx, what="dX rows")
    for g in first[2:]:
        assert torch.isfinite(g).all() and g.abs().sum() > 0


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
