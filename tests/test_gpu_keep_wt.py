"""Transposed-weight handoff from the forward GEMMs to the input gradients
(molt_nf4_*_keep_wt / molt_nf4_*_wt).

A keep_wt forward must give bitwise the plain forward's outputs and leave
deq(W)^T, bitwise the transpose of the dequantised weight (the values every
GEMM path stages); an input gradient given that copy must give bitwise the
result it computes when it stages the weight itself. Shapes cover a partial
column tile (N % 256 != 0), a ragged last row block, several row blocks per
tile column (each contraction step written by one of them), the split-K
forward (steps spread over blockIdx.y) and a fused gated MLP end to end with
the policy on and off."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests._util import seeded, uniform

import molt_amd
from molt_amd import ops
from molt_amd._lib import tuning

pytestmark = pytest.mark.gpu

R = 16


def _weight(n, k, seed):
    w = seeded((n, k), seed, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    return packed, qs, molt_amd.resolved_nf4_scales(qs)


def _dense_t(packed, qs):
    """deq(W)^T in bf16 (the dequant kernel's values), contiguous [K, N]."""
    return ops.nf4_dequantize(packed.reshape(-1), molt_amd.resolved_nf4_scales(qs), qs.code, int(qs.shape[0]),
                              int(qs.shape[1]), 64, 1, torch.bfloat16).t().contiguous()


@pytest.mark.parametrize("m,n,k,split", [(1000, 640, 1024, 0), (4096, 512, 2048, 0), (1024, 1024, 8192, 1)])
def test_single_forward_keeps_the_transpose_and_the_backward_reads_it(m, n, k, split):
    print(f"keep_wt single: M={m} N={n} K={k} split={split}", flush=True)
    packed, qs, sc = _weight(n, k, 801)
    x = seeded((m, k), 802)
    a = uniform((R, k), 803, 1 / np.sqrt(k))
    b = seeded((n, R), 804, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    dy = seeded((m, n), 805)
    u = ops.lora_project(dy, None, 2, 2.0, b, 1)
    # the split-K forward needs few output tiles and a long contraction
    knobs = dict(big_tile_min=1 if not split else 64, stage_min_mtiles=1)
    with tuning(**knobs):
        assert ops._keeps_wt(m, n, k, 1)
        y0 = ops.nf4_lora_forward(x, packed.reshape(-1), sc, qs.code, n, k, 1, 64, t, b, 2.0)
        y1, wt = ops.nf4_lora_forward_keep_wt(x, packed.reshape(-1), sc, qs.code, n, k, 1, 64, t, b, 2.0)
        assert wt.shape == (k, n), "the forward did not write the transposed weight"
        dx0 = ops.nf4_lora_backward_input(dy, packed.reshape(-1), sc, qs.code, n, k, 1, 64, u, a, 1.0)
        dx1 = ops.nf4_lora_backward_input(dy, packed.reshape(-1), sc, qs.code, n, k, 1, 64, u, a, 1.0, wt)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    assert torch.equal(wt, _dense_t(packed, qs))
    assert torch.equal(dx0, dx1)


@pytest.mark.parametrize("m,i,h", [(1000, 640, 1024), (2048, 896, 512)])
def test_gateup_forward_keeps_both_transposes_for_the_paired_gradient(m, i, h):
    print(f"keep_wt gate/up: M={m} I={i} H={h}", flush=True)
    pg, qg, sg = _weight(i, h, 811)
    pu, qu, su = _weight(i, h, 812)
    x = seeded((m, h), 813)
    ag, au = uniform((R, h), 814, 1 / np.sqrt(h)), uniform((R, h), 815, 1 / np.sqrt(h))
    bg, bu = seeded((i, R), 816, std=0.01, dtype=torch.float32), seeded((i, R), 817, std=0.01,
                                                                       dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, torch.cat([ag, au]), 0)
    dg, du = seeded((m, i), 818), seeded((m, i), 819)
    ug, uu = seeded((m, R), 820), seeded((m, R), 821)
    args = (x, pg.reshape(-1), sg, pu.reshape(-1), su, qg.code, i, h, 1, t, bg, bu, 2.0, 2.0)
    with tuning(big_tile_min=1, stage_min_mtiles=1):
        assert ops._keeps_wt(m, i, h, 2)
        plain = ops.nf4_gateup_forward(*args)
        kept = ops.nf4_gateup_forward_keep_wt(*args)
        pair = (dg, du, pg.reshape(-1), sg, pu.reshape(-1), su, qg.code, i, h, 1, ug, uu, ag, au)
        dx0 = ops.nf4_lora_backward_input_pair(*pair)
        dx1 = ops.nf4_lora_backward_input_pair(*pair, kept[3], kept[4])
    torch.cuda.synchronize()
    for a_, b_ in zip(plain, kept[:3]):
        assert torch.equal(a_, b_)
    assert torch.equal(kept[3], _dense_t(pg, qg))
    assert torch.equal(kept[4], _dense_t(pu, qu))
    assert torch.equal(dx0, dx1)


def test_swiglu_backward_reads_the_kept_down_transpose():
    m, h, i = 1000, 512, 1280
    print(f"keep_wt SwiGLU backward: M={m} H={h} I={i}", flush=True)
    pd, qd, sd = _weight(h, i, 831)
    hh = seeded((m, i), 832)
    ad = uniform((R, i), 833, 1 / np.sqrt(i))
    bd = seeded((h, R), 834, std=0.01, dtype=torch.float32)
    t = ops.lora_project(hh, None, 0, 1.0, ad, 0)
    dy, gate, up = seeded((m, h), 835), seeded((m, i), 836), seeded((m, i), 837)
    u = ops.lora_project(dy, None, 2, 2.0, bd, 1)
    with tuning(big_tile_min=1, stage_min_mtiles=1):
        _, wt = ops.nf4_lora_forward_keep_wt(hh, pd.reshape(-1), sd, qd.code, h, i, 1, 64, t, bd, 2.0)
        assert wt.shape == (i, h)
        g0, u0 = ops.nf4_swiglu_backward(dy, pd.reshape(-1), sd, qd.code, h, i, 1, u, ad, gate, up)
        g1, u1 = ops.nf4_swiglu_backward(dy, pd.reshape(-1), sd, qd.code, h, i, 1, u, ad, gate, up, wt)
    torch.cuda.synchronize()
    assert torch.equal(g0, g1) and torch.equal(u0, u1)


def test_small_batches_keep_nothing():
    """Below the staging threshold the keep_wt forward returns an empty
    tensor and the backward runs its own path."""
    m, n, k = 64, 512, 1024
    packed, qs, sc = _weight(n, k, 841)
    x = seeded((m, k), 842)
    assert not ops._keeps_wt(m, n, k, 1)
    y0 = ops.nf4_lora_forward(x, packed.reshape(-1), sc, qs.code, n, k, 1, 64, None, None, 1.0)
    y1, wt = ops.nf4_lora_forward_keep_wt(x, packed.reshape(-1), sc, qs.code, n, k, 1, 64, None, None, 1.0)
    torch.cuda.synchronize()
    assert wt.numel() == 0 and torch.equal(y0, y1)


def test_fused_gated_mlp_same_with_and_without_kept_transposes():
    from molt_amd.methods import fused_gated_nf4_lora_mlp

    # (both input gradients stage only for output widths of whole 256-column tiles)
    H, I, r, M, s = 1024, 2560, 16, 1024, 2.0
    print(f"fused gated MLP H={H} I={I} M={M}: keep_weight_transposes on vs off", flush=True)
    projs = []
    for out_f, in_f, seed in ((I, H, 851), (I, H, 852), (H, I, 853)):
        packed, qs, _ = _weight(out_f, in_f, seed)
        a = uniform((r, in_f), seed + 10, 1 / np.sqrt(in_f)).requires_grad_()
        b = seeded((out_f, r), seed + 20, std=0.01, dtype=torch.float32).requires_grad_()
        projs.append((packed, qs, a, b))
    x = seeded((M, H), 854).requires_grad_()
    dy = seeded((M, H), 855)
    (pg, qg, ag, bg), (pu, qu, au, bu), (pd, qd, ad, bd) = projs
    leaves = (x, ag, bg, au, bu, ad, bd)
    results = []
    prev = ops.keep_weight_transposes()
    try:
        with tuning(big_tile_min=1, stage_min_mtiles=1):
            assert ops._keeps_wt(M, I, H, 2) and ops._keeps_wt(M, H, I, 1)
            for keep in (False, True):
                ops.keep_weight_transposes(keep)
                for t_ in leaves:
                    t_.grad = None
                y = fused_gated_nf4_lora_mlp(x, pg, ag, bg, pu, au, bu, pd, ad, bd, qg, qu, qd, s, s, s)
                y.backward(dy)
                results.append([y.detach().clone()] + [t_.grad.clone() for t_ in leaves])
    finally:
        ops.keep_weight_transposes(prev)
    torch.cuda.synchronize()
    for a_, b_ in zip(*results):
        assert torch.equal(a_, b_)
