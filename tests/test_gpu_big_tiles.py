"""The 256 x 256-tile GEMM kernels (chosen for large problems) forced at small
shapes with row/column tails via the big_tile_min setting. They must match the
fp64 oracle, and the 128 x 128-tile kernels bit for bit (both accumulate the
same MFMA products in the same contraction order)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as O
from tests._util import assert_close_fro, bf16_values, np_f32, oracle_weight, seeded, uniform

import molt_amd
from molt_amd import ops

pytestmark = pytest.mark.gpu


def _weight(out_f, in_f, seed):
    w = seeded((out_f, in_f), seed, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    return packed.reshape(-1), qs, molt_amd.resolved_nf4_scales(qs)


def _both(monkeypatch, fn):
    from molt_amd._lib import tuning

    with tuning(big_tile_min=1):
        big = fn()
    with tuning(big_tile_min=1 << 40, split_k=0):
        small = fn()
    return big, small


@pytest.mark.parametrize("m,n,k,r", [(300, 320, 256, 16), (512, 256, 512, 64), (37, 1024, 128, 8)])
def test_forward_big_tiles(monkeypatch, m, n, k, r):
    print(f"big fwd m={m} n={n} k={k} r={r}", flush=True)
    packed, qs, scales = _weight(n, k, 1)
    x = seeded((m, k), 2)
    a = uniform((r, k), 3, 1 / np.sqrt(k))
    b = seeded((n, r), 4, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    big, small = _both(monkeypatch, lambda: ops.nf4_lora_forward(x, packed, scales, qs.code, n, k, 1, 64, t, b, 2.0))
    assert torch.equal(big, small)
    w = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    ref = bf16_values(x) @ w.T + 2.0 * (bf16_values(t) @ bf16_values(b).T)
    assert_close_fro(np_f32(big), ref, what="Y")


@pytest.mark.parametrize("m,i,h,r", [(300, 192, 256, 16), (256, 512, 128, 64)])
def test_gateup_big_tiles(monkeypatch, m, i, h, r):
    print(f"big gate/up m={m} I={i} H={h} r={r}", flush=True)
    pg, qg, sg = _weight(i, h, 5)
    pu, qu, su = _weight(i, h, 6)
    x = seeded((m, h), 7)
    ag, au = uniform((r, h), 8, 1 / np.sqrt(h)), uniform((r, h), 9, 1 / np.sqrt(h))
    bg, bu = seeded((i, r), 10, std=0.01, dtype=torch.float32), seeded((i, r), 11, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, torch.cat([ag, au]), 0)
    big, small = _both(monkeypatch, lambda: ops.nf4_gateup_forward(x, pg, sg, pu, su, qg.code, i, h, 1, t, bg, bu,
                                                                    2.0, 2.0))
    for bt, st in zip(big, small):
        assert torch.equal(bt, st)
    wg = oracle_weight(pg, qg).dequant_bf16().astype(np.float64)
    wu = oracle_weight(pu, qu).dequant_bf16().astype(np.float64)
    xo = bf16_values(x)
    g = O.bf16_round(xo @ wg.T + 2.0 * (bf16_values(t[:, :r]) @ bf16_values(bg).T))
    u = O.bf16_round(xo @ wu.T + 2.0 * (bf16_values(t[:, r:]) @ bf16_values(bu).T))
    assert_close_fro(np_f32(big[0]), g, what="gate")
    assert_close_fro(np_f32(big[1]), u, what="up")
    assert_close_fro(np_f32(big[2]), O.swiglu_forward(g, u), what="h")


@pytest.mark.parametrize("m,n,k,r", [(300, 256, 320, 16), (256, 512, 256, 64)])
def test_backward_big_tiles(monkeypatch, m, n, k, r):
    print(f"big bwd m={m} n={n} k={k} r={r}", flush=True)
    packed, qs, scales = _weight(n, k, 12)
    dy = seeded((m, n), 13)
    u = seeded((m, r), 14)
    a = uniform((r, k), 15, 1 / np.sqrt(k))
    big, small = _both(monkeypatch, lambda: ops.nf4_lora_backward_input(dy, packed, scales, qs.code, n, k, 1, 64, u,
                                                                         a, 1.0))
    assert torch.equal(big, small)
    w = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    ref = bf16_values(dy) @ w + bf16_values(u) @ bf16_values(a)
    assert_close_fro(np_f32(big), ref, what="dX")


def test_paired_backward_big_tiles(monkeypatch):
    m, i, h, r = 300, 256, 320, 16
    p0, q0, s0 = _weight(i, h, 16)
    p1, q1, s1 = _weight(i, h, 17)
    d0, d1 = seeded((m, i), 18), seeded((m, i), 19)
    u0, u1 = seeded((m, r), 20), seeded((m, r), 21)
    a0, a1 = uniform((r, h), 22, 0.05), uniform((r, h), 23, 0.05)
    big, small = _both(monkeypatch, lambda: ops.nf4_lora_backward_input_pair(d0, d1, p0, s0, p1, s1, q0.code, i, h, 1,
                                                                              u0, u1, a0, a1))
    assert torch.equal(big, small)
    w0 = oracle_weight(p0, q0).dequant_bf16().astype(np.float64)
    w1 = oracle_weight(p1, q1).dequant_bf16().astype(np.float64)
    ref = (bf16_values(d0) @ w0 + bf16_values(d1) @ w1 + bf16_values(u0) @ bf16_values(a0)
           + bf16_values(u1) @ bf16_values(a1))
    assert_close_fro(np_f32(big), ref, what="dX")


def test_swiglu_backward_big_tiles(monkeypatch):
    m, h, i, r = 300, 256, 320, 16
    pd, qd, sd = _weight(h, i, 24)
    dy = seeded((m, h), 25)
    u = seeded((m, r), 26)
    a = uniform((r, i), 27, 0.05)
    gate, up = seeded((m, i), 28), seeded((m, i), 29)
    big, small = _both(monkeypatch, lambda: ops.nf4_swiglu_backward(dy, pd, sd, qd.code, h, i, 1, u, a, gate, up))
    for bt, st in zip(big, small):
        assert torch.equal(bt, st)
    w = oracle_weight(pd, qd).dequant_bf16().astype(np.float64)
    dh = O.bf16_round(bf16_values(dy) @ w + bf16_values(u) @ bf16_values(a)).astype(np.float64)
    dg, du = O.swiglu_backward(bf16_values(gate), bf16_values(up), dh)
    assert_close_fro(np_f32(big[0]), dg, what="dgate")
    assert_close_fro(np_f32(big[1]), du, what="dup")
