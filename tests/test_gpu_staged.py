"""Staged weights in the 256 x 256 GEMMs: for many token rows the weight is
dequantised once into the caller's workspace (bf16 rows for the forward,
transposed bf16 for the input gradient) and the GEMM reads it by DMA instead of
dequantising every weight tile again in each 256-row block. The tile values, the
contraction order and so every output must equal the fused kernels' bit for bit:
each case runs staged (stage_min_mtiles=1) and fused (0) and compares, with
ragged row/column tails, LoRA terms, the gate/up pair, the paired and SwiGLU
backward, and split-K (the partials then sit after the staged copy). In the
forward, LoRA lengths (r, or 2r for the gate/up pair) that are a multiple of
64, or a multiple of 8 below 64 (one step over rows padded with zeros), also
stage bf16(s B) and stream the LoRA steps through the same ring."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests._util import assert_close_fro, bf16_values, np_f32, oracle_weight, seeded, uniform

import molt_amd
from molt_amd import _lib, ops
from molt_amd._lib import tuning

pytestmark = pytest.mark.gpu


def _weight(out_f, in_f, seed):
    w = seeded((out_f, in_f), seed, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    return packed.reshape(-1), qs, molt_amd.resolved_nf4_scales(qs)


def _staged_and_fused(fn, big_tile_min=1):
    with tuning(big_tile_min=big_tile_min, stage_min_mtiles=1):
        staged = fn()
    with tuning(big_tile_min=big_tile_min, stage_min_mtiles=0):
        fused = fn()
    torch.cuda.synchronize()
    return staged, fused


def _equal(staged, fused):
    staged = staged if isinstance(staged, tuple) else (staged,)
    fused = fused if isinstance(fused, tuple) else (fused,)
    for s, f in zip(staged, fused):
        assert torch.equal(s, f), f"staged differs from fused: max |d| {(s.float() - f.float()).abs().max().item()}"


@pytest.mark.parametrize("m,n,k,r,btm", [(300, 320, 256, 16, 1), (4173, 512, 1024, 16, 1),
                                         (4096, 1536, 8960, 16, 256), (300, 320, 256, 64, 1),
                                         (4173, 512, 1024, 128, 1), (4096, 1536, 8960, 64, 256)])
def test_forward_staged(m, n, k, r, btm):
    print(f"staged forward m={m} n={n} k={k} r={r} big_tile_min={btm}", flush=True)
    lib = _lib.load()
    with tuning(big_tile_min=btm, stage_min_mtiles=1):
        assert lib.molt_nf4_lora_forward_workspace(m, n, k, r) >= n * k * 2, "the call must stage the weight"
    packed, qs, scales = _weight(n, k, 31)
    x = seeded((m, k), 32)
    a = uniform((r, k), 33, 1 / np.sqrt(k))
    b = seeded((n, r), 34, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    staged, fused = _staged_and_fused(
        lambda: ops.nf4_lora_forward(x, packed, scales, qs.code, n, k, 1, 64, t, b, 2.0), btm)
    _equal(staged, fused)
    rows = np.sort(np.random.default_rng(3).choice(m, min(m, 64), replace=False))
    w = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    ref = bf16_values(x)[rows] @ w.T + 2.0 * (bf16_values(t)[rows] @ bf16_values(b).T)
    assert_close_fro(np_f32(staged)[rows], ref, what="staged Y rows")


@pytest.mark.parametrize("m,i,h,r", [(300, 192, 256, 16), (4100, 512, 512, 8), (300, 192, 256, 32),
                                     (4100, 512, 512, 64)])
def test_gateup_staged(m, i, h, r):
    print(f"staged gate/up m={m} I={i} H={h} r={r}", flush=True)
    with tuning(big_tile_min=1, stage_min_mtiles=1):
        assert _lib.load().molt_nf4_gateup_forward_workspace(m, i, h, r) >= 2 * i * h * 2
    pg, qg, sg = _weight(i, h, 35)
    pu, qu, su = _weight(i, h, 36)
    x = seeded((m, h), 37)
    ag, au = uniform((r, h), 38, 1 / np.sqrt(h)), uniform((r, h), 39, 1 / np.sqrt(h))
    bg, bu = seeded((i, r), 40, std=0.01, dtype=torch.float32), seeded((i, r), 41, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, torch.cat([ag, au]), 0)
    staged, fused = _staged_and_fused(
        lambda: ops.nf4_gateup_forward(x, pg, sg, pu, su, qg.code, i, h, 1, t, bg, bu, 2.0, 2.0))
    _equal(staged, fused)


@pytest.mark.parametrize("m,n,k,r", [(300, 256, 512, 16), (4173, 1024, 768, 0), (300, 256, 512, 64),
                                     (4173, 1024, 768, 128)])
def test_backward_staged(m, n, k, r):
    print(f"staged backward m={m} n={n} k={k} r={r}", flush=True)
    with tuning(big_tile_min=1, stage_min_mtiles=1):
        assert _lib.load().molt_nf4_lora_backward_workspace(m, n, k, 1) >= n * k * 2
    packed, qs, scales = _weight(n, k, 42)
    dy = seeded((m, n), 43)
    u = seeded((m, max(r, 1)), 44) if r else None
    a = uniform((r, k), 45, 1 / np.sqrt(k)) if r else None
    staged, fused = _staged_and_fused(
        lambda: ops.nf4_lora_backward_input(dy, packed, scales, qs.code, n, k, 1, 64, u, a, 1.0))
    _equal(staged, fused)
    rows = np.sort(np.random.default_rng(4).choice(m, min(m, 64), replace=False))
    w = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    ref = bf16_values(dy)[rows] @ w
    if r:
        ref = ref + bf16_values(u)[rows] @ bf16_values(a)
    assert_close_fro(np_f32(staged)[rows], ref, what="staged dX rows")


@pytest.mark.parametrize("m,i,h,r,btm", [(300, 256, 512, 16, 1), (4096, 8960, 1536, 16, 256),
                                         (300, 256, 512, 64, 1), (4096, 8960, 1536, 64, 256)])
def test_paired_backward_staged(m, i, h, r, btm):
    print(f"staged paired backward m={m} I={i} H={h} r={r} big_tile_min={btm}", flush=True)
    with tuning(big_tile_min=btm, stage_min_mtiles=1):
        assert _lib.load().molt_nf4_lora_backward_workspace(m, i, h, 2) >= 2 * i * h * 2
    p0, q0, s0 = _weight(i, h, 46)
    p1, q1, s1 = _weight(i, h, 47)
    d0, d1 = seeded((m, i), 48), seeded((m, i), 49)
    u0, u1 = seeded((m, r), 50), seeded((m, r), 51)
    a0, a1 = uniform((r, h), 52, 0.05), uniform((r, h), 53, 0.05)
    staged, fused = _staged_and_fused(
        lambda: ops.nf4_lora_backward_input_pair(d0, d1, p0, s0, p1, s1, q0.code, i, h, 1, u0, u1, a0, a1), btm)
    _equal(staged, fused)


@pytest.mark.parametrize("r", [16, 64])
def test_swiglu_backward_staged(r):
    m, h, i = 300, 256, 512
    print(f"staged SwiGLU backward m={m} H={h} I={i} r={r}", flush=True)
    pd, qd, sd = _weight(h, i, 54)
    dy = seeded((m, h), 55)
    u = seeded((m, r), 56)
    a = uniform((r, i), 57, 0.05)
    gate, up = seeded((m, i), 58), seeded((m, i), 59)
    staged, fused = _staged_and_fused(lambda: ops.nf4_swiglu_backward(dy, pd, sd, qd.code, h, i, 1, u, a, gate, up))
    _equal(staged, fused)


def test_staging_needs_the_workspace():
    """A caller that passes no workspace gets the fused kernels and the same result."""
    m, n, k = 300, 256, 512
    print(f"staged forward without workspace m={m} n={n} k={k}", flush=True)
    packed, qs, scales = _weight(n, k, 60)
    x = seeded((m, k), 61)
    w = ops._weight(packed, scales, qs.code.float(), n, k, 64, 1)
    lib = _lib.load()
    outs = []
    for ws_bytes in (0, None):
        y = torch.empty((m, n), device=x.device, dtype=torch.bfloat16)
        with tuning(big_tile_min=1, stage_min_mtiles=1):
            nbytes = lib.molt_nf4_lora_forward_workspace(m, n, k, 0) if ws_bytes is None else 0
            ws = torch.empty(nbytes, device=x.device, dtype=torch.uint8) if nbytes else None
            _lib.check(lib.molt_nf4_lora_forward(x.data_ptr(), k, m, ops.C.byref(w), None, 1, None, 0, 1.0,
                                                 y.data_ptr(), n, None if ws is None else ws.data_ptr(), nbytes,
                                                 ops._stream(x.device)))
        outs.append(y)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("r", [64, 16, 8])
def test_lora_ring_needs_its_workspace(r):
    """A workspace sized without the rank (room for the staged weight only)
    stages the weight and runs the LoRA steps outside the ring: same result
    (ranks below 64 as one ring step whose T columns past r read as zeros)."""
    m, n, k = 300, 256, 512
    print(f"staged forward, LoRA ring with and without its workspace m={m} n={n} k={k} r={r}", flush=True)
    packed, qs, scales = _weight(n, k, 62)
    x = seeded((m, k), 63)
    a = uniform((r, k), 64, 1 / np.sqrt(k))
    b = seeded((n, r), 65, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    w = ops._weight(packed, scales, qs.code.float(), n, k, 64, 1)
    bb = b.contiguous()
    lib = _lib.load()
    outs = []
    with tuning(big_tile_min=1, stage_min_mtiles=1):
        for rank in (0, r):
            nbytes = lib.molt_nf4_lora_forward_workspace(m, n, k, rank)
            ws = torch.empty(nbytes, device=x.device, dtype=torch.uint8)
            y = torch.empty((m, n), device=x.device, dtype=torch.bfloat16)
            _lib.check(lib.molt_nf4_lora_forward(x.data_ptr(), k, m, ops.C.byref(w), t.data_ptr(), r, bb.data_ptr(),
                                                 r, 2.0, y.data_ptr(), n, ws.data_ptr(), nbytes,
                                                 ops._stream(x.device)))
            outs.append(y)
        assert lib.molt_nf4_lora_forward_workspace(m, n, k, r) > lib.molt_nf4_lora_forward_workspace(m, n, k, 0)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("r", [16, 8])
def test_gateup_short_rank_ring_equals_the_unpipelined_steps(r):
    """The gate/up pair with 2r < 64 (cfg3's r = 16): its LoRA length streams
    through the ring as one zero-padded step; a workspace without the staged
    B rows runs the register-staged LoRA step instead. Gate, up and h agree
    bit for bit."""
    m, i, h = 300, 256, 512
    print(f"staged gate/up forward, LoRA ring with and without its workspace m={m} I={i} H={h} r={r}", flush=True)
    pg, qg, sg = _weight(i, h, 73)
    pu, qu, su = _weight(i, h, 74)
    x = seeded((m, h), 75)
    t = seeded((m, 2 * r), 76)
    bg = seeded((i, r), 77, std=0.01, dtype=torch.float32)
    bu = seeded((i, r), 78, std=0.01, dtype=torch.float32)
    code = qg.code.float()
    wg = ops._weight(pg, sg, code, i, h, 64, 1)
    wu = ops._weight(pu, su, code, i, h, 64, 1)
    lib = _lib.load()

    def run(tt, rank):
        nbytes = lib.molt_nf4_gateup_forward_workspace(m, i, h, rank)
        ws = torch.empty(nbytes, device=x.device, dtype=torch.uint8)
        o = [torch.empty((m, i), device=x.device, dtype=torch.bfloat16) for _ in range(3)]
        _lib.check(lib.molt_nf4_gateup_forward(x.data_ptr(), h, m, ops.C.byref(wg), ops.C.byref(wu),
                                               tt.data_ptr(), 2 * r, bg.data_ptr(), bu.data_ptr(), r, 2.0, 0.5,
                                               o[0].data_ptr(), o[1].data_ptr(), o[2].data_ptr(), i,
                                               ws.data_ptr(), nbytes, ops._stream(x.device)))
        return o

    # one row of T made infinite: the ring step's columns past 2r re-read the row's own T values, so
    # the other rows stay bitwise those of the clean T, on both paths
    bad = t.clone()
    bad[7] = float("inf")
    with tuning(big_tile_min=1, stage_min_mtiles=1):
        assert lib.molt_nf4_gateup_forward_workspace(m, i, h, r) > lib.molt_nf4_gateup_forward_workspace(m, i, h, 0)
        outs = [run(t, rank) for rank in (0, r)]
        poisoned = [run(bad, rank) for rank in (0, r)]
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    keep = torch.arange(m, device=x.device) != 7
    for clean, hit in zip(outs[0], poisoned[1]):
        assert torch.equal(clean[keep], hit[keep])
    assert not torch.isfinite(poisoned[1][0][7].float()).all()
    # and against the oracle of the pair with its LoRA terms
    xs, ts = bf16_values(x), bf16_values(t)
    g_ref = xs @ oracle_weight(pg, qg).dequant_bf16().astype(np.float64).T + ts[:, :r] @ (
        bf16_values((2.0 * bg).to(torch.bfloat16)).T)
    assert_close_fro(np_f32(outs[1][0]), g_ref, what="gate")


def test_paired_backward_reads_u_halves_in_place():
    """U_g and U_u as the column halves of one matrix (one row stride, as the
    fused MLP's backward passes them) give the result of contiguous copies."""
    m, i, h, r = 300, 256, 512, 16
    print(f"paired backward, strided U m={m} I={i} H={h} r={r}", flush=True)
    p0, q0, s0 = _weight(i, h, 66)
    p1, q1, s1 = _weight(i, h, 67)
    d0, d1 = seeded((m, i), 68), seeded((m, i), 69)
    u = seeded((m, 2 * r), 70)
    a0, a1 = uniform((r, h), 71, 0.05), uniform((r, h), 72, 0.05)
    outs = [ops.nf4_lora_backward_input_pair(d0, d1, p0, s0, p1, s1, q0.code, i, h, 1, ug, uu, a0, a1)
            for ug, uu in ((u[:, :r], u[:, r:]), (u[:, :r].contiguous(), u[:, r:].contiguous()))]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
