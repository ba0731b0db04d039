"""The rank-r LoRA kernels on their own: the projection T = z . bf16(W)^T
(plain, SwiGLU-replayed and pre-scaled activations, both adapter layouts) and
the adapter gradients scale * L^T R, against fp64 products of the same bf16
operands. Shapes cover row, depth and rank tails, unaligned widths (the
element-wise load path), every rank tile count up to 128, the two-tile row
blocking of long inputs and the split-M reduction."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as O
from tests._util import assert_close_fro, bf16_values, np_f32, seeded, uniform

import molt_amd
from molt_amd import _lib, ops
from molt_amd.errors import CapabilityError

pytestmark = pytest.mark.gpu


def _effective(z, z2, mode, scale):
    """The activation the kernels contract, in fp64: z, bf16(bf16(silu(z)) z2) or bf16(scale z)."""
    a = bf16_values(z)
    if mode == 1:
        b = bf16_values(z2)
        return O.bf16_round(O.bf16_round(a / (1.0 + np.exp(-a))) * b).astype(np.float64)
    if mode == 2:
        return O.bf16_round(a * np.float32(scale)).astype(np.float64)
    return a


@pytest.mark.parametrize("m,d,r,mode,layout", [
    (1, 64, 8, 0, 0),
    (37, 200, 16, 0, 0),        # depth tail inside the last 64-deep step
    (70, 203, 16, 0, 0),        # width not a multiple of 8: element-wise loads
    (300, 4096, 64, 2, 1),      # pre-scaled dY against LoRA B ([D, r])
    (129, 1000, 128, 0, 0),     # four 32-wide rank tiles
    (64, 520, 96, 1, 0),        # SwiGLU replay, three rank tiles
    (77, 130, 40, 1, 1),        # replay with unaligned width
    (16424, 256, 64, 0, 0),     # two 32-row tiles per workgroup, row tail
    (16384, 128, 32, 2, 1),
])
def test_lora_project(m, d, r, mode, layout):
    print(f"lora_project m={m} d={d} r={r} mode={mode} layout={layout}", flush=True)
    z = seeded((m, d), 1)
    z2 = seeded((m, d), 2) if mode == 1 else None
    w = uniform((r, d) if layout == 0 else (d, r), 3, 1 / np.sqrt(d))
    scale = 0.75
    out = ops.lora_project(z, z2, mode, scale, w, layout)
    again = ops.lora_project(z, z2, mode, scale, w, layout)
    assert torch.equal(out, again)
    wr = bf16_values(w)
    ref = _effective(z, z2, mode, scale) @ (wr.T if layout == 0 else wr)
    assert out.shape == (m, r)
    assert_close_fro(np_f32(out), O.bf16_round(ref), what="T")


def test_lora_project_rejects_rank_above_128():
    z = seeded((8, 64), 4)
    w = uniform((160, 64), 5, 0.1)
    with pytest.raises(molt_amd.CapabilityError):
        ops.lora_project(z, None, 0, 1.0, w, 0)


@pytest.mark.parametrize("m,p,q,mode,layout,scale", [
    (5, 64, 8, 0, 0, 1.0),
    (300, 200, 16, 0, 1, 1.0),
    (1000, 203, 13, 0, 0, 0.5),   # unaligned widths: element-wise loads
    (4099, 512, 64, 1, 1, 1.0),   # SwiGLU replay of L, row tail
    (9000, 1024, 64, 0, 0, 2.0),  # split-M partials summed in order
    (2048, 384, 128, 0, 1, 1.0),  # two rank tiles
])
def test_lora_grad(m, p, q, mode, layout, scale):
    print(f"lora_grad m={m} p={p} q={q} mode={mode} layout={layout}", flush=True)
    l = seeded((m, p), 6)
    l2 = seeded((m, p), 7) if mode == 1 else None
    rmat = seeded((m, q), 8)
    out = ops.lora_grad(l, l2, mode, rmat, scale, layout)
    again = ops.lora_grad(l, l2, mode, rmat, scale, layout)
    assert torch.equal(out, again)
    ref = scale * (_effective(l, l2, mode, 1.0).T @ bf16_values(rmat))
    if layout == 1:
        ref = ref.T
    assert out.shape == ref.shape
    assert_close_fro(np_f32(out), ref, tol=1e-5, what="grad")


def test_lora_grad_empty_rows_gives_zeros():
    l = torch.empty((0, 64), device="cuda", dtype=torch.bfloat16)
    rmat = torch.empty((0, 16), device="cuda", dtype=torch.bfloat16)
    out = ops.lora_grad(l, None, 0, rmat, 1.0, 1)
    assert out.shape == (16, 64)
    assert torch.count_nonzero(out).item() == 0


@pytest.mark.parametrize("m,d,r", [(300, 4096, 64), (8192, 1024, 16), (70, 200, 8)])
def test_lora_project_pair_is_the_two_projections_side_by_side(m, d, r):
    """The gate/up U pair written as column halves of one matrix equals the two
    separate pre-scaled projections bit for bit (shapes where the pair launch
    splits D as a single projection does, or falls back to two)."""
    print(f"lora_project_pair m={m} d={d} r={r}", flush=True)
    z0, z1 = seeded((m, d), 11), seeded((m, d), 12)
    b0, b1 = uniform((d, r), 13, 1 / np.sqrt(d)), uniform((d, r), 14, 1 / np.sqrt(d))
    pair = ops.lora_project_pair(z0, z1, 0.5, 2.0, b0, b1)
    u0 = ops.lora_project(z0, None, 2, 0.5, b0, 1)
    u1 = ops.lora_project(z1, None, 2, 2.0, b1, 1)
    assert pair.shape == (m, 2 * r)
    assert torch.equal(pair[:, :r], u0) and torch.equal(pair[:, r:], u1)


def test_lora_project_of_an_activation_beyond_4gib():
    """z of 4.3 GB: byte offsets past 2^32 do not fit the DMA kernel's 32-bit
    buffer offsets (they wrapped before the projection checked the range), so
    such a z takes the register kernel; its first and last rows against torch
    over the same bf16 operands."""
    m, d, r = 131200, 16384, 16
    print(f"lora_project m={m} d={d} r={r} ({m * d * 2 / 2**30:.2f} GiB of z)", flush=True)
    g = torch.Generator(device="cuda").manual_seed(7)
    z = torch.empty((m, d), device="cuda", dtype=torch.bfloat16)
    z.normal_(generator=g)
    a = uniform((r, d), 8, d ** -0.5)
    out = ops.lora_project(z, None, 0, 1.0, a, 0)
    ab = a.to(torch.bfloat16).float()
    for rows in (slice(0, 128), slice(m - 128, m)):
        ref = (z[rows].float() @ ab.T).double().cpu().numpy()
        assert_close_fro(np_f32(out[rows]), O.bf16_round(ref), what=f"T rows {rows.start}..{rows.stop}")
    del z
    torch.cuda.empty_cache()


@pytest.mark.parametrize("m,d,r,same_split", [(4096, 8960, 16, False), (2048, 2048, 32, True)])
def test_lora_project_pair_one_launch(m, d, r, same_split):
    """The pair as one launch (molt_lora_project_pair_packed): its split over D
    counts both operands' row blocks, so cfg3's U_g / U_u (4096 x 8960, r = 16)
    run unsplit where a single projection splits D in two. Each half against
    the fp64 oracle of its pre-scaled projection, and bit for bit against the
    single projection where the split counts agree."""
    print(f"lora_project_pair_packed one launch m={m} d={d} r={r}", flush=True)
    lib = _lib.load()
    # unsplit, the pair needs no partials (only the fallback's room); split, two planes of them
    assert (lib.molt_lora_project_pair_packed_workspace(m, d, r) > lib.molt_lora_project_packed_workspace(m, d, r)) \
        == same_split
    z0, z1 = seeded((m, d), 15), seeded((m, d), 16)
    b0, b1 = uniform((d, r), 17, 1 / np.sqrt(d)), uniform((d, r), 18, 1 / np.sqrt(d))
    packs = ops.lora_pack_many([b0, b1], [None, None], [1, 1])
    pair = ops.lora_project_pair_packed(z0, z1, 0.5, 2.0, packs[0], packs[1], r)
    singles = [ops.lora_project(z, None, 2, sc, b, 1) for z, sc, b in ((z0, 0.5, b0), (z1, 2.0, b1))]
    torch.cuda.synchronize()
    for half, (z, sc, b) in enumerate(((z0, 0.5, b0), (z1, 2.0, b1))):
        got = pair[:, half * r:(half + 1) * r]
        ref = _effective(z, None, 2, sc) @ bf16_values(b)
        assert_close_fro(np_f32(got), O.bf16_round(ref), what=f"U half {half}")
        if same_split:
            assert torch.equal(got, singles[half])
        else:
            assert_close_fro(np_f32(got), np_f32(singles[half]).astype(np.float64), tol=2e-3,
                             what=f"U half {half} vs its own launch")


@pytest.mark.parametrize("m,p,q,layout", [(4099, 512, 64, 0), (2048, 384, 64, 1), (300, 200, 16, 0)])
def test_lora_grad_reads_a_column_slice_in_place(m, p, q, layout):
    """R given as the column half of a wider matrix (row stride 2q, passed as
    ldr) gives the gradient of the same values made contiguous, bit for bit."""
    print(f"lora_grad strided R m={m} p={p} q={q} layout={layout}", flush=True)
    l = seeded((m, p), 15)
    wide = seeded((m, 2 * q), 16)
    for half in (wide[:, :q], wide[:, q:]):
        assert not half.is_contiguous()
        assert torch.equal(ops.lora_grad(l, None, 0, half, 1.5, layout),
                           ops.lora_grad(l, None, 0, half.contiguous(), 1.5, layout))


@pytest.mark.parametrize("m,p,q,layout,strided", [
    (300, 200, 16, 1, False),     # one step, tails in P and Q
    (4099, 512, 64, 0, False),    # row tail in the last slice, several slices
    (1000, 136, 24, 0, True),     # P past one 128 tile, R a column slice (row stride 2q)
    (2048, 384, 128, 1, False),   # two rank tiles
    (8192, 4096, 128, 1, True),   # cfg4's paired dA over X, U halves of one matrix
    (5000, 14336, 64, 0, False),  # long rows (dB over dg)
    (3000, 8960, 80, 1, False),   # a 64-column rank tile, then a 16-column one (narrow-Q waves)
    (4096, 8960, 16, 0, False),   # cfg3's dB over dg: one narrow rank tile
])
def test_lora_grad_dma_kernel_equals_the_register_kernel(m, p, q, layout, strided):
    """The DMA-staged gradient kernel (plain aligned operands) has the same
    tiles, slices and MFMA operands as the register-staged one: bitwise equal."""
    print(f"lora_grad DMA vs register m={m} p={p} q={q} layout={layout} strided={strided}", flush=True)
    l = seeded((m, p), 17)
    wide = seeded((m, 2 * q), 18)
    rmat = wide[:, q:] if strided else wide[:, :q].contiguous()
    with molt_amd._lib.tuning(lora_dma=1):
        dma = ops.lora_grad(l, None, 0, rmat, 0.5, layout)
    with molt_amd._lib.tuning(lora_dma=0):
        reg = ops.lora_grad(l, None, 0, rmat, 0.5, layout)
    torch.cuda.synchronize()
    assert torch.equal(dma, reg)


@pytest.mark.parametrize("m,p,q,layout", [(300, 200, 16, 1), (4099, 512, 64, 1), (8192, 14336, 64, 1),
                                          (2048, 384, 128, 0), (4096, 8960, 16, 1), (1000, 700, 32, 0)])
def test_lora_grad_dma_replay_equals_register_and_materialised(m, p, q, layout):
    """The DMA-staged SwiGLU-replay gradient equals the register-staged replay
    and the gradient over the materialised h = bf16(bf16(silu(g)) u), bit for bit."""
    print(f"lora_grad replay DMA m={m} p={p} q={q} layout={layout}", flush=True)
    g, u = seeded((m, p), 19), seeded((m, p), 20)
    rmat = seeded((m, q), 21)
    h = ops.silu_mul_forward(g, u, True)
    with molt_amd._lib.tuning(lora_dma=1):
        dma = ops.lora_grad(g, u, 1, rmat, 1.0, layout)
        mat = ops.lora_grad(h, None, 0, rmat, 1.0, layout)
    with molt_amd._lib.tuning(lora_dma=0):
        reg = ops.lora_grad(g, u, 1, rmat, 1.0, layout)
    torch.cuda.synchronize()
    assert torch.equal(dma, reg)
    assert torch.equal(dma, mat)


@pytest.mark.parametrize("case", ["cfg4_mlp", "projection_pair", "mixed_fallback"])
def test_lora_grad_many_equals_separate_calls(case):
    """Several gradients from one launch pair (molt_lora_grad_many) equal the
    separate lora_grad calls bit for bit: the cfg4 gated-MLP backward's five
    (dB over dY, dg, du with the column halves of T, dA over h, the paired dA
    over X), a scheduled projection's dA/dB pair, and a set with an unaligned
    and an empty gradient (run one after another)."""
    print(f"lora_grad_many {case}", flush=True)
    if case == "cfg4_mlp":
        m, h, i, r = 8192, 4096, 14336, 64
        dy, dg, du, hh, x = seeded((m, h), 30), seeded((m, i), 31), seeded((m, i), 32), seeded((m, i), 33), \
            seeded((m, h), 34)
        t_d, t_gu, u_d, u_gu = seeded((m, r), 35), seeded((m, 2 * r), 36), seeded((m, r), 37), seeded((m, 2 * r), 38)
        sets = [(dy, None, 0, t_d, 2.0, 0), (dg, None, 0, t_gu[:, :r], 2.0, 0), (du, None, 0, t_gu[:, r:], 2.0, 0),
                (hh, None, 0, u_d, 1.0, 1), (x, None, 0, u_gu, 1.0, 1)]
    elif case == "projection_pair":
        m, k, n, r = 4096, 1536, 256, 16
        x, g = seeded((m, k), 40), seeded((m, n), 41)
        u, t = seeded((m, r), 42), seeded((m, r), 43)
        sets = [(x, None, 0, u, 1.0, 1), (g, None, 0, t, 0.5, 0)]
    else:
        sets = [(seeded((300, 200), 50), None, 0, seeded((300, 16), 51), 1.0, 1),
                (seeded((1000, 203), 52), None, 0, seeded((1000, 13), 53), 0.5, 0),   # unaligned widths
                (torch.empty((0, 64), device="cuda", dtype=torch.bfloat16), None, 0,
                 torch.empty((0, 16), device="cuda", dtype=torch.bfloat16), 1.0, 1),
                (seeded((4099, 512), 54), seeded((4099, 512), 55), 1, seeded((4099, 64), 56), 1.0, 1)]
    sep = [ops.lora_grad(*s_) for s_ in sets]
    many = ops.lora_grad_many([s_[0] for s_ in sets], [s_[1] for s_ in sets], [s_[2] for s_ in sets],
                              [s_[3] for s_ in sets], [s_[4] for s_ in sets], [s_[5] for s_ in sets])
    again = ops.lora_grad_many([s_[0] for s_ in sets], [s_[1] for s_ in sets], [s_[2] for s_ in sets],
                               [s_[3] for s_ in sets], [s_[4] for s_ in sets], [s_[5] for s_ in sets])
    torch.cuda.synchronize()
    assert len(many) == len(sets)
    for a_, b_, c_ in zip(sep, many, again):
        assert a_.shape == b_.shape
        assert torch.equal(a_, b_) and torch.equal(b_, c_)


def test_lora_grad_many_with_replayed_operands():
    """The RMSNorm-replay recipe's adapter gradients at cfg3's shapes as one
    call: dB over dY, dg and du (one launch together), dA_d over h replayed
    from gate and up, dA_gate / dA_up over the RMSNorm output replayed from
    its source, and one split-sum launch. Each is bitwise its own lora_grad /
    lora_grad_rmsnorm call. A replayed norm whose rows the kernel cannot take
    is refused before any launch."""
    m, h, i, r = 4096, 1536, 8960, 16
    print(f"lora_grad_many with SwiGLU and RMSNorm replay m={m} H={h} I={i} r={r}", flush=True)
    dy, dg, du = seeded((m, h), 90), seeded((m, i), 91), seeded((m, i), 92)
    g, u = seeded((m, i), 93), seeded((m, i), 94)
    src, w = seeded((m, h), 95, std=1.3), seeded((h,), 96, std=0.3)
    inv = ops.rmsnorm_inv(src, w, 1e-6)
    t_d, t_gu, u_d, u_gu = seeded((m, r), 97), seeded((m, 2 * r), 98), seeded((m, r), 99), seeded((m, 2 * r), 100)
    many = ops.lora_grad_many([dy, dg, du, g, src], [None, None, None, u, None], [0, 0, 0, 1, 2],
                              [t_d, t_gu[:, :r], t_gu[:, r:], u_d, u_gu], [2.0, 2.0, 2.0, 1.0, 1.0],
                              [0, 0, 0, 1, 1], inv, w, 0.25)
    sep = [ops.lora_grad(dy, None, 0, t_d, 2.0, 0), ops.lora_grad(dg, None, 0, t_gu[:, :r], 2.0, 0),
           ops.lora_grad(du, None, 0, t_gu[:, r:], 2.0, 0), ops.lora_grad(g, u, 1, u_d, 1.0, 1),
           ops.lora_grad_rmsnorm(src, inv, w, 0.25, u_gu, 1.0, 1)]
    torch.cuda.synchronize()
    for k, (a_, b_) in enumerate(zip(sep, many)):
        assert a_.shape == b_.shape and torch.equal(a_, b_), f"gradient {k}"
    bad, bad_w = seeded((64, 203), 101), seeded((203,), 102)    # 203 features: rows of 406 bytes
    with pytest.raises(CapabilityError):
        ops.lora_grad_many([bad], [None], [2], [seeded((64, 8), 103)], [1.0], [1],
                           torch.ones(64, device="cuda"), bad_w, 0.0)


@pytest.mark.parametrize("m,d,r,mode,layout,stacked", [
    (8192, 4096, 64, 0, 0, True),     # [A_gate; A_up] stacked without a copy (rank 128)
    (8192, 14336, 64, 0, 0, False),   # A_down over h
    (8192, 4096, 64, 2, 1, False),    # B_down over s dY
    (300, 4096, 16, 2, 1, True),      # small M: the K split and its partials; stacked B columns
    (70, 200, 8, 0, 0, False),        # tails (the register kernel)
])
def test_lora_pack_many_and_packed_projection_equal_lora_project(m, d, r, mode, layout, stacked):
    """Adapters packed several to a launch (molt_lora_pack_many) and projected
    without a pack launch give bitwise the output of lora_project on the same
    (stacked) adapter."""
    print(f"lora_pack_many + project_packed m={m} d={d} r={r} mode={mode} layout={layout} stacked={stacked}",
          flush=True)
    z = seeded((m, d), 60)
    shape = (r, d) if layout == 0 else (d, r)
    a0, a1 = uniform(shape, 61, 1 / np.sqrt(d)), uniform(shape, 62, 1 / np.sqrt(d))
    other = uniform((16, 96), 63, 0.1)   # a second adapter packed in the same launch
    packs = ops.lora_pack_many([other, a0], [None, a1 if stacked else None], [0, layout])
    full = torch.cat([a0, a1], 0 if layout == 0 else 1) if stacked else a0
    rr = 2 * r if stacked else r
    ref = ops.lora_project(z, None, mode, 0.5, full, layout)
    got = ops.lora_project_packed(z, None, mode, 0.5, packs[1], rr)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(ops.lora_project_packed(seeded((5, 96), 64), None, 0, 1.0, packs[0], 16),
                       ops.lora_project(seeded((5, 96), 64), None, 0, 1.0, other, 0))
    if layout == 1 and not stacked:
        z1 = seeded((m, d), 65)
        p2 = ops.lora_pack_many([a0, a1], [None, None], [1, 1])
        pair = ops.lora_project_pair_packed(z, z1, 0.5, 2.0, p2[0], p2[1], r)
        assert torch.equal(pair, ops.lora_project_pair(z, z1, 0.5, 2.0, a0, a1))
