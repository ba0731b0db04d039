"""Split-K GEMMs: a long contraction with too few output tiles to fill the GPU
runs over several workgroups per tile whose fp32 partials are summed in split
order. The 256 x 256 kernels split the cfg3 down projection and the paired
gate/up input gradient at M = 4096; the 128 x 128 kernels split the narrow
grouped-query k/v projection (1536 -> 256) and small ragged shapes. Checked
against the fp64 oracle (5e-3), against the unsplit kernels (same values up to
fp32 summation order), and for bitwise repeatability."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as O
from tests._util import assert_close_fro, bf16_values, np_f32, oracle_weight, seeded, uniform

import molt_amd
from molt_amd import _lib, ops
from molt_amd._lib import tuning

pytestmark = pytest.mark.gpu


def _weight(out_f, in_f, seed):
    w = seeded((out_f, in_f), seed, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    return packed.reshape(-1), qs, molt_amd.resolved_nf4_scales(qs)


def _rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("m,n,k,r", [(4096, 1536, 8960, 16), (512, 512, 4096, 8), (300, 256, 2048, 0),
                                     (4096, 256, 1536, 16), (300, 384, 1024, 8), (77, 136, 512, 5)])
def test_split_forward(m, n, k, r):
    print(f"split-K forward m={m} n={n} k={k} r={r}", flush=True)
    lib = _lib.load()
    assert lib.molt_nf4_lora_forward_workspace(m, n, k, r) > 0, "the shape must take the split path"
    packed, qs, scales = _weight(n, k, 11)
    x = seeded((m, k), 12)
    a = uniform((max(r, 1), k), 13, 1 / np.sqrt(k))
    b = seeded((n, max(r, 1)), 14, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0) if r else None
    bb = b if r else None

    def run():
        return ops.nf4_lora_forward(x, packed, scales, qs.code, n, k, 1, 64, t, bb, 2.0)

    y1, y2 = run(), run()
    with tuning(split_k=0):
        y0 = run()
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), "split-K forward is not repeatable"
    assert _rel(y1.float(), y0.float()) <= 2e-3
    rows = np.sort(np.random.default_rng(1).choice(m, min(m, 96), replace=False))
    wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    ref = bf16_values(x)[rows] @ wo.T
    if r:
        ref = ref + 2.0 * (bf16_values(t)[rows] @ bf16_values(b).T)
    assert_close_fro(np_f32(y1)[rows], ref, what="split-K Y rows")


@pytest.mark.parametrize("m,nw,kw,pair,r", [(4096, 8960, 1536, True, 16), (4096, 8960, 1536, False, 16),
                                            (512, 4096, 512, True, 8), (200, 2048, 256, False, 0),
                                            (512, 1536, 1536, False, 16), (200, 1024, 384, True, 8)])
def test_split_backward(m, nw, kw, pair, r):
    print(f"split-K backward m={m} nw={nw} kw={kw} pair={pair} r={r}", flush=True)
    lib = _lib.load()
    assert lib.molt_nf4_lora_backward_workspace(m, nw, kw, 2 if pair else 1) > 0
    w0 = _weight(nw, kw, 21)
    w1 = _weight(nw, kw, 22) if pair else None
    dy0, dy1 = seeded((m, nw), 23), seeded((m, nw), 24)
    u0, u1 = seeded((m, max(r, 1)), 25), seeded((m, max(r, 1)), 26)
    a0 = uniform((max(r, 1), kw), 27, 1 / np.sqrt(kw))
    a1 = uniform((max(r, 1), kw), 28, 1 / np.sqrt(kw))

    def run():
        if pair:
            return ops.nf4_lora_backward_input_pair(dy0, dy1, w0[0], w0[2], w1[0], w1[2], w0[1].code, nw, kw, 1,
                                                    u0 if r else None, u1 if r else None, a0 if r else None,
                                                    a1 if r else None)
        return ops.nf4_lora_backward_input(dy0, w0[0], w0[2], w0[1].code, nw, kw, 1, 64, u0 if r else None,
                                           a0 if r else None, 1.0)

    d1, d2 = run(), run()
    with tuning(split_k=0):
        d0 = run()
    torch.cuda.synchronize()
    assert torch.equal(d1, d2), "split-K backward is not repeatable"
    assert _rel(d1.float(), d0.float()) <= 2e-3
    rows = np.sort(np.random.default_rng(2).choice(m, min(m, 64), replace=False))
    ref = bf16_values(dy0)[rows] @ oracle_weight(w0[0], w0[1]).dequant_bf16().astype(np.float64)
    if r:
        ref = ref + bf16_values(u0)[rows] @ bf16_values(a0)
    if pair:
        ref = ref + bf16_values(dy1)[rows] @ oracle_weight(w1[0], w1[1]).dequant_bf16().astype(np.float64)
        if r:
            ref = ref + bf16_values(u1)[rows] @ bf16_values(a1)
    assert_close_fro(np_f32(d1)[rows], ref, what="split-K dX rows")
