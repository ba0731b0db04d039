"""Multi-step training check of the gated NF4-LoRA MLP (the role of the
reference's adapter-trajectory gate, benchmarks/nf4_trajectory_gate.py:85-112).

Twenty AdamW steps (MOLT's optimizer and default learning rate,
training/qlora.py:218-243, core/specs.py:118) of the cfg1 gated MLP through
``fused_gated_nf4_lora_mlp``, each step on its own seeded microbatch. Two
trajectories run beside it on the CPU from the same start, each independent
(neither sees the GPU's adapters):
* the fp64 oracle: gradients from the oracle in fp64 over the identical bf16
  operands (X, dY, the dequantised weights, the bf16 values of the adapters),
  AdamW in fp64;
* the reference's own bf16 step: gradients with every autocast rounding point
  of MOLT's path (``gated_mlp_reference_bf16``), fp32 masters, AdamW in fp32.
AdamW's first steps are close to ``lr * sign(g)``, so a gradient element
inside the bf16 noise can flip its update whichever bf16 path computes it; the
drift the per-step error causes is therefore judged against the reference
path's own drift from the fp64 trajectory. Checked at every step, for each of
the six adapters: the adapter and its accumulated update (adapter - start)
against the fp64 trajectory, no worse than 1.25x the reference path's error
(or an absolute floor); and two GPU runs from the same start agree bit for bit
at every step (the reference's gate requires bitwise-equal trajectories)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as O
from tests._util import oracle_weight, seeded, uniform

import molt_amd
from molt_amd.methods import fused_gated_nf4_lora_mlp

pytestmark = pytest.mark.gpu

H, I, R, M, S = 896, 4864, 16, 1024, 2.0
STEPS, LR = 20, 2e-4
RATIO = 1.25                  # HIP drift / reference-path drift, per adapter and step
FLOOR_ADAPTER, FLOOR_UPDATE = 1e-5, 1e-3   # below these the comparison is not made


def _proj(out_f, in_f, seed):
    w = seeded((out_f, in_f), seed, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    a = uniform((R, in_f), seed + 1, 1.0 / np.sqrt(in_f))
    b = seeded((out_f, R), seed + 2, std=0.01, dtype=torch.float32)
    return packed, qs, a, b


def _gpu_trajectory(projs, batches):
    (pg, qg, _, _), (pu, qu, _, _), (pd, qd, _, _) = projs
    leaves = [t.detach().clone().requires_grad_() for _, _, a, b in projs for t in (a, b)]
    opt = torch.optim.AdamW(leaves, lr=LR)
    snaps = []
    for x, dy in batches:
        opt.zero_grad(set_to_none=True)
        y = fused_gated_nf4_lora_mlp(x, pg, leaves[0], leaves[1], pu, leaves[2], leaves[3], pd, leaves[4],
                                     leaves[5], qg, qu, qd, S, S, S)
        y.backward(dy)
        opt.step()
        snaps.append([t.detach().clone() for t in leaves])
    torch.cuda.synchronize()
    return snaps


def test_cfg1_adamw_trajectory_follows_the_fp64_oracle_and_repeats_bitwise():
    print(f"trajectory: cfg1 gated MLP, {STEPS} AdamW steps (lr {LR})", flush=True)
    projs = [_proj(I, H, 1300), _proj(I, H, 1310), _proj(H, I, 1320)]
    batches = [(seeded((M, H), 1400 + 2 * i), seeded((M, H), 1401 + 2 * i)) for i in range(STEPS)]
    first = _gpu_trajectory(projs, batches)
    second = _gpu_trajectory(projs, batches)
    for step, (sa, sb) in enumerate(zip(first, second)):
        for ta, tb in zip(sa, sb):
            assert torch.equal(ta, tb), f"step {step}: the two GPU runs differ"
    print("trajectory: GPU runs bitwise equal at every step", flush=True)

    ws = [oracle_weight(p, q).dequant_bf16().astype(np.float64) for p, q, _, _ in projs]
    start = [t.detach().cpu().double() for _, _, a, b in projs for t in (a, b)]
    exact = [t.clone().requires_grad_() for t in start]
    emul = [t.float().clone().requires_grad_() for t in start]
    opt_exact, opt_emul = torch.optim.AdamW(exact, lr=LR), torch.optim.AdamW(emul, lr=LR)
    names = ("A_gate", "B_gate", "A_up", "B_up", "A_down", "B_down")

    def rel(a, b):
        return float(torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b))

    worst = {"adapter": (0.0, 0.0), "update": (0.0, 0.0)}
    print(f"  {'step':>4s} {'adapter HIP':>12s} {'reference':>10s} {'update HIP':>11s} {'reference':>10s}",
          flush=True)
    for step, (x, dy) in enumerate(batches):
        xo = O.bf16_round(x.float().cpu().numpy()).astype(np.float64)
        dyo = O.bf16_round(dy.float().cpu().numpy()).astype(np.float64)
        ops = [O.bf16_round(t.detach().numpy().astype(np.float32)).astype(np.float64) for t in exact]
        _, saved = O.gated_mlp_forward(xo, ws[0], ws[1], ws[2], *ops, S)
        _, grads = O.gated_mlp_backward(xo, ws[0], ws[1], ws[2], *ops, S, dyo, saved)
        masters = [t.detach().numpy().astype(np.float64) for t in emul]
        _, _, egrads = O.gated_mlp_reference_bf16(xo, ws[0], ws[1], ws[2], *masters, S, dyo)
        for opt, leaves, gs, dt in ((opt_exact, exact, grads, np.float64), (opt_emul, emul, egrads, np.float32)):
            opt.zero_grad(set_to_none=True)
            for t, gr in zip(leaves, gs):
                t.grad = torch.from_numpy(np.ascontiguousarray(gr, dtype=dt))
            opt.step()
        rows = []
        for name, got, want, ref, s0 in zip(names, first[step], exact, emul, start):
            g64, w64, r64 = got.cpu().double(), want.detach(), ref.detach().double()
            rows.append((name, rel(g64, w64), rel(r64, w64), rel(g64 - s0, w64 - s0), rel(r64 - s0, w64 - s0)))
        top = [max(r[i] for r in rows) for i in (1, 2, 3, 4)]
        if step in (0, 1, 4, 9, 14, 19):
            print(f"  {step + 1:4d} {top[0]:12.2e} {top[1]:10.2e} {top[2]:11.2e} {top[3]:10.2e}", flush=True)
        worst["adapter"] = max(worst["adapter"], (top[0], top[1]))
        worst["update"] = max(worst["update"], (top[2], top[3]))
        for name, ea, ra, eu, ru in rows:
            assert ea <= max(RATIO * ra, FLOOR_ADAPTER), \
                f"step {step + 1} {name}: adapter error {ea:.3e} vs the reference path's {ra:.3e}"
            assert eu <= max(RATIO * ru, FLOOR_UPDATE), \
                f"step {step + 1} {name}: update error {eu:.3e} vs the reference path's {ru:.3e}"
    print(f"trajectory: over {STEPS} steps, worst adapter error HIP {worst['adapter'][0]:.2e} "
          f"(reference bf16 {worst['adapter'][1]:.2e}), worst update error HIP {worst['update'][0]:.2e} "
          f"(reference bf16 {worst['update'][1]:.2e})", flush=True)
