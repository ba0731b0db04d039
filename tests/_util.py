"""Helpers shared by the GPU parity tests: seeded inputs and oracle views of
device tensors. Tolerance for every floating-point comparison: relative
Frobenius error <= 5e-3 against an fp64 oracle over the same bf16 operands
(the acceptance bar of the NF4 QLoRA hot path)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import nf4_oracle as O

TOL = 5e-3


def np_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def np_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def bf16_values(t: torch.Tensor) -> np.ndarray:
    """bf16 or fp32 tensor -> fp64 numpy of its bf16-rounded values."""
    return O.bf16_round(np_f32(t)).astype(np.float64)


def oracle_weight(packed: torch.Tensor, qs) -> O.OracleNF4:
    """Oracle view of a device NF4 weight (packed bytes + statistics read back)."""
    rows, cols = int(qs.shape[0]), int(np.prod(qs.shape[1:]))
    t = O.OracleNF4(packed.reshape(-1).cpu().numpy(), (rows, cols), int(qs.blocksize),
                    int(getattr(qs, "nibble_order", 1)), np_f32(qs.code), None, None)
    if qs.nested:
        t.nested = True
        t.q = qs.absmax.cpu().numpy()
        t.absmax2 = np_f32(qs.state2.absmax)
        t.code2 = np_f32(qs.state2.code)
        t.offset = np.float32(float(qs.offset))
        t.scales = O.resolve_scales(t.q, t.absmax2, t.code2, t.offset, int(qs.state2.blocksize))
    else:
        t.scales = np_f32(qs.absmax)
    t.absmax = t.scales
    return t


def seeded(shape, seed: int, std: float = 1.0, device="cuda", dtype=torch.bfloat16) -> torch.Tensor:
    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(device=device, dtype=dtype)


def uniform(shape, seed: int, bound: float, device="cuda") -> torch.Tensor:
    g = torch.Generator(device="cpu").manual_seed(seed)
    return ((torch.rand(*shape, generator=g) * 2 - 1) * bound).to(device=device, dtype=torch.float32)


def assert_close_fro(actual, expected, tol: float = TOL, what: str = "") -> float:
    err = O.rel_fro(actual, expected)
    assert err <= tol, f"{what}: relative Frobenius error {err:.3e} > {tol:.1e}"
    return err
