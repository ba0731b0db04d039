"""Argument checks of the frozen-head cross-entropy (no GPU): the reference's
own refusal and validation tests (tests/kernels/test_frozen_linear_cross_entropy.py:80-120),
run where they fail before any device work."""
from __future__ import annotations

import pytest
import torch

from molt_amd.kernels.frozen_linear_cross_entropy import frozen_linear_cross_entropy
from molt_amd.kernels.partitioned_loss import exact_partitioned_linear_cross_entropy


def test_refusal_when_weight_requires_grad():
    h = torch.randn(4, 16, requires_grad=True)
    w = torch.randn(32, 16, requires_grad=True)
    t = torch.randint(32, (4,))
    with pytest.raises(ValueError, match="requires a frozen classifier"):
        frozen_linear_cross_entropy(h, w, t, 2)


def test_explicit_fused_backend_never_silently_falls_back_on_cpu():
    h = torch.randn(4, 16, requires_grad=True)
    w = torch.randn(32, 16)
    t = torch.randint(32, (4,))
    with pytest.raises(RuntimeError, match="unavailable"):
        exact_partitioned_linear_cross_entropy(h, w, t, 2, precompute_frozen_gradient=True, backend="triton")


def test_validation_errors():
    w = torch.randn(32, 16)
    t = torch.randint(32, (4,))
    with pytest.raises(ValueError, match="hidden must be"):
        frozen_linear_cross_entropy(torch.randn(16), w, t, 2)
    with pytest.raises(ValueError, match="targets must match"):
        frozen_linear_cross_entropy(torch.randn(4, 16), w, torch.randint(32, (5,)), 2)
    with pytest.raises(ValueError, match="hidden width and classifier weight width must match"):
        frozen_linear_cross_entropy(torch.randn(4, 16), torch.randn(32, 20), t, 2)
    with pytest.raises(ValueError, match="chunk_size must be positive"):
        frozen_linear_cross_entropy(torch.randn(4, 16), w, t, 0)
    with pytest.raises(ValueError, match="Unknown backend"):
        exact_partitioned_linear_cross_entropy(torch.randn(4, 16), w, t, 2, backend="cuda")
