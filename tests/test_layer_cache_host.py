"""dense_nf4_layer_cache behaviour on the CPU: the reference's four tests
(tests/training/test_nf4_layer_cache.py:48-91) restated on this package's
NF4-LoRA module, with the NF4 decode replaced by a stub (as the reference
stubs bitsandbytes' dequantize_4bit) so that no GPU is needed."""
from __future__ import annotations

import pytest
import torch

import molt_amd
from molt_amd.errors import CapabilityError
from molt_amd.methods import nf4_layer_cache
from molt_amd.methods.nf4_layer_cache import dense_nf4_layer_cache
from molt_amd.modules import NF4Linear, NF4LoRALinear
from molt_amd.nf4 import QuantState


def _layer(monkeypatch: pytest.MonkeyPatch):
    qs = QuantState(torch.ones(1), (1, 1), molt_amd.NF4_CODEBOOK, blocksize=64)
    base = NF4Linear(torch.zeros(1, dtype=torch.uint8), qs)
    base.forward = lambda inputs: inputs + 7          # stands in for the NF4 GEMM
    layer = torch.nn.Sequential(NF4LoRALinear(base, 1, 1.0))
    monkeypatch.setattr(nf4_layer_cache, "dequantize_4bit", lambda data, quant_state: torch.tensor([[2.0]]))
    return layer, base


def test_dense_nf4_cache_restores_forward_after_success(monkeypatch):
    layer, base = _layer(monkeypatch)
    original = base.forward
    inputs = torch.tensor([[3.0]], dtype=torch.bfloat16)
    with dense_nf4_layer_cache(layer) as projection_count:
        assert projection_count == 1
        torch.testing.assert_close(base(inputs), torch.tensor([[6.0]], dtype=torch.bfloat16))
    assert base.forward == original
    torch.testing.assert_close(base(inputs), torch.tensor([[10.0]], dtype=torch.bfloat16))


def test_dense_nf4_cache_restores_forward_after_error(monkeypatch):
    layer, base = _layer(monkeypatch)
    original = base.forward
    with pytest.raises(RuntimeError, match="injected"):
        with dense_nf4_layer_cache(layer):
            raise RuntimeError("injected")
    assert base.forward == original


def test_dense_nf4_cache_rejects_layer_without_nf4_projection():
    with pytest.raises(CapabilityError, match="contains no PEFT NF4"):
        with dense_nf4_layer_cache(torch.nn.Sequential(torch.nn.Linear(2, 2))):
            pass


def test_dense_nf4_cache_rejects_biased_projection(monkeypatch):
    layer, base = _layer(monkeypatch)
    original = base.forward
    base.bias = torch.tensor([0.5], dtype=torch.bfloat16)
    with pytest.raises(CapabilityError, match="biased NF4"):
        with dense_nf4_layer_cache(layer):
            pass
    assert base.forward == original


def test_dense_nf4_cache_rejects_trainable_base_and_restores_earlier_patches(monkeypatch):
    layer, base = _layer(monkeypatch)
    qs = QuantState(torch.ones(1), (1, 1), molt_amd.NF4_CODEBOOK, blocksize=64)
    second = NF4Linear(torch.zeros(1, dtype=torch.uint8), qs)
    second.weight = torch.nn.Parameter(torch.zeros(1), requires_grad=True)   # an unfrozen base
    second.weight.quant_state = qs
    layer.append(NF4LoRALinear(second, 1, 1.0))
    original = base.forward
    with pytest.raises(CapabilityError, match="frozen NF4"):
        with dense_nf4_layer_cache(layer):
            pass
    assert base.forward == original
