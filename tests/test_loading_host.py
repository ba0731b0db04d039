"""Host-side checks of the load-time preparation and the bitsandbytes 4-bit
serialisation (no GPU): target selection, and the packed quant-state
dictionary round trip."""
from __future__ import annotations

import json

import pytest
import torch

from molt_amd.errors import CapabilityError
from molt_amd.loading import _targets, quant_state_as_dict, quant_state_from_dict
from molt_amd.nf4 import QuantState


def _tiny_llama():
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=50, tie_word_embeddings=False)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg)


def test_all_linear_targets_every_projection_but_the_output_head():
    model = _tiny_llama()
    names = [n for _, _, _, n in _targets(model, "all-linear")]
    assert len(names) == 14 and not any("lm_head" in n for n in names)
    assert "model.layers.1.self_attn.k_proj" in names and "model.layers.0.mlp.down_proj" in names
    mlp_only = [n for _, _, _, n in _targets(model, ("gate_proj", "up_proj", "down_proj"))]
    assert len(mlp_only) == 6 and all(".mlp." in n for n in mlp_only)


def _state(nested: bool) -> QuantState:
    g = torch.Generator().manual_seed(3)
    code = torch.linspace(-1, 1, 16)
    if not nested:
        return QuantState(torch.rand(24, generator=g), (32, 48), code, 64, "nf4", torch.bfloat16)
    s2 = QuantState(torch.rand(1, generator=g), (1,), torch.linspace(-1, 1, 256), 256, "dynamic", torch.float32)
    absmax_q = torch.randint(0, 256, (24,), generator=g, dtype=torch.uint8)
    return QuantState(absmax_q, (32, 48), code, 64, "nf4", torch.bfloat16, torch.tensor(0.125), s2)


@pytest.mark.parametrize("nested", [True, False])
def test_quant_state_dict_round_trip(nested):
    qs = _state(nested)
    d = quant_state_as_dict(qs)
    keys = {"absmax", "quant_map", "quant_state.bitsandbytes__nf4"}
    if nested:
        keys |= {"nested_absmax", "nested_quant_map"}
    assert set(d) == keys
    meta = json.loads(bytes(d["quant_state.bitsandbytes__nf4"].tolist()).decode("utf-8"))
    assert meta["quant_type"] == "nf4" and meta["blocksize"] == 64 and meta["shape"] == [32, 48]
    assert meta["dtype"] == "bfloat16"
    if nested:
        assert meta["nested_blocksize"] == 256 and meta["nested_offset"] == 0.125 and meta["nested_dtype"] == "float32"
    back = quant_state_from_dict(d, "cpu")
    assert back.nested == nested and tuple(back.shape) == (32, 48) and back.blocksize == 64
    assert torch.equal(back.absmax, qs.absmax) and torch.equal(back.code, qs.code)
    assert back.dtype == torch.bfloat16 and back.nibble_order == 1
    if nested:
        assert torch.equal(back.state2.absmax, qs.state2.absmax) and torch.equal(back.state2.code, qs.state2.code)
        assert float(back.offset) == 0.125 and back.state2.blocksize == 256


def test_quant_state_dict_refusals():
    qs = _state(False)
    qs.nibble_order = 0
    with pytest.raises(CapabilityError, match="high nibble"):
        quant_state_as_dict(qs)
    with pytest.raises(CapabilityError, match="missing"):
        quant_state_from_dict({"absmax": torch.zeros(1)})
    d = quant_state_as_dict(_state(False))
    d["quant_state.bitsandbytes__nf4"] = torch.tensor(list(json.dumps({"quant_type": "fp4"}).encode()),
                                                      dtype=torch.uint8)
    with pytest.raises(CapabilityError, match="fp4"):
        quant_state_from_dict(d)
