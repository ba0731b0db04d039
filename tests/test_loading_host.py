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


def _tiny_qwen2(seed: int = 0):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=50, tie_word_embeddings=False)
    torch.manual_seed(seed)
    model = Qwen2ForCausalLM(cfg)
    g = torch.Generator().manual_seed(seed + 100)
    for name, mod in model.named_modules():     # HF initialises biases to zero: make them distinctive
        if isinstance(mod, torch.nn.Linear) and mod.bias is not None:
            mod.bias.data.copy_(torch.randn(mod.bias.shape, generator=g))
    return model


def _packed_state(model, nested: bool = True) -> dict:
    """A bitsandbytes-layout state dict for every linear of ``model`` built on
    the host (random packed bytes and statistics; no quantiser run), with the
    linears' biases under ``<prefix>.bias``."""
    g = torch.Generator().manual_seed(9)
    state = {}
    for _, _, lin, name in _targets(model, "all-linear"):
        n, k = lin.out_features, lin.in_features
        blocks = n * k // 64
        state[f"{name}.weight"] = torch.randint(0, 256, (n * k // 2, 1), generator=g, dtype=torch.uint8)
        s2 = QuantState(torch.rand(-(-blocks // 256), generator=g), (1,), torch.linspace(-1, 1, 256), 256,
                        "dynamic", torch.float32)
        qs = QuantState(torch.randint(0, 256, (blocks,), generator=g, dtype=torch.uint8), (n, k),
                        torch.linspace(-1, 1, 16), 64, "nf4", torch.bfloat16, torch.tensor(0.01), s2)
        for field, value in quant_state_as_dict(qs).items():
            state[f"{name}.weight.{field}"] = value
        if lin.bias is not None:
            state[f"{name}.bias"] = (lin.bias.detach() * 3 + 1).to(torch.bfloat16)
    return state


def test_load_prequantized_carries_the_checkpoint_biases():
    """Qwen2's q/k/v projections carry biases: the loaded NF4 bases hold the
    checkpoint's biases bit for bit (in the module's dtype), and the
    projections without one stay bias-free."""
    from molt_amd.loading import load_prequantized_nf4
    from molt_amd.modules import NF4Linear

    src = _tiny_qwen2(1)
    state = _packed_state(src)
    dst = _tiny_qwen2(2).to(torch.bfloat16)
    assert load_prequantized_nf4(dst, state, device="cpu") == 14
    biased = 0
    for name, mod in dst.named_modules():
        if not isinstance(mod, NF4Linear):
            continue
        if f"{name}.bias" in state:
            biased += 1
            assert mod.bias is not None and not mod.bias.requires_grad
            assert torch.equal(mod.bias.data.view(torch.int16), state[f"{name}.bias"].view(torch.int16)), name
        else:
            assert mod.bias is None, name
    assert biased == 6      # q, k, v of both layers
    # the rest of the checkpoint loads without unexpected keys
    rest = {k: v for k, v in state.items() if ".weight." not in k and not k.endswith("proj.weight")}
    _, unexpected = dst.load_state_dict(rest, strict=False)
    assert not unexpected, unexpected


def test_load_prequantized_refuses_a_bias_for_a_bias_free_module():
    from molt_amd.loading import load_prequantized_nf4

    model = _tiny_llama()
    state = _packed_state(model)
    state["model.layers.0.mlp.down_proj.bias"] = torch.zeros(64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="bias-free"):
        load_prequantized_nf4(model, state, device="cpu")


def test_bias_rule_routes_biased_bases():
    """A biased NF4 base may run the scheduled projection (which adds the bias)
    but not the gated-MLP nodes (which have no bias term)."""
    from molt_amd.loading import load_prequantized_nf4
    from molt_amd.modules import NF4LoRALinear
    from molt_amd.patching import lora_operands

    model = _tiny_qwen2(3)
    load_prequantized_nf4(model, _packed_state(model), device="cpu")
    q = NF4LoRALinear(model.model.layers[0].self_attn.q_proj, 4, 8.0)
    o = NF4LoRALinear(model.model.layers[0].self_attn.o_proj, 4, 8.0)
    assert lora_operands(q) == "the NF4 base projection has a bias"
    ops = lora_operands(q, allow_bias=True)
    assert not isinstance(ops, str) and ops.bias is q.base_layer.bias
    plain = lora_operands(o)
    assert not isinstance(plain, str) and plain.bias is None
