"""dense_nf4_layer_cache on the GPU: inside the context each NF4 base
projection of the layer is ``F.linear`` over the bit-exact bf16 decode of its
weight (bitwise), the LoRA branch is untouched, and the NF4 forward comes back
afterwards (methods/nf4_layer_cache.py:22-66)."""
from __future__ import annotations

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from tests._util import np_bits, oracle_weight, seeded

import molt_amd
from molt_amd.methods import dense_nf4_layer_cache
from molt_amd.modules import GatedMLP, synthetic_nf4_lora

pytestmark = pytest.mark.gpu


def test_cached_layer_forward_is_bitwise_the_dense_decode():
    g = torch.Generator(device="cuda").manual_seed(5)
    mlp = GatedMLP(synthetic_nf4_lora(512, 256, 8, 16.0, device="cuda", generator=g),
                   synthetic_nf4_lora(512, 256, 8, 16.0, device="cuda", generator=g),
                   synthetic_nf4_lora(256, 512, 8, 16.0, device="cuda", generator=g))
    x = seeded((2, 24, 256), 6)
    bases = [mlp.gate_proj.base_layer, mlp.up_proj.base_layer, mlp.down_proj.base_layer]
    originals = [b.forward for b in bases]
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):   # the PEFT dataflow runs under autocast
        before = mlp(x)
        with dense_nf4_layer_cache(mlp) as n:
            assert n == 3
            for b in bases:
                dense = molt_amd.dequantize_4bit(b.weight, b.weight.quant_state).to(torch.bfloat16)
                ow = oracle_weight(b.weight, b.weight.quant_state)
                assert np.array_equal(np_bits(dense), ow.dequant_bf16_bits())
                z = seeded((3, 7, b.in_features), 7)
                assert torch.equal(b(z), F.linear(z, dense))
            inside = mlp(x)
        after = mlp(x)
    assert [b.forward for b in bases] == originals
    assert torch.equal(before, after)
    torch.testing.assert_close(inside.float(), before.float(), rtol=2e-2, atol=2e-2)
