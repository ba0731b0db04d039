"""Host-side wiring of the RMSNorm-replay recipe (methods/gated_replay.py:13-47):
which norm output leaves a recipe on its MLP, and when it leaves None. No
kernel runs; the norm here is a stand-in that returns its input cast to the
requested dtype."""
from __future__ import annotations

import pytest
import torch

from molt_amd.errors import CapabilityError
from molt_amd.methods import gated_replay as G


class _Norm(torch.nn.Module):
    def __init__(self, dtype=torch.bfloat16):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(8), requires_grad=False)
        self.variance_epsilon = 1e-6
        self.weight_offset = 0.0
        self.dtype = dtype

    def forward(self, hidden):
        return hidden.to(self.dtype)


class _Layer(torch.nn.Module):
    def __init__(self, dtype=torch.bfloat16):
        super().__init__()
        self.post_attention_layernorm = _Norm(dtype)
        self.mlp = torch.nn.Identity()


def test_hook_leaves_recipe_for_bf16_output_under_grad():
    layer = _Layer()
    assert G.enable_rmsnorm_replay(layer) == 1
    x = torch.randn(3, 8)
    out = layer.post_attention_layernorm(x)
    recipe = layer.mlp._molt_norm_replay_recipe
    assert isinstance(recipe, G._RMSNormReplayRecipe)
    assert recipe.source is x and recipe.target is out
    assert recipe.eps == pytest.approx(1e-6) and recipe.weight_offset == 0.0


def test_hook_leaves_none_without_grad_or_for_other_dtypes():
    layer = _Layer()
    G.enable_rmsnorm_replay(layer)
    with torch.no_grad():
        layer.post_attention_layernorm(torch.randn(2, 8))
    assert layer.mlp._molt_norm_replay_recipe is None
    fp32 = _Layer(torch.float32)
    G.enable_rmsnorm_replay(fp32)
    fp32.post_attention_layernorm(torch.randn(2, 8))
    assert fp32.mlp._molt_norm_replay_recipe is None


def test_enable_is_idempotent_and_refuses_models_without_pairs():
    layer = _Layer()
    assert G.enable_rmsnorm_replay(layer) == 1
    with pytest.raises(CapabilityError):
        G.enable_rmsnorm_replay(layer)
    with pytest.raises(CapabilityError):
        G.enable_rmsnorm_replay(torch.nn.Linear(2, 2))


def test_hand_wired_replayable_norm_forward_matches_the_hook():
    norm, mlp = _Norm(), torch.nn.Identity()
    norm._molt_original_forward = norm.forward
    norm._molt_target_mlp = mlp
    x = torch.randn(4, 8)
    out = G._replayable_norm_forward(norm, x)
    assert torch.equal(out, x.to(torch.bfloat16))
    assert mlp._molt_norm_replay_recipe.source is x and mlp._molt_norm_replay_recipe.target is out
    with torch.no_grad():
        G._replayable_norm_forward(norm, x)
    assert mlp._molt_norm_replay_recipe is None
