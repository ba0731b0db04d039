"""Projections that share one input as one stacked NF4-LoRA node
(molt_lora_stack_adapters, molt_nf4_stacked_forward,
molt_nf4_stacked_backward_input; methods.stacked_lora).

Every output column and every gradient of the stacked node is checked against
the fp64 oracle of that projection's own linear (oracle.lora_linear_forward /
lora_linear_backward over the same bf16 operands) and against the separate
scheduled nodes (same rounding points, fp32 sums in another order). Shapes: a
small stack with the staged plan forced, the Qwen2.5-1.5B q/k/v shapes at
cfg3's 4096 tokens with the library's own plan, and a patched decoder layer
whose attention runs its q/k/v through one node."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as O
from tests._util import assert_close_fro, bf16_values, np_f32, oracle_weight, seeded, uniform

import molt_amd
from molt_amd import ops
from molt_amd._lib import tuning
from molt_amd.errors import CapabilityError
from molt_amd.kernels import enable_frozen_rmsnorm_bf16
from molt_amd.methods import enable_scheduled_nf4_lora, enable_stacked_nf4_lora, scheduled_nf4_lora
from molt_amd.methods.stacked_lora import stacked_nf4_lora

pytestmark = pytest.mark.gpu


def _projections(rows, k, r, seed):
    out = []
    for i, n in enumerate(rows):
        w = seeded((n, k), seed + 10 * i, std=0.02, dtype=torch.float32)
        packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
        a = uniform((r, k), seed + 10 * i + 1, 1 / np.sqrt(k)).requires_grad_()
        b = seeded((n, r), seed + 10 * i + 2, std=0.02, dtype=torch.float32).requires_grad_()
        out.append((packed, qs, a, b))
    return out


def _check(rows, k, r, m, s, seed):
    projs = _projections(rows, k, r, seed)
    x = seeded((m, k), seed + 100).requires_grad_()
    dys = [seeded((m, n), seed + 200 + i) for i, n in enumerate(rows)]
    outs = stacked_nf4_lora(x, [p[0] for p in projs], [p[2] for p in projs], [p[3] for p in projs],
                            [p[1] for p in projs], s)
    assert "StackedNF4LoRA" in type(outs[0].grad_fn).__name__
    torch.autograd.backward(outs, dys)
    got = [o.detach().clone() for o in outs]
    dx = x.grad.clone()
    dab = [(p[2].grad.clone(), p[3].grad.clone()) for p in projs]

    # the separate scheduled nodes over the same operands
    x.grad = None
    for p in projs:
        p[2].grad = p[3].grad = None
    sep = [scheduled_nf4_lora(x, p[0], p[2], p[3], p[1], s) for p in projs]
    torch.autograd.backward(sep, dys)
    torch.cuda.synchronize()
    rdx = np.zeros((m, k))
    xs = bf16_values(x)
    for i, (p, dy) in enumerate(zip(projs, dys)):
        w = oracle_weight(p[0], p[1]).dequant_bf16().astype(np.float64)
        a, b = bf16_values(p[2]), bf16_values(p[3])
        ry = O.lora_linear_forward(xs, w, a, b, s)
        pdx, rda, rdb = O.lora_linear_backward(xs, w, a, b, s, bf16_values(dy))
        rdx += pdx
        assert_close_fro(np_f32(got[i]), ry, what=f"Y[{i}]")
        assert_close_fro(np_f32(dab[i][0]), rda, what=f"dA[{i}]")
        assert_close_fro(np_f32(dab[i][1]), rdb, what=f"dB[{i}]")
        assert_close_fro(np_f32(got[i]), np_f32(sep[i]).astype(np.float64), tol=2e-3, what=f"Y[{i}] vs node")
        assert_close_fro(np_f32(dab[i][0]), np_f32(p[2].grad).astype(np.float64), tol=1e-4,
                         what=f"dA[{i}] vs node")
        assert_close_fro(np_f32(dab[i][1]), np_f32(p[3].grad).astype(np.float64), tol=1e-4,
                         what=f"dB[{i}] vs node")
    assert_close_fro(np_f32(dx), rdx, what="dX")
    assert_close_fro(np_f32(dx), np_f32(x.grad).astype(np.float64), tol=4e-3, what="dX vs nodes")


def test_stacked_node_small_forced_staging():
    print("stacked q/k/v 768+256+256 x 1024, M=1024, r=16 (staged plan forced)", flush=True)
    with tuning(big_tile_min=1, stage_min_mtiles=1):
        assert ops._keeps_wt(1024, 1280, 1024, 1)
        _check([768, 256, 256], 1024, 16, 1024, 2.0, 900)


def test_stacked_node_qwen_attention_shapes():
    """Qwen2.5-1.5B q/k/v (1536 and 2 x 256 outputs of 1536) at 4096 tokens,
    the library's own plan."""
    print("stacked q/k/v 1536+256+256 x 1536, M=4096, r=16", flush=True)
    assert ops._keeps_wt(4096, 2048, 1536, 1)
    _check([1536, 256, 256], 1536, 16, 4096, 2.0, 950)


def test_stacked_node_two_weights_rank_32():
    print("stacked 512+512 x 512, M=2048, r=32 (staged plan forced)", flush=True)
    with tuning(big_tile_min=1, stage_min_mtiles=1):
        _check([512, 512], 512, 32, 2048, 0.5, 970)


def test_stacked_forward_refuses_unstaged_batches():
    projs = _projections([256, 256], 512, 16, 990)
    x = seeded((64, 512), 991)
    assert not ops._keeps_wt(64, 512, 512, 1)
    with pytest.raises(CapabilityError):
        stacked_nf4_lora(x, [p[0] for p in projs], [p[2] for p in projs], [p[3] for p in projs],
                         [p[1] for p in projs], 2.0)


def _llama(seed=0):
    from transformers import LlamaConfig, LlamaModel

    from molt_amd.loading import prepare_nf4_qlora

    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=64, rms_norm_eps=1e-6, attention_bias=False,
                      mlp_bias=False)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(seed)
    with torch.device("cuda"):
        model = LlamaModel(cfg)
    prepare_nf4_qlora(model, 16, 32.0)
    enable_frozen_rmsnorm_bf16(model)       # bf16 norm outputs: the projections' inputs
    # LoRA B starts at zero; give it values so that the adapters contribute
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "lora_B" in name:
                p.normal_(0.0, 0.02)
    return model


def test_patched_decoder_stack_runs_qkv_as_one_node():
    base, stacked = _llama(3), _llama(3)
    assert enable_scheduled_nf4_lora(base, module_suffixes=("q_proj", "k_proj", "v_proj", "o_proj")) == 8
    assert enable_scheduled_nf4_lora(stacked, module_suffixes=("q_proj", "k_proj", "v_proj", "o_proj")) == 8
    assert enable_stacked_nf4_lora(stacked) == 2
    x = seeded((2, 256, 256), 31)
    dy = seeded((2, 256, 256), 32)
    results = []
    with tuning(big_tile_min=1, stage_min_mtiles=1):
        for model in (base, stacked):
            xi = x.clone().requires_grad_()
            seen = []
            hook = model.layers[0].self_attn.k_proj.register_forward_hook(
                lambda mod, inp, out: seen.append(type(out.grad_fn).__name__))
            with torch.autocast("cuda", dtype=torch.bfloat16):
                out = model(inputs_embeds=xi).last_hidden_state
            hook.remove()
            out.backward(dy)
            grads = {n: p.grad.clone() for n, p in model.named_parameters() if p.grad is not None}
            results.append((out.detach().float(), xi.grad.float(), grads, seen))
    torch.cuda.synchronize()
    (o0, g0, p0, s0), (o1, g1, p1, s1) = results
    assert "ScheduledNF4LoRA" in s0[0] and "StackedNF4LoRA" in s1[0]
    assert_close_fro(np_f32(o1), np_f32(o0).astype(np.float64), tol=5e-3, what="stack output")
    assert_close_fro(np_f32(g1), np_f32(g0).astype(np.float64), tol=5e-3, what="stack dX")
    assert p0.keys() == p1.keys() and any("q_proj" in n for n in p1)
    for name in p0:
        assert_close_fro(np_f32(p1[name]), np_f32(p0[name]).astype(np.float64), tol=2e-2, what=name)



def test_siblings_called_before_the_first_projection_run_their_own_node():
    """A parent whose forward calls k_proj before q_proj, twice on the same
    input tensor, with k's adapter changed between the calls: k must never
    get an output the stacked node left in an earlier call (the parent's
    pre-hook clears them), and every output matches that projection's own
    node."""
    from torch import nn

    attn = _llama(5).layers[0].self_attn

    class KFirst(nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj, self.k_proj, self.v_proj = attn.q_proj, attn.k_proj, attn.v_proj

        def forward(self, x):
            return self.k_proj(x), self.q_proj(x), self.v_proj(x)

    parent = KFirst()
    assert enable_scheduled_nf4_lora(parent) == 3
    assert enable_stacked_nf4_lora(parent) == 1
    x = seeded((2, 256, 256), 41)
    with tuning(big_tile_min=1, stage_min_mtiles=1), torch.autocast("cuda", dtype=torch.bfloat16):
        for i in range(3):
            with torch.no_grad():
                parent.k_proj.lora_B["default"].weight.add_(0.05)
            k, q, v = parent(x)
            for mod, out in ((parent.k_proj, k), (parent.q_proj, q), (parent.v_proj, v)):
                ref = mod._molt_unstacked_forward(x)
                assert_close_fro(np_f32(out), np_f32(ref).astype(np.float64), tol=2e-3,
                                 what=f"call {i} {type(mod).__name__}")
    torch.cuda.synchronize()
