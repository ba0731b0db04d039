"""The cfg3 workload: a 28-layer decoder stack shaped like Qwen2.5-1.5B
(hidden 1536, 12 query / 2 key-value heads of dim 128, intermediate 8960,
RMSNorm), NF4 QLoRA r = 16, alpha = 32 on all seven projections of every
layer, random-init weights N(0, 0.02), one forward + backward over bf16 token
embeddings N(0, 1) at batch 4 x seq 1024 with the gated MLP's RMSNorm replay
(the trainer loop of training/qlora.py:818-945 on the
configs/molt-qwen2.5-1.5b-endurance.json shapes).

The stack is built as a transformers Llama decoder with those shapes: Qwen2's
q/k/v biases are left out because NF4 QLoRA projections here are bias-free
(the reference's scheduled path falls back to PEFT for biased projections,
methods/nf4_lora.py:148-156). Attention itself is torch SDPA, outside this
path.

Checks: forward output bitwise equal across two runs; every patched module
whose incoming gradient is bitwise equal across the runs produces bitwise
equal LoRA gradients (SDPA's backward, upstream of most modules, is torch's
and may not repeat bitwise); every gradient finite; and one layer's seven
projections against the fp64 oracle (Y and dX on 64 sampled rows, dA and dB
over all 4096 rows) from the inputs and output gradients captured at those
modules."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as O
from tests._util import assert_close_fro, bf16_values, np_f32, oracle_weight, seeded

from molt_amd.kernels import enable_frozen_rmsnorm_bf16
from molt_amd.loading import prepare_nf4_qlora
from molt_amd.methods import enable_fused_gated_nf4_lora, enable_rmsnorm_replay, enable_scheduled_nf4_lora
from molt_amd.modules import NF4LoRALinear

pytestmark = pytest.mark.gpu

H, I, HEADS, KV, LAYERS, R, ALPHA = 1536, 8960, 12, 2, 28, 16, 32.0
BATCH, SEQ = 4, 1024
CHECK_LAYER = 13
ATTN = ("q_proj", "k_proj", "v_proj", "o_proj")


def _stack():
    from transformers import LlamaConfig, LlamaModel

    cfg = LlamaConfig(hidden_size=H, intermediate_size=I, num_hidden_layers=LAYERS, num_attention_heads=HEADS,
                      num_key_value_heads=KV, head_dim=128, vocab_size=256, rms_norm_eps=1e-6,
                      max_position_embeddings=SEQ, attention_bias=False, mlp_bias=False)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(1337)
    with torch.device("cuda"):
        model = LlamaModel(cfg)
    prepare_nf4_qlora(model, R, ALPHA)
    g = torch.Generator(device="cuda").manual_seed(7)
    for m in model.modules():
        if isinstance(m, NF4LoRALinear):   # B ~ N(0, 0.01) so that every LoRA gradient is exercised
            w = m.lora_B["default"].weight
            w.data.copy_(torch.randn(w.shape, generator=g, device="cuda") * 0.01)
    assert enable_frozen_rmsnorm_bf16(model) == 2 * LAYERS + 1
    assert enable_scheduled_nf4_lora(model, module_suffixes=ATTN) == 4 * LAYERS
    assert enable_fused_gated_nf4_lora(model) == LAYERS
    assert enable_rmsnorm_replay(model) == LAYERS
    return model


class _Capture:
    """Input and output (forward hook) and the gradient arriving at the output
    (a tensor hook on it) of selected modules. Hooks of this kind leave the
    tensors the modules see untouched, so the RMSNorm replay recipe (which
    matches its target by identity) stays in effect."""

    def __init__(self, modules: dict[str, torch.nn.Module], keep_forward: set[str]):
        self.fwd: dict[str, tuple[torch.Tensor, torch.Tensor]] = {}
        self.grad_out: dict[str, torch.Tensor] = {}
        self.handles = [mod.register_forward_hook(self._hook(name, name in keep_forward))
                        for name, mod in modules.items()]

    def _hook(self, name, keep):
        def store(grad):
            self.grad_out[name] = grad.detach().clone()

        def hook(_m, inputs, output):
            if keep:
                self.fwd[name] = (inputs[0].detach().clone(), output.detach().clone())
            output.register_hook(store)
        return hook

    def close(self):
        for h in self.handles:
            h.remove()


def _lora_params(model):
    return {n: p for n, p in model.named_parameters() if p.requires_grad}


def _step(model, x, dy, capture):
    for p in model.parameters():
        p.grad = None
    xr = x.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = model(inputs_embeds=xr).last_hidden_state
    out.backward(dy)
    torch.cuda.synchronize()
    grads = {n: p.grad.detach().clone() for n, p in _lora_params(model).items()}
    capture.close()
    return out.detach().clone(), xr.grad.detach().clone(), grads


def _proj_oracle(mod, x, dy, rows):
    """Y and dX rows (fp64 oracle) and full dA, dB (fp64 oracle algebra on all rows)."""
    w = oracle_weight(mod.base_layer.weight, mod.base_layer.weight.quant_state).dequant_bf16().astype(np.float64)
    a, b = bf16_values(mod.lora_A["default"].weight), bf16_values(mod.lora_B["default"].weight)
    s = float(mod.scaling["default"])
    xo, dyo = bf16_values(x).reshape(-1, w.shape[1]), bf16_values(dy).reshape(-1, w.shape[0])
    y = O.lora_linear_forward(xo[rows], w, a, b, s)
    dx, _, _ = O.lora_linear_backward(xo[rows], w, a, b, s, dyo[rows])
    _, da, db = O.lora_linear_backward(xo, w, a, b, s, dyo)
    return y, dx, da, db


def test_cfg3_decoder_stack_fwd_bwd():
    print("cfg3: building and quantising the 28-layer stack", flush=True)
    model = _stack()
    x = seeded((BATCH, SEQ, H), 31)
    dy = seeded((BATCH, SEQ, H), 32)
    layer = model.layers[CHECK_LAYER]
    watched = {f"{i}.{n}": getattr(model.layers[i].self_attn, n) for i in range(LAYERS) for n in ATTN}
    watched.update({f"{i}.mlp": model.layers[i].mlp for i in range(LAYERS)})
    keep = {f"{CHECK_LAYER}.{n}" for n in ATTN} | {f"{CHECK_LAYER}.mlp"}

    print("cfg3: run 1", flush=True)
    cap1 = _Capture(watched, keep)
    out1, dx1, grads1 = _step(model, x, dy, cap1)
    print("cfg3: run 2", flush=True)
    cap2 = _Capture(watched, set())
    out2, dx2, grads2 = _step(model, x, dy, cap2)

    assert out1.shape == (BATCH, SEQ, H) and torch.isfinite(out1).all()
    assert torch.equal(out1, out2), "forward output differs between runs"
    assert len(grads1) == 2 * 7 * LAYERS
    for n, g in grads1.items():
        assert torch.isfinite(g).all() and g.abs().sum() > 0, n
    same_input = 0
    for name in watched:
        if not torch.equal(cap1.grad_out[name], cap2.grad_out[name]):
            continue
        same_input += 1
        i, proj = name.split(".", 1)
        prefix = f"layers.{i}.self_attn.{proj}" if proj in ATTN else f"layers.{i}.mlp"
        for pn in grads1:
            if pn.startswith(prefix + "."):
                assert torch.equal(grads1[pn], grads2[pn]), f"{pn}: same incoming gradient, different result"
    print(f"cfg3: {same_input}/{len(watched)} modules saw bitwise-equal incoming gradients", flush=True)
    assert same_input >= 2   # the last layer's MLP and o_proj see no attention backward above them
    assert torch.isfinite(dx1).all()

    print(f"cfg3: layer {CHECK_LAYER} against the oracle", flush=True)
    rows = np.sort(np.random.default_rng(3).choice(BATCH * SEQ, 64, replace=False))
    for proj in ATTN:
        mod = getattr(layer.self_attn, proj)
        xin, yout = cap1.fwd[f"{CHECK_LAYER}.{proj}"]
        gout = cap1.grad_out[f"{CHECK_LAYER}.{proj}"]
        ry, rdx, rda, rdb = _proj_oracle(mod, xin, gout, rows)
        assert_close_fro(np_f32(yout).reshape(-1, ry.shape[1])[rows], ry, what=f"{proj} Y rows")
        pre = f"layers.{CHECK_LAYER}.self_attn.{proj}"
        assert_close_fro(np_f32(grads1[f"{pre}.lora_A.default.weight"]), rda, what=f"{proj} dA")
        assert_close_fro(np_f32(grads1[f"{pre}.lora_B.default.weight"]), rdb, what=f"{proj} dB")
        # the projection's own input gradient, recomputed through the same module
        xr = xin.clone().requires_grad_()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = mod(xr)
        y.backward(gout)
        assert torch.equal(y, yout)
        assert_close_fro(np_f32(xr.grad).reshape(-1, rdx.shape[1])[rows], rdx, what=f"{proj} dX rows")

    mlp = layer.mlp
    xin, yout = cap1.fwd[f"{CHECK_LAYER}.mlp"]
    gout = cap1.grad_out[f"{CHECK_LAYER}.mlp"]
    projs = [mlp.gate_proj, mlp.up_proj, mlp.down_proj]
    ws = [oracle_weight(p.base_layer.weight, p.base_layer.weight.quant_state).dequant_bf16().astype(np.float64)
          for p in projs]
    av = []
    for p in projs:
        av += [bf16_values(p.lora_A["default"].weight), bf16_values(p.lora_B["default"].weight)]
    s = ALPHA / R
    xo, dyo = bf16_values(xin).reshape(-1, H), bf16_values(gout).reshape(-1, H)
    ry, saved = O.gated_mlp_forward(xo, ws[0], ws[1], ws[2], *av, s)
    rdx, rgrads = O.gated_mlp_backward(xo, ws[0], ws[1], ws[2], *av, s, dyo, saved)
    assert_close_fro(np_f32(yout).reshape(-1, H), ry, what="MLP Y")
    names = ("gate_proj.lora_A", "gate_proj.lora_B", "up_proj.lora_A", "up_proj.lora_B", "down_proj.lora_A",
             "down_proj.lora_B")
    for n, ref in zip(names, rgrads):
        assert_close_fro(np_f32(grads1[f"layers.{CHECK_LAYER}.mlp.{n}.default.weight"]), ref, what=f"MLP d{n}")
    xr = xin.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = mlp(xr)
    y.backward(gout)
    assert torch.equal(y, yout)
    assert_close_fro(np_f32(xr.grad).reshape(-1, H), rdx, what="MLP dX")
