"""The HIP path against the committed golden fixtures (tests/golden/*.npz):
the GPU quantiser, double quantisation, scale resolution and dequantisation
must reproduce the stored bytes and bf16 bit patterns exactly; the NF4-LoRA
linear and the gated MLP, fed the stored packed weights and activations, must
match the stored fp64-derived results to relative Frobenius 5e-3."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from tests._util import assert_close_fro, np_bits, np_f32

import molt_amd
from molt_amd.methods import asymmetric_gated_nf4_lora, fused_gated_nf4_lora_mlp, scheduled_nf4_lora
from molt_amd.nf4 import NF4_CODEBOOK, QuantState

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
CODEC_CASES = ["bnb_64x64", "clean_70x66", "bnb_32x1024", "clean_48x40_b16"]


def _load(fname):
    with np.load(GOLDEN / fname, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.uint16).view(np.int16)).view(torch.bfloat16).cuda()


def _state(g: dict, prefix: str, shape) -> tuple[torch.Tensor, QuantState]:
    dev = torch.device("cuda")
    code2 = torch.from_numpy(g[f"{prefix}/code2"]).to(dev)
    absmax2 = torch.from_numpy(g[f"{prefix}/absmax2"]).to(dev)
    state2 = QuantState(absmax2, (absmax2.numel(),), code2, 256, "dynamic", torch.float32)
    qs = QuantState(torch.from_numpy(g[f"{prefix}/q"]).to(dev), shape, NF4_CODEBOOK.to(dev), 64, "nf4",
                    torch.bfloat16, torch.tensor(float(g[f"{prefix}/offset"]), device=dev), state2, 1)
    n = int(np.prod(shape))
    packed = torch.from_numpy(g[f"{prefix}/packed"][: (n + 1) // 2].copy()).to(dev).reshape(-1, 1)
    return packed, qs


@pytest.mark.parametrize("name", CODEC_CASES)
def test_codec_reproduces_golden_bytes(name):
    print(f"golden codec {name}", flush=True)
    g = _load("nf4_codec.npz")
    w = torch.from_numpy(g[f"{name}/w"]).cuda()
    block, order = int(g[f"{name}/block"]), int(g[f"{name}/order"])
    nested = f"{name}/q" in g
    packed, qs = molt_amd.quantize_4bit(w, blocksize=block, compress_statistics=nested, nibble_order=order)
    n = w.numel()
    assert np.array_equal(packed.reshape(-1).cpu().numpy(), g[f"{name}/packed"][: (n + 1) // 2])
    if nested:
        assert np.array_equal(qs.absmax.cpu().numpy(), g[f"{name}/q"])
        assert np.array_equal(np_f32(qs.state2.absmax), g[f"{name}/absmax2"])
        assert np.array_equal(np_f32(qs.state2.code), g[f"{name}/code2"])
        assert np.float32(float(qs.offset)) == g[f"{name}/offset"]
    else:
        assert np.array_equal(np_f32(qs.absmax), g[f"{name}/absmax"])
    assert np.array_equal(np_f32(molt_amd.resolved_nf4_scales(qs)), g[f"{name}/scales"])
    deq = molt_amd.dequantize_4bit(packed, qs, torch.bfloat16)
    assert np.array_equal(np_bits(deq).reshape(-1), g[f"{name}/dequant_bf16_bits"].reshape(-1))


def test_linear_matches_golden():
    g = _load("nf4_lora_linear.npz")
    x = _bf16(g["linear/x_bf16_bits"])
    dy = _bf16(g["linear/dy_bf16_bits"])
    m, k = x.shape
    n = dy.shape[1]
    packed, qs = _state(g, "linear", (n, k))
    a = torch.from_numpy(g["linear/lora_a"]).cuda().requires_grad_()
    b = torch.from_numpy(g["linear/lora_b"]).cuda().requires_grad_()
    xr = x.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = scheduled_nf4_lora(xr, packed, a, b, qs, float(g["linear/scaling"]))
    y.backward(dy)
    assert_close_fro(np_f32(y), g["linear/y"], what="Y")
    assert_close_fro(np_f32(xr.grad), g["linear/dx"], what="dX")
    assert_close_fro(np_f32(a.grad), g["linear/da"], what="dA")
    assert_close_fro(np_f32(b.grad), g["linear/db"], what="dB")


def _mlp_inputs(g):
    x = _bf16(g["mlp/x_bf16_bits"])
    dy = _bf16(g["mlp/dy_bf16_bits"])
    h = x.shape[1]
    i = g["mlp/gate/lora_b"].shape[0]
    parts = []
    for name, shape in (("gate", (i, h)), ("up", (i, h)), ("down", (h, i))):
        packed, qs = _state(g, f"mlp/{name}", shape)
        a = torch.from_numpy(g[f"mlp/{name}/lora_a"]).cuda().requires_grad_()
        b = torch.from_numpy(g[f"mlp/{name}/lora_b"]).cuda().requires_grad_()
        parts.append((packed, qs, a, b))
    return x, dy, parts, float(g["mlp/scaling"])


def _check_mlp(g, y, dx, parts):
    assert_close_fro(np_f32(y).reshape(g["mlp/y"].shape), g["mlp/y"], what="Y")
    assert_close_fro(np_f32(dx).reshape(g["mlp/dx"].shape), g["mlp/dx"], what="dX")
    for (_, _, a, b), name in zip(parts, ("gate", "up", "down")):
        assert_close_fro(np_f32(a.grad), g[f"mlp/da_{name}"], what=f"dA_{name}")
        assert_close_fro(np_f32(b.grad), g[f"mlp/db_{name}"], what=f"dB_{name}")


def test_fused_gated_mlp_matches_golden():
    g = _load("gated_mlp.npz")
    x, dy, parts, s = _mlp_inputs(g)
    xr = x.clone().requires_grad_()
    (pg, qg, ag, bg), (pu, qu, au, bu), (pd, qd, ad, bd) = parts
    y = fused_gated_nf4_lora_mlp(xr, pg, ag, bg, pu, au, bu, pd, ad, bd, qg, qu, qd, s, s, s)
    y.backward(dy)
    _check_mlp(g, y, xr.grad, parts)


def test_asymmetric_gated_replay_matches_golden():
    g = _load("gated_mlp.npz")
    x, dy, parts, s = _mlp_inputs(g)
    xr = x.clone().requires_grad_()
    (pg, qg, ag, bg), (pu, qu, au, bu), (pd, qd, ad, bd) = parts
    with torch.autocast("cuda", dtype=torch.bfloat16):
        gate = scheduled_nf4_lora(xr, pg, ag, bg, qg, s)
        up = scheduled_nf4_lora(xr, pu, au, bu, qu, s)
        y = asymmetric_gated_nf4_lora(xr, gate, up, pu, au, bu, pd, ad, bd, qu, qd, s, s, True)
    y.backward(dy)
    _check_mlp(g, y, xr.grad, parts)
