"""The hot path under HIP graph capture: a scheduled NF4-LoRA projection, the
frozen RMSNorm and the fused gated MLP with the RMSNorm-replay recipe,
forward + backward, captured once and replayed several times with eager work
and synchronisations between the replays. Every replay must equal the eager
step bit for bit (the library records no memset into a graph; its split-K
partials and workspaces come from the stream's allocations)."""
from __future__ import annotations

import pytest
import torch
from torch import nn

from tests._util import seeded

from molt_amd.kernels import FrozenRMSNormBF16
from molt_amd.methods import enable_fused_gated_nf4_lora, enable_rmsnorm_replay, enable_scheduled_nf4_lora
from molt_amd.modules import GatedMLP, synthetic_nf4_lora

pytestmark = pytest.mark.gpu


class _Norm(nn.Module):
    def __init__(self, weight: torch.Tensor) -> None:
        super().__init__()
        self.weight = nn.Parameter(weight, requires_grad=False)
        self.variance_epsilon = 1e-6


class _Block(nn.Module):
    """x + proj(x), then residual + mlp(post_attention_layernorm(residual))."""

    def __init__(self, hidden: int, inter: int, r: int, gen: torch.Generator) -> None:
        super().__init__()
        dev = torch.device("cuda")
        self.proj = synthetic_nf4_lora(hidden, hidden, r, 2.0 * r, device=dev, generator=gen)
        self.post_attention_layernorm = FrozenRMSNormBF16(
            _Norm(torch.randn(hidden, generator=gen, device=dev) * 0.2 + 1.0), weight_offset=0.0)
        self.mlp = GatedMLP(synthetic_nf4_lora(inter, hidden, r, 2.0 * r, device=dev, generator=gen),
                            synthetic_nf4_lora(inter, hidden, r, 2.0 * r, device=dev, generator=gen),
                            synthetic_nf4_lora(hidden, inter, r, 2.0 * r, device=dev, generator=gen))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        residual = x + self.proj(x)
        return residual + self.mlp(self.post_attention_layernorm(residual))


@pytest.mark.parametrize("hidden,inter,r,m", [(256, 512, 16, 256), (1536, 8960, 16, 4096)])
def test_graph_replays_equal_the_eager_step(hidden, inter, r, m):
    print(f"graph capture H={hidden} I={inter} r={r} M={m}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(11)
    model = nn.Sequential(_Block(hidden, inter, r, gen), _Block(hidden, inter, r, gen))
    assert enable_scheduled_nf4_lora(model, module_suffixes=(".proj",)) == 2
    assert enable_fused_gated_nf4_lora(model) == 2
    assert enable_rmsnorm_replay(model) == 2
    x = seeded((m, hidden), 12).requires_grad_()
    dy = seeded((m, hidden), 13)
    params = [p for p in model.parameters() if p.requires_grad]

    def clear():
        x.grad = None
        for p in params:
            p.grad = None

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = model(x)
        y.backward(dy)
        return y.detach()

    # warm up and take the eager reference on a side stream, keeping no autograd graph alive
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            clear()
            step()
        clear()
        ref_y = step().clone()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    ref = [x.grad.clone()] + [p.grad.clone() for p in params]

    clear()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = step()
    outs = [x.grad] + [p.grad for p in params]
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref_y), f"replay {rep}: output differs from the eager step"
        for i, (a, b) in enumerate(zip(outs, ref)):
            assert torch.equal(a, b), f"replay {rep}: gradient {i} differs from the eager step"
        # eager work between the replays, on the default stream
        noise = seeded((m, hidden), 100 + rep) * 2.0
        torch.cuda.synchronize()
        del noise
