"""Block statistics and adapters handed to the ops in a form that needs a
converted copy (non-contiguous fp32 views, bf16 values) must give bitwise the
same result as the same values passed contiguous in fp32. The copies are made
inside the op: each must stay alive until its launch is enqueued, or a later
allocation of the same call (a workspace, the fp32 copy of LoRA B) can take
its memory and overwrite the statistics before the GEMM reads them."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests._util import seeded, uniform

import molt_amd
from molt_amd import ops
from molt_amd._lib import tuning

pytestmark = pytest.mark.gpu


def _strided(t: torch.Tensor) -> torch.Tensor:
    """The same fp32 values as a non-contiguous view (every other element)."""
    wide = torch.zeros((t.numel(), 2), device=t.device, dtype=torch.float32)
    wide[:, 0] = t.reshape(-1).float()
    return wide[:, 0].reshape(t.shape)


@pytest.mark.parametrize("m,n,k,stage", [(4173, 512, 1024, 1), (300, 512, 1024, 0), (256, 256, 14336, 0)])
def test_forward_with_converted_scales_and_adapter(m, n, k, stage):
    print(f"nf4_lora_forward m={m} n={n} k={k} stage={stage} with strided statistics", flush=True)
    r = 16
    w = seeded((n, k), 701, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    scales = molt_amd.resolved_nf4_scales(qs)
    x = seeded((m, k), 702)
    a = uniform((r, k), 703, 1 / np.sqrt(k))
    b = seeded((n, r), 704, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    with tuning(big_tile_min=1, stage_min_mtiles=stage):
        plain = ops.nf4_lora_forward(x, packed.reshape(-1), scales, qs.code, n, k, 1, 64, t, b, 2.0)
        conv = ops.nf4_lora_forward(x, packed.reshape(-1), _strided(scales), _strided(qs.code), n, k, 1, 64, t,
                                    _strided(b), 2.0)
    torch.cuda.synchronize()
    assert torch.equal(plain, conv)


def test_input_gradient_with_converted_scales_and_adapter():
    m, n, k, r = 4173, 512, 1024, 16
    print(f"nf4_lora_backward_input m={m} n={n} k={k} with strided statistics", flush=True)
    w = seeded((n, k), 711, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    scales = molt_amd.resolved_nf4_scales(qs)
    dy = seeded((m, n), 712)
    a = uniform((r, k), 713, 1 / np.sqrt(k))
    u = seeded((m, r), 714)
    with tuning(big_tile_min=1, stage_min_mtiles=1):
        plain = ops.nf4_lora_backward_input(dy, packed.reshape(-1), scales, qs.code, n, k, 1, 64, u, a, 1.0)
        conv = ops.nf4_lora_backward_input(dy, packed.reshape(-1), _strided(scales), _strided(qs.code), n, k, 1,
                                           64, u, _strided(a), 1.0)
    torch.cuda.synchronize()
    assert torch.equal(plain, conv)


@pytest.mark.parametrize("m", [1, 4, 16])
def test_gemv_with_converted_nested_statistics(m):
    n, k, r = 1024, 14336, 16
    print(f"nf4_gemv M={m} N={n} K={k} with strided nested statistics", flush=True)
    w = seeded((n, k), 721, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    s2 = qs.state2
    x = seeded((m, k), 722)
    a = uniform((r, k), 723, 1 / np.sqrt(k))
    b = seeded((n, r), 724, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    plain = ops.nf4_gemv(x, packed.reshape(-1), None, qs.absmax, s2.absmax, s2.code, float(qs.offset),
                         int(s2.blocksize), qs.code, n, k, 1, t, b, 2.0)
    conv = ops.nf4_gemv(x, packed.reshape(-1), None, qs.absmax, _strided(s2.absmax), _strided(s2.code),
                        float(qs.offset), int(s2.blocksize), _strided(qs.code), n, k, 1, t, _strided(b), 2.0)
    torch.cuda.synchronize()
    assert torch.equal(plain, conv)


def test_gemm_timing_events_are_consumed_by_a_failing_call():
    """``molt_amd_time_next_gemm`` arms events for the next GEMM entry point of
    the calling thread. A call that fails (null weight) or returns early (no
    token rows) must consume them, so they are not recorded around the next,
    unrelated GEMM."""
    import ctypes as C

    from molt_amd import _lib

    lib = _lib.load()
    n = k = 4096
    m = 8192
    w = seeded((n, k), 731, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    scales = molt_amd.resolved_nf4_scales(qs)
    x = seeded((m, k), 732)
    stream = torch.cuda.current_stream().cuda_stream
    for case in ("null weight", "no rows"):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        end.record()
        torch.cuda.synchronize()
        assert lib.molt_amd_time_next_gemm(C.c_void_p(start.cuda_event), C.c_void_p(end.cuda_event)) == 0
        if case == "null weight":
            rc = lib.molt_nf4_lora_forward(x.data_ptr(), k, m, None, None, 1, None, 0, 1.0, None, n, None, 0,
                                           C.c_void_p(stream))
            assert rc != 0
        else:
            ops.nf4_lora_forward(x[:0], packed.reshape(-1), scales, qs.code, n, k, 1, 64, None, None, 1.0)
        y = ops.nf4_lora_forward(x, packed.reshape(-1), scales, qs.code, n, k, 1, 64, None, None, 1.0)
        torch.cuda.synchronize()
        span = start.elapsed_time(end)
        print(f"{case}: armed events span {span * 1e3:.1f} us after a {m}x{n}x{k} GEMM", flush=True)
        assert span < 0.05, f"{case}: the events were recorded around a later GEMM ({span:.3f} ms)"
        del y
