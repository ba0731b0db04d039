"""Skinny-M NF4 GEMV (M <= 16) with the LoRA add-on vs the fp64 oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as O
from tests._util import assert_close_fro, bf16_values, np_f32, oracle_weight, seeded, uniform

import molt_amd
from molt_amd import ops

pytestmark = pytest.mark.gpu


def _gemv(x, packed, qs, t=None, b=None, s=0.0, nested=True):
    rows, cols = int(qs.shape[0]), int(qs.shape[1])
    if nested and qs.nested:
        s2 = qs.state2
        return ops.nf4_gemv(x, packed.reshape(-1), None, qs.absmax, s2.absmax, s2.code, float(qs.offset),
                            int(s2.blocksize), qs.code, rows, cols, qs.nibble_order, t, b, s)
    return ops.nf4_gemv(x, packed.reshape(-1), molt_amd.resolved_nf4_scales(qs), None, None, None, 0.0, 256,
                        qs.code, rows, cols, qs.nibble_order, t, b, s)


@pytest.mark.parametrize("n,k", [(64, 64), (256, 512), (1024, 4096), (96, 192), (4096, 4096)])
@pytest.mark.parametrize("m", [1, 2, 4, 8, 16])
def test_gemv_matches_oracle(n, k, m):
    print(f"gemv n={n} k={k} m={m}", flush=True)
    w = seeded((n, k), 50 + n, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    x = seeded((m, k), 60 + m)
    y = _gemv(x, packed, qs)
    wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    assert_close_fro(np_f32(y), bf16_values(x) @ wo.T, what="Y")


@pytest.mark.parametrize("m,n,r", [(1, 1024, 16), (1, 1000, 96), (1, 4100, 128), (5, 1024, 16), (16, 1024, 16),
                                   (3, 1000, 64),
                                   (16, 520, 96), (2, 256, 128),
                                   # ranks that are not a multiple of 4 (B read one float at a time),
                                   # one ending inside a lane group's 8
                                   (8, 1024, 5), (12, 3000, 70), (3, 4100, 30)])
def test_gemv_with_lora_matches_oracle(m, n, r):
    print(f"gemv lora m={m} n={n} r={r}", flush=True)
    k, s = 4096, 2.0
    w = seeded((n, k), 70, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    x = seeded((m, k), 71)
    a = uniform((r, k), 72, 1.0 / np.sqrt(k))
    b = seeded((n, r), 73, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    y = _gemv(x, packed, qs, t, b, s)
    wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    ref = O.lora_linear_forward(bf16_values(x), wo, bf16_values(a), bf16_values(b), s)
    assert_close_fro(np_f32(y), ref, what="Y")


@pytest.mark.parametrize("m,n,k,nested,order", [(1, 1000, 4096, True, 1), (1, 520, 4096, False, 0),
                                                 (1, 776, 14336, True, 1), (1, 264, 14336, False, 1),
                                                 (1, 4104, 14336, True, 0), (1, 2056, 4096, True, 1),
                                                 (1, 14344, 4096, True, 1), (3, 520, 4096, False, 0),
                                                 (2, 776, 14336, True, 1), (4, 2056, 4096, True, 1),
                                                 (2, 4104, 4096, False, 0), (3, 264, 14336, True, 0),
                                                 (4, 4100, 14336, False, 1), (4, 2048, 4096, True, 1),
                                                 # the MFMA kernel with resolved scales, one and four K slices
                                                 (8, 1000, 4096, False, 0), (16, 776, 14336, False, 1),
                                                 # one round per workgroup (4096 rows: 256 groups of 16)
                                                 (5, 4096, 4096, True, 1)])
def test_gemv_decode_shapes_match_oracle(m, n, k, nested, order):
    # K = 4096 / 14336 take the streaming dot-product decode kernel at M <= 2,
    # and at M = 3, 4 when K = 14336 or N <= 2048 (two or four X rows; M = 3
    # repeats the last row and stores three); ragged row counts exercise its
    # clamped loads and guarded stores. (4, 2056, 4096) covers the MFMA kernel.
    print(f"gemv decode m={m} n={n} k={k} nested={nested} order={order}", flush=True)
    w = seeded((n, k), 100 + n, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=nested, nibble_order=order)
    x = seeded((m, k), 101 + m)
    y = _gemv(x, packed, qs, nested=nested)
    wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    assert_close_fro(np_f32(y), bf16_values(x) @ wo.T, what="Y")


@pytest.mark.parametrize("m,n,k,r", [(2, 1000, 14336, 16), (3, 4100, 14336, 128), (4, 776, 14336, 96),
                                     (3, 1024, 4096, 64), (2, 4096, 4096, 16)])
def test_gemv_decode_tokens_with_lora_match_oracle(m, n, k, r):
    # Multi-token decode kernel with the LoRA add-on: every token row has its
    # own T row; r = 128 fills both halves of the lanes' rank slots.
    print(f"gemv decode lora m={m} n={n} k={k} r={r}", flush=True)
    s = 2.0
    w = seeded((n, k), 110 + m, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    x = seeded((m, k), 111 + r)
    a = uniform((r, k), 112, 1.0 / np.sqrt(k))
    b = seeded((n, r), 113, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    y = _gemv(x, packed, qs, t, b, s)
    wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    ref = O.lora_linear_forward(bf16_values(x), wo, bf16_values(a), bf16_values(b), s)
    assert_close_fro(np_f32(y), ref, what="Y")


@pytest.mark.parametrize("m,n", [(3, 1000), (16, 264)])
def test_gemv_nested_codes_at_odd_address(m, n):
    # u8 block codes 1 byte past a 4-byte boundary: the K = 4096 MFMA kernel's
    # per-block code loads (no 4-block code words) with LoRA rank chunks 0..2.
    print(f"gemv odd-address codes m={m} n={n}", flush=True)
    k, r, s = 4096, 80, 2.0
    w = seeded((n, k), 110 + n, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    buf = torch.zeros(qs.absmax.numel() + 16, device=qs.absmax.device, dtype=torch.uint8)
    codes = buf[1:1 + qs.absmax.numel()]
    codes.copy_(qs.absmax)
    assert codes.data_ptr() % 4 == 1
    x = seeded((m, k), 111 + m)
    a = uniform((r, k), 112, 1.0 / np.sqrt(k))
    b = seeded((n, r), 113, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    s2 = qs.state2
    y = ops.nf4_gemv(x, packed.reshape(-1), None, codes, s2.absmax, s2.code, float(qs.offset), int(s2.blocksize),
                     qs.code, n, k, qs.nibble_order, t, b, s)
    wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    ref = O.lora_linear_forward(bf16_values(x), wo, bf16_values(a), bf16_values(b), s)
    assert_close_fro(np_f32(y), ref, what="Y")


@pytest.mark.parametrize("m,n,r", [(16, 1000, 64), (2, 4100, 16), (7, 520, 128), (9, 1000, 70)])
def test_gemv_split_k_with_lora_matches_oracle(m, n, r):
    # K = 14336 with M >= 2: four K slices of fp32 partials summed by a second kernel.
    print(f"gemv split-K m={m} n={n} r={r}", flush=True)
    k, s = 14336, 2.0
    w = seeded((n, k), 120 + n, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    x = seeded((m, k), 121 + m)
    a = uniform((r, k), 122, 1.0 / np.sqrt(k))
    b = seeded((n, r), 123, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    y = _gemv(x, packed, qs, t, b, s)
    assert torch.equal(y, _gemv(x, packed, qs, t, b, s))
    wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    ref = O.lora_linear_forward(bf16_values(x), wo, bf16_values(a), bf16_values(b), s)
    assert_close_fro(np_f32(y), ref, what="Y")


def test_gemv_resolved_scales_and_low_nibble_layout():
    w = seeded((512, 1024), 80, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=False, nibble_order=0)
    x = seeded((3, 1024), 81)
    y = _gemv(x, packed, qs, nested=False)
    wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    assert_close_fro(np_f32(y), bf16_values(x) @ wo.T, what="Y")


def test_gemv_repeat_is_deterministic_and_workspace_reusable():
    w = seeded((14336, 4096), 90, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    del w
    x = seeded((16, 4096), 91)
    first = _gemv(x, packed, qs)
    for _ in range(3):
        assert torch.equal(_gemv(x, packed, qs), first)
    xs = seeded((2, 4096), 92)
    wo = oracle_weight(packed, qs).dequant_bf16()
    ref = bf16_values(xs) @ wo.astype(np.float64).T
    assert_close_fro(np_f32(_gemv(xs, packed, qs)), ref, what="Y")
    # property at full size: the GEMV row equals the GEMM row for the same token
    ref16 = bf16_values(x) @ wo.astype(np.float64).T
    assert_close_fro(np_f32(first), ref16, what="Y16")


def test_gemv_rejects_unsupported_geometry():
    w = seeded((64, 96), 1, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=False)
    with pytest.raises(molt_amd.CapabilityError, match="cols"):
        _gemv(seeded((2, 96), 2), packed, qs, nested=False)
    w2 = seeded((64, 128), 1, std=0.02, dtype=torch.float32)
    packed2, qs2 = molt_amd.quantize_4bit(w2, blocksize=64, compress_statistics=False)
    with pytest.raises(ValueError, match="1..16"):
        _gemv(seeded((17, 128), 2), packed2, qs2, nested=False)


def test_gemv_rejects_rank_above_128():
    w = seeded((64, 128), 3, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    x = seeded((2, 128), 4)
    t = seeded((2, 160), 5)
    b = seeded((64, 160), 6, std=0.01, dtype=torch.float32)
    with pytest.raises(molt_amd.CapabilityError, match="rank"):
        _gemv(x, packed, qs, t, b, 1.0)


@pytest.mark.parametrize("m", [1, 2, 4])
def test_patched_module_decode_runs_the_gemv(m):
    """A decode-sized batch through a patched NF4-LoRA module (the generate
    path of training/qlora.py:1332-1358, no gradient) runs the GEMV entry
    point and matches the oracle; the same batch carrying a gradient takes the
    dequantised-weight GEMM, as bnb.matmul_4bit does for a training forward,
    and its backward runs the NF4 dX GEMM."""
    from molt_amd.methods import enable_scheduled_nf4_lora
    from molt_amd.modules import synthetic_nf4_lora

    g = torch.Generator(device="cuda").manual_seed(90 + m)
    mod = synthetic_nf4_lora(1024, 4096, 16, 32.0, device="cuda", generator=g)
    model = torch.nn.Sequential(mod)
    assert enable_scheduled_nf4_lora(model) == 1
    x = seeded((1, m, 4096), 91 + m)
    qs = mod.base_layer.weight.quant_state
    wo = oracle_weight(mod.base_layer.weight, qs).dequant_bf16().astype(np.float64)
    a, b = mod.lora_A["default"].weight, mod.lora_B["default"].weight
    ref = O.lora_linear_forward(bf16_values(x).reshape(m, -1), wo, bf16_values(a), bf16_values(b), 2.0)
    for grad in (False, True):
        xin = x.detach().clone().requires_grad_(grad)
        calls = ops.probe_events("molt_nf4_gemv")
        gemm = ops.probe_events("molt_nf4_lora_forward")
        try:
            with torch.set_grad_enabled(grad), torch.autocast("cuda", dtype=torch.bfloat16):
                y = model(xin)
            n_gemv, n_gemm = len(calls), len(gemm)
        finally:
            ops.probe_events("molt_nf4_gemv", False)
            ops.probe_events("molt_nf4_lora_forward", False)
        assert (n_gemv, n_gemm) == ((0, 1) if grad else (1, 0)), (grad, n_gemv, n_gemm)
        assert_close_fro(np_f32(y).reshape(m, -1), ref, what=f"patched decode M={m} grad={grad}")
    dy = seeded((1, m, 1024), 92 + m)
    y.backward(dy)
    rdx, _, _ = O.lora_linear_backward(bf16_values(x).reshape(m, -1), wo, bf16_values(a), bf16_values(b), 2.0,
                                       bf16_values(dy).reshape(m, -1))
    assert_close_fro(np_f32(xin.grad).reshape(m, -1), rdx, what=f"patched decode dX M={m}")
    # the plain NF4 base projection under no_grad takes the GEMV as well
    calls = ops.probe_events("molt_nf4_gemv")
    try:
        with torch.no_grad():
            base = mod.base_layer(x)
        assert len(calls) == 1
    finally:
        ops.probe_events("molt_nf4_gemv", False)
    assert_close_fro(np_f32(base).reshape(m, -1), bf16_values(x).reshape(m, -1) @ wo.T, what="base decode")


@pytest.mark.parametrize("n,k", [(1536, 1536), (256, 1536), (8960, 1536), (1536, 8960), (4864, 896), (896, 4864),
                                 (520, 2112), (300, 8192), (130, 6144), (70, 10240)])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8])
def test_gemv_any_k_matches_oracle_and_repeats(n, k, m):
    """K outside {4096, 14336}: the Qwen2.5-1.5B decode shapes of the reference's
    generate_qlora (training/qlora.py:1332-1358) and pieces that end inside a
    row (2112, 896), an instantiated piece count above the row's (8192 -> 5
    pieces, 10240 -> 5), with the r = 16 LoRA add-on and both nibble orders:
    against the fp64 oracle, and two calls bitwise equal."""
    print(f"gemv any-k n={n} k={k} m={m}", flush=True)
    r, s, order = 16, 2.0, (n + m) % 2
    w = seeded((n, k), 900 + n + k, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True, nibble_order=order)
    x = seeded((m, k), 901 + m)
    a = uniform((r, k), 902, 1.0 / np.sqrt(k))
    b = seeded((n, r), 903, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    y1, y2 = _gemv(x, packed, qs, t, b, s), _gemv(x, packed, qs, t, b, s)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    ref = O.lora_linear_forward(bf16_values(x), wo, bf16_values(a), bf16_values(b), s)
    assert_close_fro(np_f32(y1), ref, what="Y")


@pytest.mark.parametrize("m,n,k,r", [(8, 8960, 1536, 16), (16, 4100, 1536, 96), (5, 4104, 2048, 32),
                                     (12, 4096, 3072, 64), (16, 8960, 1536, 128), (9, 1536, 1536, 16)])
def test_gemv_small_k_token_batches_match_oracle(m, n, k, r):
    """M = 5-16 at K = 1536, 2048, 3072 with at least one 16-row group per CU:
    the MFMA kernel with 3, 4 or 6 active waves; ranks above 32 per active
    wave (r = 128 at K = 1536) and fewer rows (1536) take the other kernel.
    Against the fp64 oracle, two calls bitwise equal."""
    print(f"gemv small-k batch m={m} n={n} k={k} r={r}", flush=True)
    s = 2.0
    w = seeded((n, k), 940 + n + k, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    x = seeded((m, k), 941 + m)
    a = uniform((r, k), 942, 1.0 / np.sqrt(k))
    b = seeded((n, r), 943, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    y1, y2 = _gemv(x, packed, qs, t, b, s), _gemv(x, packed, qs, t, b, s)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    ref = O.lora_linear_forward(bf16_values(x), wo, bf16_values(a), bf16_values(b), s)
    assert_close_fro(np_f32(y1), ref, what="Y")


@pytest.mark.parametrize("m,n,k,nested", [(8, 1536, 8960, True), (16, 256, 8960, True), (5, 520, 4864, True),
                                          (12, 1000, 6144, False), (16, 1536, 8960, False)])
def test_gemv_narrow_outputs_split_k_match_oracle(m, n, k, nested):
    """The fallback kernel for narrow outputs (at most 128 groups of 16 rows)
    with K split over workgroups and the fp32 partials summed in slice order:
    the Qwen2.5-1.5B down projection at M = 8 and 16, a K with an odd unit
    count and resolved scales; against the fp64 oracle, repeat bitwise."""
    print(f"gemv narrow split-k m={m} n={n} k={k} nested={nested}", flush=True)
    r, s = 16, 2.0
    w = seeded((n, k), 960 + n + k, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=nested)
    x = seeded((m, k), 961 + m)
    a = uniform((r, k), 962, 1.0 / np.sqrt(k))
    b = seeded((n, r), 963, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    y1, y2 = _gemv(x, packed, qs, t, b, s, nested=nested), _gemv(x, packed, qs, t, b, s, nested=nested)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
    ref = O.lora_linear_forward(bf16_values(x), wo, bf16_values(a), bf16_values(b), s)
    assert_close_fro(np_f32(y1), ref, what="Y")
