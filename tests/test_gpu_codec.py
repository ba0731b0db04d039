"""NF4 codec on the GPU vs the CPU oracle: codes, absmax, nested statistics,
resolved scales and dequantised bf16/fp32 weights must be bit-exact."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as O
from tests._util import np_bits, np_f32, oracle_weight, seeded

import molt_amd
from molt_amd import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,block", [((64, 64), 64), ((70, 65), 64), ((8, 8), 16), ((33, 7), 32),
                                         ((128, 96), 64), ((5, 200), 50)])
@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quantize_codes_and_absmax_bit_exact(shape, block, order, dtype):
    print(f"quantize shape={shape} block={block} order={order} dtype={dtype}", flush=True)
    x = seeded(shape, 100 + block + order, std=0.02, dtype=dtype)
    packed, absmax = ops.nf4_quantize(x, block, order, molt_amd.NF4_CODEBOOK.cuda())
    idx, am = O.quantize_blocks(np_f32(x), block)
    assert np.array_equal(np_f32(absmax).view(np.uint32), am.view(np.uint32))
    assert np.array_equal(packed.cpu().numpy(), O.pack_nibbles(idx, order))


@pytest.mark.parametrize("block", [32, 64])
def test_quantize_special_values(block):
    """Zero blocks (absmax clamped to FLT_MIN), exact codes, ties; block 64
    takes the one-element-per-lane path, block 32 the pair-per-lane one."""
    code = O.NF4_CODE
    lo, hi = code[9], code[10]
    mid = np.float32((np.float64(lo) + np.float64(hi)) / 2)
    x = np.concatenate([np.zeros(64, np.float32), code * np.float32(3.0), code * np.float32(-0.25),
                        np.array([1.0, mid, -mid] + [0.0] * 29, np.float32)]).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    for order in (0, 1):
        packed, absmax = ops.nf4_quantize(xt, block, order, molt_amd.NF4_CODEBOOK.cuda())
        idx, am = O.quantize_blocks(x, block)
        assert np.array_equal(np_f32(absmax).view(np.uint32), am.view(np.uint32))
        assert np.array_equal(packed.cpu().numpy(), O.pack_nibbles(idx, order))


def test_quantize_block64_more_blocks_than_one_pass():
    """135,168 blocks of 64: more than one pass of the block-64 path's grid
    (8192 workgroups x 4 waves x 4 blocks), the second pass partial."""
    shape = (4096, 2112)
    print(f"quantize block64 multi-pass shape={shape}", flush=True)
    x = seeded(shape, 7, std=0.02, dtype=torch.bfloat16)
    packed, absmax = ops.nf4_quantize(x, 64, 1, molt_amd.NF4_CODEBOOK.cuda())
    idx, am = O.quantize_blocks(np_f32(x), 64)
    assert np.array_equal(np_f32(absmax).view(np.uint32), am.view(np.uint32))
    assert np.array_equal(packed.cpu().numpy(), O.pack_nibbles(idx, 1))


@pytest.mark.parametrize("n", [1, 255, 256, 4096, 4097, 70000, 300000])
def test_double_quantize_bit_exact(n):
    print(f"double quantize n={n}", flush=True)
    g = torch.Generator().manual_seed(n)
    absmax = (torch.randn(n, generator=g).abs() * 0.02 + 1e-4).float()
    code2 = molt_amd.dynamic_map()
    q, absmax2, offset = ops.nf4_double_quantize(absmax.cuda(), code2.cuda(), 256)
    oq, oa2, ooff, _ = O.double_quantize(absmax.numpy(), code2.numpy())
    assert np.float32(offset.item()).view(np.uint32) == np.float32(ooff).view(np.uint32)
    assert np.array_equal(np_f32(absmax2).view(np.uint32), oa2.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), oq)


@pytest.mark.parametrize("shape", [(64, 64), (70, 65), (256, 384), (4864, 896)])
@pytest.mark.parametrize("nested", [True, False])
def test_quantize_4bit_dequantize_4bit_bit_exact(shape, nested):
    print(f"quantize_4bit/dequantize_4bit shape={shape} nested={nested}", flush=True)
    w = seeded(shape, 7, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=nested)
    ow = O.quantize_bnb_layout(np_f32(w), 64, nested=nested)
    assert np.array_equal(packed.reshape(-1).cpu().numpy(), ow.packed[: packed.numel()])
    if nested:
        assert np.array_equal(qs.absmax.cpu().numpy(), ow.q)
        assert np.float32(float(qs.offset)).view(np.uint32) == np.float32(ow.offset).view(np.uint32)
    scales = molt_amd.resolved_nf4_scales(qs)
    assert np.array_equal(np_f32(scales).view(np.uint32), ow.scales.view(np.uint32))
    dense = molt_amd.dequantize_4bit(packed, qs)
    assert dense.dtype == torch.float32 and dense.shape == shape
    assert np.array_equal(np_f32(dense).view(np.uint32), ow.dequant_f32().view(np.uint32))
    dense_bf16 = molt_amd.dequantize_4bit(packed, qs, torch.bfloat16)
    assert np.array_equal(np_bits(dense_bf16), ow.dequant_bf16_bits())


def test_dequantize_bf16_weights_of_bf16_input():
    w = seeded((1536, 256), 944, std=1.0, dtype=torch.bfloat16)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    assert qs.dtype == torch.bfloat16
    ow = oracle_weight(packed, qs)
    assert np.array_equal(np_bits(molt_amd.dequantize_4bit(packed, qs)), ow.dequant_bf16_bits())


def test_cleanroom_nf4tensor_round_trip():
    """streaming/nf4.py semantics: low nibble first, fp32 scales, padding."""
    torch.manual_seed(1)
    value = torch.randn(64, 64)
    t = molt_amd.NF4Tensor.quantize(value, block_size=64)
    ow = O.quantize_cleanroom(value.numpy(), 64)
    assert np.array_equal(t.packed.numpy(), ow.packed)
    assert np.array_equal(t.scales.numpy().view(np.uint32), ow.scales.view(np.uint32))
    assert t.storage_bytes == value.numel() // 2 + value.numel() // 64 * 4
    restored = t.dequantize(device="cuda").cpu()
    assert np.array_equal(restored.numpy().view(np.uint32), ow.dequant_f32().view(np.uint32))
    assert torch.mean((restored - value) ** 2).sqrt() < 0.15
    odd = torch.randn(3, 37)
    t2 = molt_amd.NF4Tensor.quantize(odd, block_size=16)
    ow2 = O.quantize_cleanroom(odd.numpy(), 16)
    assert np.array_equal(t2.packed.numpy(), ow2.packed)
    bf = t2.dequantize(device="cuda", dtype=torch.bfloat16).cpu()
    assert np.array_equal(np_bits(bf), ow2.dequant_bf16_bits())
