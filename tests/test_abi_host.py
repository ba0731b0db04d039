"""CPU-only checks: the C ABI library loads and exports every function declared
in include/molt_amd.h; the Python boundary mirrors the reference's error
behaviour without touching a GPU."""
from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch

import molt_amd
from molt_amd import _lib
from molt_amd.errors import CapabilityError

HEADER = Path(__file__).resolve().parents[1] / "include" / "molt_amd.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(molt_\w+)\s*\(", text, flags=re.M))


def test_library_exports_every_declared_symbol():
    declared = _declared()
    assert len(declared) >= 18
    lib = _lib.load()
    for name in declared:
        assert hasattr(lib, name), name
    assert set(_lib.SIGNATURES) == declared
    assert lib.molt_amd_version().startswith(b"molt_amd")


def test_workspace_queries_need_no_gpu():
    lib = _lib.load()
    assert lib.molt_nf4_double_quantize_workspace(917504) == 224 * 8
    assert lib.molt_lora_grad_workspace(8192, 4096, 64) > 0
    assert lib.molt_nf4_gemv_workspace(1, 4096, 4096) >= 0
    assert lib.molt_nf4_gemv_workspace(0, 4096, 4096) == 0


def test_invalid_arguments_return_codes_without_a_gpu():
    lib = _lib.load()
    rc = lib.molt_nf4_quantize(None, 0, 10, 64, 1, None, None, None, None)
    assert rc == _lib.MOLT_EINVAL
    assert b"null" in lib.molt_amd_last_error()
    w = _lib.NF4Weight()
    w.rows, w.cols, w.block_size = 4, 4, 64
    rc = lib.molt_nf4_gemv(None, 4, 32, w, None, 1, None, 0, 0.0, None, 4, None, 0, None)
    assert rc == _lib.MOLT_EINVAL
    with pytest.raises(ValueError):
        _lib.check(_lib.MOLT_EINVAL)
    with pytest.raises(CapabilityError):
        _lib.check(_lib.MOLT_EUNSUPPORTED)


def test_scheduled_nf4_lora_refuses_cpu():
    """tests/kernels/test_nf4_lora.py:82-93."""
    from molt_amd.methods import scheduled_nf4_lora

    class QuantState:
        pass

    x = torch.randn(2, 4, requires_grad=True)
    packed = torch.zeros(8, 1, dtype=torch.uint8)
    a = torch.randn(2, 4, requires_grad=True)
    b = torch.randn(4, 2, requires_grad=True)
    with pytest.raises(Exception, match="requires CUDA"):
        scheduled_nf4_lora(x, packed, a, b, QuantState(), 1.0)


def test_module_suffix_filter_refuses_when_no_compatible_projection():
    """tests/kernels/test_nf4_lora.py:96-103."""
    from molt_amd.methods import enable_scheduled_nf4_lora

    with pytest.raises(CapabilityError, match="down_proj"):
        enable_scheduled_nf4_lora(torch.nn.Sequential(torch.nn.Linear(4, 4)), module_suffixes=("down_proj",))


def test_gated_replay_patcher_validates_arguments():
    from molt_amd.methods import enable_asymmetric_gated_replay

    model = torch.nn.Sequential(torch.nn.Linear(4, 4))
    with pytest.raises(ValueError, match="negative"):
        enable_asymmetric_gated_replay(model, offload_blocks=-1)
    with pytest.raises(ValueError, match="mutually exclusive"):
        enable_asymmetric_gated_replay(model, offload_blocks=1)
    with pytest.raises(CapabilityError, match="No compatible"):
        enable_asymmetric_gated_replay(model)


def test_fused_silu_multiply_rejects_mismatch_and_cpu():
    """tests/kernels/test_gated_activation.py:45-47; CPU tensors are refused
    (no host fallback on the shipped path)."""
    from molt_amd.kernels import fused_silu_multiply

    with pytest.raises(ValueError, match="identical"):
        fused_silu_multiply(torch.randn(2, 3), torch.randn(2, 4))
    with pytest.raises(CapabilityError, match="CUDA"):
        fused_silu_multiply(torch.randn(2, 3), torch.randn(2, 3))


def test_codec_front_ends_refuse_cpu():
    with pytest.raises(CapabilityError):
        molt_amd.quantize_4bit(torch.randn(8, 64))
    from molt_amd import ops

    with pytest.raises(CapabilityError):
        ops.nf4_dequantize(torch.zeros(4, dtype=torch.uint8), torch.ones(1), molt_amd.NF4_CODEBOOK, 1, 8, 64, 1,
                           torch.bfloat16)


def test_quant_state_shape_and_dynamic_map():
    qs = molt_amd.QuantState(torch.zeros(4), (8, 32), molt_amd.NF4_CODEBOOK, 64)
    assert qs.quant_type == "nf4" and not qs.nested and qs.shape == torch.Size([8, 32])
    m = molt_amd.dynamic_map()
    assert m.shape == (256,) and bool((m[1:] > m[:-1]).all())


def test_fake_impls_give_shapes_without_a_gpu():
    from molt_amd import ops

    with torch._subclasses.fake_tensor.FakeTensorMode():
        x = torch.empty(10, 128, dtype=torch.bfloat16, device="cuda")
        a = torch.empty(4, 128, device="cuda")
        t = ops.lora_project(x, None, 0, 1.0, a, 0)
        assert t.shape == (10, 4)
        g = ops.lora_grad(x, None, 0, t, 1.0, 1)
        assert g.shape == (4, 128) and g.dtype == torch.float32
        inv = ops.rmsnorm_inv(x, torch.empty(128, device="cuda"), 1e-6)
        assert inv.shape == (10,) and inv.dtype == torch.float32
        gn = ops.lora_grad_rmsnorm(x, inv, torch.empty(128, device="cuda"), 0.0, t, 1.0, 1)
        assert gn.shape == (4, 128) and gn.dtype == torch.float32


def test_norm_replay_gradient_refuses_before_any_launch():
    lib = _lib.load()
    out = 0x1000
    # weight dtype, null operands, then 16-byte alignment / multiples of 8
    rc = lib.molt_lora_grad_rmsnorm(0x1000, 64, 0x1000, 0x1000, 7, 0.0, 0x1000, 8, 64, 64, 8, 1.0, out, 1, 0x1000,
                                    1 << 20, None)
    assert rc == _lib.MOLT_EINVAL and b"dtype" in lib.molt_amd_last_error()
    rc = lib.molt_lora_grad_rmsnorm(0x1000, 64, None, 0x1000, 0, 0.0, 0x1000, 8, 64, 64, 8, 1.0, out, 1, 0x1000,
                                    1 << 20, None)
    assert rc == _lib.MOLT_EINVAL and b"null" in lib.molt_amd_last_error()
    rc = lib.molt_lora_grad_rmsnorm(0x1002, 64, 0x1000, 0x1000, 0, 0.0, 0x1000, 8, 64, 64, 8, 1.0, out, 1, 0x1000,
                                    1 << 20, None)
    assert rc == _lib.MOLT_EUNSUPPORTED
    rc = lib.molt_lora_grad_rmsnorm(0x1000, 60, 0x1000, 0x1000, 0, 0.0, 0x1000, 8, 64, 60, 8, 1.0, out, 1, 0x1000,
                                    1 << 20, None)
    assert rc == _lib.MOLT_EUNSUPPORTED
    # too small a workspace is refused before the launch
    rc = lib.molt_lora_grad_rmsnorm(0x1000, 64, 0x1000, 0x1000, 0, 0.0, 0x1000, 8, 64, 64, 8, 1.0, out, 1, 0x1000,
                                    4, None)
    assert rc == _lib.MOLT_EWORKSPACE
    # inv-only RMSNorm needs an inv output
    rc = lib.molt_rmsnorm_forward(0x1000, 0, 64, 4, 64, 0x1000, 0, 1e-6, 0.0, None, 64, None, None)
    assert rc == _lib.MOLT_EINVAL


def test_statistics_and_row_checks_run_before_any_launch():
    """The ops refuse short or missing block statistics and low-rank operands
    with the wrong row count on the host, so no undersized pointer reaches a
    kernel (the checks need no GPU)."""
    from molt_amd.ops import _check_rows, _check_stats

    code = torch.zeros(16)
    _check_stats("t", 128, 64, 64, code, scales=torch.zeros(128))
    with pytest.raises(ValueError, match="127 block scales for 128 blocks"):
        _check_stats("t", 128, 64, 64, code, scales=torch.zeros(127))
    with pytest.raises(ValueError, match="0 block scales"):
        _check_stats("t", 128, 64, 64, code)
    with pytest.raises(ValueError, match="16 entries"):
        _check_stats("t", 128, 64, 64, torch.zeros(15), scales=torch.zeros(128))
    q = torch.zeros(1000, dtype=torch.uint8)
    _check_stats("t", 1000, 64, 64, code, absmax_q=q, absmax2=torch.zeros(4), code2=torch.zeros(256))
    with pytest.raises(ValueError, match="nested absmax"):
        _check_stats("t", 1001, 64, 64, code, absmax_q=q, absmax2=torch.zeros(4), code2=torch.zeros(256))
    with pytest.raises(ValueError, match="nested absmax"):
        _check_stats("t", 1000, 64, 64, code, absmax_q=q.float(), absmax2=torch.zeros(4), code2=torch.zeros(256))
    with pytest.raises(ValueError, match="second-level"):
        _check_stats("t", 1000, 64, 64, code, absmax_q=q, absmax2=torch.zeros(3), code2=torch.zeros(256))
    with pytest.raises(ValueError, match="256 entries"):
        _check_stats("t", 1000, 64, 64, code, absmax_q=q, absmax2=torch.zeros(4), code2=torch.zeros(255))
    _check_rows("t", "T", torch.zeros(5, 3), 5)
    with pytest.raises(ValueError, match="must have 6 rows"):
        _check_rows("t", "T", torch.zeros(5, 3), 6)


def test_tuning_settings_round_trip_without_a_gpu():
    from molt_amd._lib import TUNING_KEYS, tuning

    lib = _lib.load()
    before = {k: int(lib.molt_amd_get_tuning(v)) for k, v in TUNING_KEYS.items()}
    with tuning(big_tile_min=7, gemv_dot_m=2, lora_dma=0):
        assert lib.molt_amd_get_tuning(TUNING_KEYS["big_tile_min"]) == 7
        assert lib.molt_amd_get_tuning(TUNING_KEYS["gemv_dot_m"]) == 2
        assert lib.molt_amd_get_tuning(TUNING_KEYS["lora_dma"]) == 0
    assert {k: int(lib.molt_amd_get_tuning(v)) for k, v in TUNING_KEYS.items()} == before
    assert lib.molt_amd_set_tuning(TUNING_KEYS["gemv_dot_m"], 9) == _lib.MOLT_EINVAL
    assert lib.molt_amd_set_tuning(99, 1) == _lib.MOLT_EINVAL
    assert lib.molt_amd_get_tuning(99) == -2
    with pytest.raises(ValueError, match="unknown tuning"):
        tuning(nope=1)


def test_noalloc_gemv_refuses_oversized_partials_before_any_device_call():
    """The size check of molt_nf4_gemv_noalloc runs before it touches the
    device (this container has none), so an oversized request never launches."""
    lib = _lib.load()
    limit = int(lib.molt_nf4_gemv_noalloc_limit())
    assert limit == 8 << 20
    w = _lib.NF4Weight()
    w.rows, w.cols, w.block_size, w.dq_block, w.nested = 40000, 14336, 64, 256, 1
    need = int(lib.molt_nf4_gemv_workspace(16, w.rows, w.cols))
    assert need > limit
    rc = lib.molt_nf4_gemv_noalloc(None, 14336, 16, w, None, 1, None, 0, 0.0, None, 40000, None)
    assert rc == _lib.MOLT_EUNSUPPORTED
    assert b"static scratch" in lib.molt_amd_last_error()


def test_split_k_workspace_queries_need_no_gpu():
    """The split plan: a long contraction with few 256 x 256 output tiles gets
    fp32 partials for S splits; a problem that fills the GPU gets none."""
    from molt_amd._lib import tuning

    lib = _lib.load()
    with tuning(stage_min_mtiles=0):
        assert lib.molt_nf4_lora_forward_workspace(8192, 14336, 4096, 0) == 0
        assert lib.molt_nf4_lora_forward_workspace(4096, 1536, 8960, 0) == 2 * 4096 * 1536 * 4
        assert lib.molt_nf4_lora_backward_workspace(4096, 8960, 1536, 2) == 2 * 4096 * 1536 * 4
        assert lib.molt_nf4_lora_backward_workspace(8192, 14336, 4096, 2) == 0
        assert lib.molt_nf4_lora_forward_workspace(4096, 1000, 8960, 0) == 0       # N not a multiple of 256
        with tuning(split_k=0):
            assert lib.molt_nf4_lora_forward_workspace(4096, 1536, 8960, 0) == 0


def _stage(rows, cols):
    return (rows * cols * 2 + 255) // 256 * 256


def test_staged_weight_workspace_queries_need_no_gpu():
    """From stage_min_mtiles 256-row blocks of X (default 16) the large-tile
    GEMMs take a bf16 copy of each weight first in the workspace, then any
    split-K partials; fewer rows, or a setting of 0, stage nothing."""
    from molt_amd._lib import tuning

    lib = _lib.load()
    assert lib.molt_amd_get_tuning(_lib.TUNING_KEYS["stage_min_mtiles"]) == 16
    assert lib.molt_nf4_lora_forward_workspace(8192, 14336, 4096, 0) == _stage(14336, 4096)
    assert lib.molt_nf4_gateup_forward_workspace(8192, 14336, 4096, 0) == 2 * _stage(14336, 4096)
    assert lib.molt_nf4_lora_backward_workspace(8192, 14336, 4096, 2) == 2 * _stage(14336, 4096)
    assert lib.molt_nf4_lora_backward_workspace(8192, 4096, 14336, 1) == _stage(4096, 14336)
    assert lib.molt_nf4_lora_forward_workspace(4096, 1536, 8960, 0) == _stage(1536, 8960) + 2 * 4096 * 1536 * 4
    assert lib.molt_nf4_lora_backward_workspace(4096, 8960, 1536, 2) == 2 * _stage(8960, 1536) + 2 * 4096 * 1536 * 4
    assert lib.molt_nf4_lora_forward_workspace(2048, 14336, 4096, 0) == 0          # 8 row blocks
    assert lib.molt_nf4_gateup_forward_workspace(256, 14336, 4096, 0) == 0
    assert lib.molt_nf4_lora_backward_workspace(8192, 1024, 4160, 1) == 0       # Kw not a multiple of 256
    with tuning(stage_min_mtiles=0):
        assert lib.molt_nf4_gateup_forward_workspace(8192, 14336, 4096, 0) == 0
    with tuning(stage_min_mtiles=8):
        assert lib.molt_nf4_lora_forward_workspace(2048, 14336, 4096, 0) == _stage(14336, 4096)
    # in the forward, a LoRA length that is a multiple of 64 adds the bf16(s B) rows the ring streams;
    # a shorter one (a multiple of 8) adds them padded to 64 columns
    assert lib.molt_nf4_lora_forward_workspace(8192, 4096, 14336, 64) == _stage(4096, 14336) + _stage(4096, 64)
    assert lib.molt_nf4_gateup_forward_workspace(8192, 14336, 4096, 64) == 2 * (_stage(14336, 4096)
                                                                                 + _stage(14336, 128))
    assert lib.molt_nf4_gateup_forward_workspace(8192, 14336, 4096, 16) == 2 * (_stage(14336, 4096)
                                                                                 + _stage(14336, 64))  # 2r = 32
    assert lib.molt_nf4_lora_forward_workspace(8192, 4096, 14336, 16) == _stage(4096, 14336) + _stage(4096, 64)
    assert lib.molt_nf4_lora_forward_workspace(8192, 4096, 14336, 12) == _stage(4096, 14336)   # not a multiple of 8
    assert lib.molt_nf4_lora_forward_workspace(4096, 1536, 8960, 64) == (_stage(1536, 8960) + _stage(1536, 64)
                                                                         + 2 * 4096 * 1536 * 4)
