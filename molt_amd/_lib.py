"""ctypes binding of libmolt_amd.so (the C ABI declared in include/molt_amd.h).

torch is imported before the library is opened so that its
``libamdhip64.so.7`` (SONAME-identical to ROCm's) satisfies the library's HIP
dependency: one HIP runtime per process, so torch stream handles and device
pointers are valid arguments. There is no CPU fallback: every op raises when
the library is missing or no GPU is present.
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

from .errors import CapabilityError

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libmolt_amd.so"

MOLT_OK, MOLT_EINVAL, MOLT_EUNSUPPORTED, MOLT_ELAUNCH, MOLT_EWORKSPACE = 0, 1, 2, 3, 4
DTYPE_BF16, DTYPE_F32 = 0, 1
TUNING_KEYS = {"big_tile_min": 0, "gemv_dot_m": 1, "lora_dma": 2, "split_k": 3, "split_min_steps": 4,
               "stage_min_mtiles": 5}   # MOLT_TUNE_* of include/molt_amd.h

_p = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int32
_f32 = C.c_float
_sz = C.c_size_t


class NF4Weight(C.Structure):
    """Mirror of ``molt_nf4_weight``."""
    _fields_ = [
        ("packed", _p), ("scales", _p), ("absmax_q", _p), ("absmax2", _p),
        ("code2", _p), ("code", _p), ("offset", _f32), ("nested", _i32),
        ("block_size", _i32), ("dq_block", _i32), ("nibble_order", _i32),
        ("rows", _i64), ("cols", _i64),
    ]


_W = C.POINTER(NF4Weight)


class LoraGradDesc(C.Structure):
    """``molt_lora_grad_desc`` of include/molt_amd.h (one gradient of
    ``molt_lora_grad_many``)."""
    _fields_ = [
        ("l", C.c_void_p), ("l2", C.c_void_p), ("ldl", C.c_int64), ("l_mode", C.c_int32),
        ("rmat", C.c_void_p), ("ldr", C.c_int64),
        ("M", C.c_int64), ("P", C.c_int64), ("Q", C.c_int64),
        ("scale", C.c_float), ("out", C.c_void_p), ("out_layout", C.c_int32),
        ("inv_rms", C.c_void_p), ("norm_weight", C.c_void_p), ("w_dtype", C.c_int32), ("norm_offset", C.c_float),
    ]


_GD = C.POINTER(LoraGradDesc)


class LoraPackDesc(C.Structure):
    """``molt_lora_pack_desc`` of include/molt_amd.h (one adapter of
    ``molt_lora_pack_many``)."""
    _fields_ = [
        ("lora", C.c_void_p), ("lora2", C.c_void_p), ("split", C.c_int32), ("layout", C.c_int32),
        ("r", C.c_int32), ("D", C.c_int64), ("packed", C.c_void_p),
    ]


_PD = C.POINTER(LoraPackDesc)

# name -> (restype, argtypes); the exact list of include/molt_amd.h.
SIGNATURES: dict[str, tuple] = {
    "molt_amd_last_error": (C.c_char_p, []),
    "molt_amd_version": (C.c_char_p, []),
    "molt_amd_set_tuning": (C.c_int, [_i32, _i64]),
    "molt_amd_get_tuning": (_i64, [_i32]),
    "molt_nf4_dequantize": (C.c_int, [_W, _p, _i32, _p]),
    "molt_nf4_resolve_scales": (C.c_int, [_W, _p, _p]),
    "molt_nf4_quantize": (C.c_int, [_p, _i32, _i64, _i32, _i32, _p, _p, _p, _p]),
    "molt_nf4_double_quantize_workspace": (_sz, [_i64]),
    "molt_nf4_double_quantize": (C.c_int, [_p, _i64, _i32, _p, _p, _p, _p, _p, _sz, _p]),
    "molt_lora_project_workspace": (_sz, [_i64, _i64, _i32]),
    "molt_lora_project": (C.c_int, [_p, _p, _i64, _i32, _f32, _i64, _i64, _p, _i32, _i32, _p, _i64, _p, _sz,
                                    _p]),
    "molt_lora_packed_bytes": (_sz, [_i64, _i32]),
    "molt_lora_pack_many": (C.c_int, [_i32, _PD, _p]),
    "molt_lora_project_packed_workspace": (_sz, [_i64, _i64, _i32]),
    "molt_lora_project_packed": (C.c_int, [_p, _p, _i64, _i32, _f32, _i64, _i64, _p, _i32, _p, _i64, _p, _sz, _p]),
    "molt_lora_project_pair_packed_workspace": (_sz, [_i64, _i64, _i32]),
    "molt_lora_project_pair_packed": (C.c_int, [_p, _p, _i64, _i32, _f32, _f32, _i64, _i64, _p, _p, _i32, _p, _i64,
                                                _p, _sz, _p]),
    "molt_amd_time_next_gemm": (C.c_int, [_p, _p]),
    "molt_nf4_lora_forward_workspace": (_sz, [_i64, _i64, _i64, _i32]),
    "molt_nf4_lora_forward": (C.c_int, [_p, _i64, _i64, _W, _p, _i64, _p, _i32, _f32, _p, _i64, _p, _sz, _p]),
    "molt_nf4_gateup_forward_workspace": (_sz, [_i64, _i64, _i64, _i32]),
    "molt_nf4_gateup_forward": (C.c_int, [_p, _i64, _i64, _W, _W, _p, _i64, _p, _p, _i32, _f32, _f32,
                                          _p, _p, _p, _i64, _p, _sz, _p]),
    "molt_nf4_lora_backward_workspace": (_sz, [_i64, _i64, _i64, _i32]),
    "molt_nf4_lora_backward_input": (C.c_int, [_p, _i64, _i64, _W, _p, _i64, _p, _i32, _f32, _p, _i64, _p, _sz,
                                               _p]),
    "molt_nf4_lora_backward_input_pair": (C.c_int, [_p, _p, _i64, _i64, _W, _W, _p, _p, _i64, _p, _p,
                                                    _i32, _p, _i64, _p, _sz, _p]),
    "molt_nf4_swiglu_backward": (C.c_int, [_p, _i64, _i64, _W, _p, _i64, _p, _i32, _p, _p, _i64, _p, _p,
                                           _p, _sz, _p]),
    "molt_nf4_keeps_wt": (_i32, [_i64, _i64, _i64, _i32]),
    "molt_nf4_lora_forward_keep_wt": (C.c_int, [_p, _i64, _i64, _W, _p, _i64, _p, _i32, _f32, _p, _i64, _p, _p,
                                                _p, _sz, _p]),
    "molt_nf4_gateup_forward_keep_wt": (C.c_int, [_p, _i64, _i64, _W, _W, _p, _i64, _p, _p, _i32, _f32, _f32,
                                                  _p, _p, _p, _i64, _p, _p, _p, _p, _sz, _p]),
    "molt_nf4_lora_backward_workspace_wt": (_sz, [_i64, _i64, _i64, _i32]),
    "molt_nf4_lora_backward_input_wt": (C.c_int, [_p, _i64, _i64, _W, _p, _p, _i64, _p, _i32, _f32, _p, _i64,
                                                  _p, _sz, _p]),
    "molt_nf4_lora_backward_input_pair_wt": (C.c_int, [_p, _p, _i64, _i64, _W, _W, _p, _p, _p, _p, _i64, _p,
                                                       _p, _i32, _p, _i64, _p, _sz, _p]),
    "molt_nf4_swiglu_backward_wt": (C.c_int, [_p, _i64, _i64, _W, _p, _p, _i64, _p, _i32, _p, _p, _i64, _p,
                                              _p, _p, _sz, _p]),
    "molt_lora_grad_workspace": (_sz, [_i64, _i64, _i64]),
    "molt_lora_grad": (C.c_int, [_p, _p, _i64, _i32, _p, _i64, _i64, _i64, _i64, _f32, _p, _i32, _p, _sz,
                                 _p]),
    "molt_lora_grad_many_workspace": (_sz, [_i32, _GD]),
    "molt_lora_grad_many": (C.c_int, [_i32, _GD, _p, _sz, _p]),
    "molt_lora_stack_adapters": (C.c_int, [_i32, C.POINTER(_p), C.POINTER(_p), C.POINTER(_i64), _i32, _i64, _i32,
                                           _p, _p, _p]),
    "molt_nf4_stacked_forward": (C.c_int, [_p, _i64, _i64, _i32, _W, _p, _i64, _i32, _p, _i64, _f32, _p, _i64,
                                           _p, _p, _p, _sz, _p]),
    "molt_nf4_stacked_backward_input": (C.c_int, [_p, _i64, _i64, _i32, _W, _p, _p, _i64, _p, _i32, _f32, _p,
                                                  _i64, _p, _sz, _p]),
    "molt_lora_grad_rmsnorm": (C.c_int, [_p, _i64, _p, _p, _i32, _f32, _p, _i64, _i64, _i64, _i64, _f32, _p,
                                         _i32, _p, _sz, _p]),
    "molt_nf4_gemv_workspace": (_sz, [_i64, _i64, _i64]),
    "molt_nf4_gemv": (C.c_int, [_p, _i64, _i64, _W, _p, _i64, _p, _i32, _f32, _p, _i64, _p, _sz, _p]),
    "molt_nf4_gemv_noalloc_limit": (_sz, []),
    "molt_nf4_gemv_noalloc": (C.c_int, [_p, _i64, _i64, _W, _p, _i64, _p, _i32, _f32, _p, _i64, _p]),
    "molt_silu_mul_forward": (C.c_int, [_p, _p, _p, _i64, _i32, _i32, _p]),
    "molt_silu_mul_backward": (C.c_int, [_p, _p, _p, _p, _p, _i64, _i32, _p]),
    "molt_rmsnorm_forward": (C.c_int, [_p, _i32, _i64, _i64, _i64, _p, _i32, _f32, _f32, _p, _i64, _p, _p]),
    "molt_rmsnorm_backward": (C.c_int, [_p, _i64, _p, _i32, _i64, _i64, _i64, _p, _i32, _f32, _f32, _p, _i64,
                                        _p]),
    "molt_cross_entropy_rows": (C.c_int, [_p, _i32, _i64, _i64, _i64, _p, _f32, _p, _p, _i64, _p]),
    "molt_cross_entropy_rows_exact": (C.c_int, [_p, _i32, _i64, _i64, _i64, _p, _f32, _p, _p, _p, _i64, _p]),
}

_lock = threading.Lock()
_lib: C.CDLL | None = None


def load(path: Path | str | None = None) -> C.CDLL:
    """Open the library (once) and bind every declared symbol."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = Path(path) if path is not None else LIB_PATH
        if not target.exists():
            raise CapabilityError(
                f"{target} is not built; run `python -m molt_amd.build` (hipcc, gfx950)")
        lib = C.CDLL(str(target))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def check(rc: int) -> None:
    if rc == MOLT_OK:
        return
    msg = (load().molt_amd_last_error() or b"").decode(errors="replace")
    if rc == MOLT_EUNSUPPORTED:
        raise CapabilityError(msg)
    if rc in (MOLT_EINVAL, MOLT_EWORKSPACE):
        raise ValueError(msg)
    raise RuntimeError(msg)


# Bumped by every change made through `tuning`, so that cached workspace sizes
# (which follow the kernel choice) are looked up again.
tuning_generation = 0


class tuning:
    """Kernel-choice settings of the library (``molt_amd_set_tuning``), as a
    context manager that restores the previous values on exit::

        with tuning(big_tile_min=1):   # force the 256 x 256 tile GEMMs
            ...

    Keys: ``big_tile_min``, ``gemv_dot_m``, ``lora_dma``, ``split_k``, ``split_min_steps``,
    ``stage_min_mtiles``. Settings are process wide; callers that change them concurrently race."""

    def __init__(self, **values: int) -> None:
        unknown = set(values) - set(TUNING_KEYS)
        if unknown:
            raise ValueError(f"unknown tuning keys {sorted(unknown)}; known: {sorted(TUNING_KEYS)}")
        self.values = values
        self.saved: dict[str, int] = {}

    def __enter__(self) -> "tuning":
        global tuning_generation
        lib = load()
        for name, value in self.values.items():
            key = TUNING_KEYS[name]
            self.saved[name] = int(lib.molt_amd_get_tuning(key))
            check(lib.molt_amd_set_tuning(key, int(value)))
        tuning_generation += 1
        return self

    def __exit__(self, *exc) -> None:
        global tuning_generation
        lib = load()
        for name, value in self.saved.items():
            check(lib.molt_amd_set_tuning(TUNING_KEYS[name], value))
        tuning_generation += 1
