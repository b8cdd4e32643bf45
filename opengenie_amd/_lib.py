"""ctypes binding of libopengenie_amd.so (the C ABI in include/opengenie_amd.h).

The library is loaded on first use. If it is missing the call raises: a GPU
tensor never silently takes another path because the extension is absent.
"""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libopengenie_amd.so")

DT_BF16 = 0
DT_F32 = 1
DT_F16 = 2
ROWS_ADAZERO = 0
ROWS_ELEMENTWISE = 1

_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_p = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); must match include/opengenie_amd.h
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "oga_abi_version": (_i32, []),
    "oga_last_error": (ctypes.c_char_p, []),
    "oga_adazero_from_ada": (_i32, [_p, _p, _i64, _i64, _i64, _p, _i32, _i64, _i64, _p, _i32, _i64p, _i32, _i32,
                                    _f32, _p]),
    "oga_adazero_from_ada_fp8": (_i32, [_p, _p, _i64, _i64, _i64, _p, _i32, _i64, _i64, _p, _i32, _i64p, _i32,
                                        _i32, _f32, _p, _i32, _p]),
    "oga_adazero": (_i32, [_p, _p, _i64, _i64, _i64, _p, _i32, _i64p, _p, _i32, _i64p, _f32, _p]),
    "oga_adaln_affine_from_ada": (_i32, [_p, _p, _i64, _i64, _i64, _p, _i32, _i64, _i64, _p, _i32, _i64p, _i32,
                                         _i32, _p]),
    "oga_mul_from_ada": (_i32, [_p, _p, _i64, _i64, _i64, _p, _i32, _i64, _i64, _p, _i32, _i64p, _i32, _p]),
    "oga_residual_gate_from_ada": (_i32, [_p, _p, _p, _i64, _i64, _i64, _p, _i32, _i64, _i64, _p, _i32, _i64p,
                                          _i32, _p]),
    "oga_residual_gate_bias_from_ada": (_i32, [_p, _p, _p, _i32, _p, _i64, _i64, _i64, _p, _i32, _i64, _i64, _p,
                                               _i32, _i64p, _i32, _p]),
    "oga_residual_gate_adazero_from_ada": (_i32, [_p, _p, _p, _i32, _p, _p, _i64, _i64, _i64, _p, _i32, _i64, _i64,
                                                  _p, _i32, _i64p, _i32, _i32, _i32, _f32, _p, _i32, _p]),
    "oga_residual_gate_bf16": (_i32, [_p, _p, _p, _i64p, _p, _i64, _i64, _i64, _p]),
    "oga_bias_add_bf16": (_i32, [_p, _p, _i32, _p, _i64, _i64, _p]),
    "oga_head_gate_mul_bf16": (_i32, [_p, _p, _i64, _i64, _p, _i64, _i64, _i64, _p]),
    "oga_fp8_quantize_e4m3": (_i32, [_p, _i32, _p, _i32, _p, _i64, _p]),
    "oga_gelu_tanh_fp8_quantize_e4m3": (_i32, [_p, _i32, _p, _i32, _p, _i64, _p]),
    "oga_fp8_per_head_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "oga_fp8_quantize_per_head": (_i32, [_p, _i32, _p, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "oga_video_qk_rmsnorm_rope": (_i32, [_p, _p, _p, _p, _i32, _p, _p, _i32, _i64p, _i64p, _p, _p, _i64, _i64,
                                         _i64, _i64, _f32, _p]),
    "oga_video_rmsnorm_rope": (_i32, [_p, _p, _i32, _p, _p, _i32, _i64p, _i64p, _p, _i64, _i64, _i64, _i64, _f32,
                                      _p]),
    "oga_rmsnorm": (_i32, [_p, _p, _i32, _p, _i64, _i64, _f32, _p]),
    "oga_video_qk_bias_rmsnorm_rope": (_i32, [_p, _p, _p, _p, _i32, _p, _p, _i32, _p, _p, _i32, _i64p, _i64p, _p,
                                              _p, _i64, _i64, _i64, _i64, _f32, _p]),
    "oga_video_qkv_rmsnorm_rope_pack": (_i32, [_p, _p, _p, _p, _p, _i32, _p, _p, _i32, _i64p, _i64p, _p, _i64,
                                               _i64, _i64, _i64, _f32, _p]),
    "oga_fp8_linear": (_i32, [_p, _i64, _p, _i64, _p, _p, _p, _i32, _p, _i64, _i64, _i64, _i64, _p]),
    "oga_fp8_linear_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "oga_fp8_linear_ws": (_i32, [_p, _i64, _p, _i64, _p, _p, _p, _i32, _p, _i64, _i64, _i64, _i64, _p, _i64, _p]),
    "oga_fp8_linear_dt_ws": (_i32, [_p, _i64, _p, _i64, _p, _p, _p, _i32, _p, _i32, _i64, _i64, _i64, _i64, _p, _i64,
                                    _p]),
    "oga_fp8_linear_grouped_ws": (_i32, [_p, _i64, _p, _i64, _p, _p, _p, _i32, _p, _i64, _i64, _i64, _i64, _i64, _p,
                                         _i64, _p]),
    "oga_attention": (_i32, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _i64, _f32, _p]),
    "oga_attention_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "oga_attention_ws": (_i32, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _i64, _f32, _p,
                                _i64, _p]),
    "oga_attention_e4m3_out_ws": (_i32, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _i64,
                                         _f32, _p, _i32, _p, _i64, _p]),
    "oga_fp8_dequant_per_head": (_i32, [_p, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "oga_attention_fp8_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "oga_attention_fp8_ws": (_i32, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _p, _p, _p, _i64p, _i64, _i64, _i64, _i64,
                                    _i64, _f32, _p, _i64, _p]),
    "oga_selftest_convert": (_i32, [_p, _p, _p, _i64, _p]),
    "oga_rows_per_wave": (_i64, [_i32, _i64, _i64, _i64]),
    "oga_fp8_per_head_noalloc_max_bytes": (_i64, []),
    "oga_fp8_quantize_per_head_noalloc": (_i32, [_p, _i32, _p, _p, _i64, _i64, _i64, _i64, _p]),
}

_lock = threading.Lock()
_lib = None


class LibraryMissing(RuntimeError):
    pass


class KernelError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """The loaded library (raises LibraryMissing if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise LibraryMissing(
                    f"{LIB_PATH} is not built; run `python -m opengenie_amd.build` (needs ROCm hipcc)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def available() -> bool:
    return os.path.exists(LIB_PATH)


def strides(values) -> ctypes.Array:
    arr = (ctypes.c_int64 * len(values))(*[int(v) for v in values])
    return arr


def call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.oga_last_error().decode() if rc < 0 else f"hipError {rc}"
        raise KernelError(f"{name} failed (rc={rc}): {msg}")
