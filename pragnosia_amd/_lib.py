"""ctypes binding of libpragnosia_hip.so (the C ABI declared in include/pragnosia_hip.h).

There is no fallback: if the library is missing or a call is made on a non-ROCm tensor, this raises."""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpragnosia_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "pragnosia_hip.h")

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# argument types of every entry point, in header order
SIGNATURES = {
    "pragnosia_abi_version": [],
    "pragnosia_error_string": [_i32],
    "pragnosia_diag_scan_fwd": [_p] * 9 + [_i64] * 3 + [_p],
    "pragnosia_diag_scan_bwd": [_p] * 14 + [_i64] * 3 + [_p],
    "pragnosia_aspin_chunk_fwd": [_p] * 8 + [_i64] * 5 + [_p],
    "pragnosia_aspin_chunk_bwd": [_p] * 12 + [_i64] * 5 + [_p],
    "pragnosia_aspin_chunk_seg_workspace_bytes": [_i64] * 6,
    "pragnosia_aspin_chunk_fwd_seg": [_p] * 6 + [_i64] + [_p] * 4 + [_i64] * 7 + [_p],
    "pragnosia_aspin_chunk_bwd_seg": [_p] * 13 + [_i64] * 7 + [_p],
    "pragnosia_aspin_chunk_fwd_seg_noalloc": [_p] * 6 + [_i64] + [_p] * 3 + [_i64] * 6 + [_p],
    "pragnosia_aspin_chunk_wide_workspace_bytes": [_i64] * 6 + [_i32],
    "pragnosia_aspin_chunk_fwd_wide": [_p] * 9 + [_i64] * 7 + [_p],
    "pragnosia_aspin_chunk_bwd_wide": [_p] * 13 + [_i64] * 7 + [_p],
    "pragnosia_aspin_out_fwd": [_p] * 2 + [_f32, _p, _i32, _p] + [_i64] * 4 + [_p],
    "pragnosia_layer_norm_fwd": [_p] * 3 + [_f32, _p, _i32, _p, _p, _i64, _i64, _p],
    "pragnosia_layer_norm_partials": [_i64] * 2,
    "pragnosia_layer_norm_bwd": [_p, _i32] + [_p] * 7 + [_i64, _i64, _p],
    "pragnosia_colsum_f32": [_p, _i64, _i64, _p, _p],
    "pragnosia_wgrad_workspace_bytes": [_i64] * 3,
    "pragnosia_wgrad_bf16": [_p, _i64, _p, _i64, _p, _i64, _i32, _p, _i64, _i64, _i64, _i64, _p],
    "pragnosia_aspin_out_weight_partials": [_i64] * 3,
    "pragnosia_aspin_out_bwd": [_p, _i32] + [_p] * 5 + [_i64] * 4 + [_p],
    "pragnosia_aspin_exact_fwd": [_p] * 10 + [_i64] * 5 + [_i32, _p],
    "pragnosia_aspin_exact_bwd": [_p] * 15 + [_i64] * 5 + [_i32, _p],
    "pragnosia_aspin_delta_fwd": [_p] * 11 + [_i64] * 5 + [_p],
    "pragnosia_aspin_delta_bwd_workspace_bytes": [_i64] * 5,
    "pragnosia_aspin_delta_bwd": [_p] * 17 + [_i64] * 6 + [_p],
    "pragnosia_aspin_delta_window_prefix": [_p] * 4 + [_f32, _p] + [_i64] * 3 + [_p],
    "pragnosia_aspin_delta_window_maps": [_p] * 6 + [_i64] * 2 + [_p],
    "pragnosia_aspin_prep_fwd": [_p] * 9 + [_i64] * 5 + [_i32, _p],
    "pragnosia_aspin_prep_theta_partials": [_i64] * 2,
    "pragnosia_aspin_prep_bwd": [_p] * 14 + [_i64] * 5 + [_i32, _p],
    "pragnosia_aspin_prep_proj_fwd": [_p] + [_i64] * 4 + [_p] * 5 + [_f32] + [_p] * 7 + [_i64] * 4 + [_i32, _p],
    "pragnosia_aspin_prep_proj_partials": [_i64] * 3,
    "pragnosia_aspin_prep_proj_bwd": [_p] + [_i64] * 4 + [_p] * 5 + [_f32] + [_p] * 10 + [_i64] * 4 + [_i32, _p],
    "pragnosia_aspin_rebase_fwd": [_p] * 3 + [_f32, _p] + [_i64] * 3 + [_p],
    "pragnosia_aspin_rebase_bwd": [_p] * 3 + [_f32] + [_p] * 3 + [_i64] * 3 + [_p],
    "pragnosia_aspin_decode_step": [_p] * 10 + [_f32, _p] + [_i64] * 3 + [_p],
    "pragnosia_aspin_decode_proj": [_p] * 3 + [_i64] * 4 + [_p] * 5 + [_f32] + [_p] * 2 + [_f32, _p, _f32, _p]
                                   + [_i64] * 3 + [_p],
    "pragnosia_aspin_decode_oproj": [_p] * 3 + [_i64] * 4 + [_p] * 5 + [_f32] + [_p] * 2 + [_f32, _p, _f32, _p, _i64]
                                    + [_p] * 2 + [_i64] * 3 + [_p],
    "pragnosia_decode_gemv": [_p, _i64, _i64, _p, _p, _f32, _p, _i64, _p, _p, _i32, _p, _p, _p],
    "pragnosia_decode_gemv_rms": [_p, _i64, _i64, _p, _i64, _f32, _p, _i64, _p, _p, _i32, _p, _p, _p],
    "pragnosia_decode_tail": [_p, _i64, _i64, _p, _p, _i64, _i64] + [_p] * 5 + [_i64, _p, _p, _p, _i64, _p, _p],
    "pragnosia_decode_gemm_waves": [_i64, _i32],
    "pragnosia_decode_gemm": [_p, _i64, _i64, _i32, _p, _f32, _p, _i64, _p, _p, _i32, _p, _p, _p],
    "pragnosia_decode_gemm_acc": [_p, _i64, _i64, _i32, _f32, _p, _i64, _p, _p, _p, _p],
    "pragnosia_decode_gemv_acc": [_p, _i64, _i64, _p, _i64, _p, _p, _p, _p],
}

# entry points that return a size (int64) rather than a status code
_RET_I64 = {"pragnosia_aspin_delta_bwd_workspace_bytes", "pragnosia_aspin_prep_theta_partials",
            "pragnosia_aspin_chunk_seg_workspace_bytes", "pragnosia_aspin_out_weight_partials",
            "pragnosia_aspin_prep_proj_partials", "pragnosia_aspin_chunk_wide_workspace_bytes",
            "pragnosia_layer_norm_partials", "pragnosia_wgrad_workspace_bytes"}

_lib = None


class PragnosiaError(RuntimeError):
    pass


def lib():
    """The loaded library, with argument and return types set. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise PragnosiaError(f"{LIB_PATH} is missing: build it with `python -m pragnosia_amd.build` "
                                 "(there is no CPU or PyTorch fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = (ctypes.c_char_p if name == "pragnosia_error_string" else
                          _i64 if name in _RET_I64 else _i32)
        _lib = L
    return _lib


def check(code: int, what: str) -> None:
    if code != 0:
        msg = lib().pragnosia_error_string(code).decode()
        raise PragnosiaError(f"{what} failed with code {code}: {msg}")
