"""ctypes binding of lib/libktmi.so (the C ABI declared in include/ktmi.h).

The library is loaded once per process; a missing library raises at import of the
first op (there is no CPU fallback). Every wrapper raises RuntimeError with
ktmi_last_error()'s text when a call returns a negative status.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("KTMI_LIB", Path(__file__).resolve().parent / "lib" / "libktmi.so"))

KTMI_OK = 0
KTMI_F32, KTMI_F16, KTMI_BF16 = 0, 1, 2
MODE_AUTO, MODE_GEMV, MODE_GROUPED, MODE_DECODE = 0, 1, 2, 3
STAGE_EVENTS = 6
NOALLOC_SCRATCH_BYTES = 64 << 20  # KTMI_NOALLOC_SCRATCH_BYTES

_i64, _i32, _vp = C.c_int64, C.c_int, C.c_void_p


class ktmi_layer(C.Structure):
    _fields_ = [
        ("hidden", C.c_int64),
        ("inter", C.c_int64),
        ("n_slots", C.c_int64),
        ("type13", C.c_int32),
        ("type2", C.c_int32),
        ("w13", C.c_void_p),
        ("w2", C.c_void_p),
        ("w_is_table", C.c_int32),
        ("reserved", C.c_int32),
    ]


class ktmi_bank(C.Structure):
    _fields_ = [
        ("gate", C.c_void_p),
        ("up", C.c_void_p),
        ("down", C.c_void_p),
        ("part_gate", C.c_int64),
        ("part_up", C.c_int64),
        ("part_down", C.c_int64),
        ("n_experts", C.c_int64),
    ]


# name -> (restype, argtypes); every symbol declared in include/ktmi.h
SIGNATURES = {
    "ktmi_last_error": (C.c_char_p, []),
    "ktmi_version": (_i32, []),
    "ktmi_type_supported": (_i32, [_i32]),
    "ktmi_row_bytes": (_i64, [_i64, _i32]),
    "ktmi_q8_1_row_bytes": (_i64, [_i64]),
    "ktmi_quantize_q8_1": (_i32, [_vp, _i32, _i64, _i64, _vp, _vp]),
    "ktmi_moe_a8_vec_workspace": (_i64, [_i64, _i64]),
    "ktmi_moe_a8_vec": (_i32, [_vp, _i32, _i64, _vp, _i32, _vp, _i64, _i32, _i64, _i64, _i32, _vp, _vp, _i64, _vp]),
    "ktmi_dequant_experts": (_i32, [_vp, _i64, _i32, _i64, _i64, _i64, _vp, _i64, _vp]),
    "ktmi_hot_route": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ktmi_silu_and_mul": (_i32, [_vp, _i32, _i64, _i64, _vp, _vp]),
    "ktmi_combine": (_i32, [_vp, _i32, _vp, _i64, _i64, _i64, _vp, _vp]),
    "ktmi_moe_layer_workspace": (_i64, [C.POINTER(ktmi_layer), _i64, _i64, _i32]),
    "ktmi_moe_layer": (_i32, [C.POINTER(ktmi_layer), _vp, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _i32, _vp]),
    "ktmi_moe_layer_mode": (_i32, [C.POINTER(ktmi_layer), _i64, _i64]),
    "ktmi_moe_layer_pass_tokens": (_i64, [C.POINTER(ktmi_layer), _i64]),
    "ktmi_moe_layer_noalloc": (_i32, [C.POINTER(ktmi_layer), _vp, _vp, _vp, _i64, _i64, _vp, _i32, _vp]),
    "ktmi_set_stage_events": (_i32, [C.POINTER(C.c_void_p), _i32]),
    "ktmi_quantize_rows_host": (_i32, [_vp, _i64, _i64, _i32, _vp, _i32]),
    "ktmi_streamer_create": (_vp, [_i64, _i64, _i64, _i32]),
    "ktmi_streamer_destroy": (_i32, [_vp]),
    "ktmi_streamer_slot": (_i32, [_vp, _i32, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)]),
    "ktmi_streamer_stage": (_i32, [_vp, _i32, C.POINTER(ktmi_bank), _i64, _i64]),
    "ktmi_streamer_acquire": (_i32, [_vp, _i32, _vp]),
    "ktmi_streamer_release": (_i32, [_vp, _i32, _vp]),
    "ktmi_streamer_sync": (_i32, [_vp]),
    "ktmi_streamer_copy_stream": (_vp, [_vp]),
    "ktmi_remap_ids": (_i32, [_vp, _i64, _i32, _i32, _vp, _vp]),
    "ktmi_add_bf16": (_i32, [_vp, _vp, _i64, _vp]),
    "ktmi_host_alloc": (_vp, [_i64]),
    "ktmi_host_free": (_i32, [_vp]),
    "ktmi_cpu_moe_create": (_vp, [_i64, _i64, _i32, _i32, C.POINTER(ktmi_bank), _i32, _i64, _i64]),
    "ktmi_cpu_moe_destroy": (_i32, [_vp]),
    "ktmi_cpu_moe_forward": (_i32, [_vp, _i64, _i64, _vp, _vp, _vp, _vp]),
    "ktmi_cpu_moe_submit": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "ktmi_cpu_moe_sync_add": (_i32, [_vp, _vp, _vp]),
    "ktmi_cpu_moe_threads": (_i32, [_vp]),
    "ktmi_cpu_moe_isa": (C.c_char_p, [_vp]),
    "ktmi_cpu_moe_set_add_wait": (_i32, [_vp, _i64]),
}

_lib = None


def lib():
    """The loaded library; raises if it was not built (there is no fallback)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"ktmi: {LIB_PATH} is missing; build it with kt-prefill-lend_amd/build.py")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str = "ktmi") -> None:
    if rc != KTMI_OK:
        msg = lib().ktmi_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def ptr(t) -> int:
    """Device (or host) address of a tensor's first element."""
    return t.data_ptr() if t is not None else 0


def stream_ptr(device=None) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype) -> int:
    import torch

    if dtype == torch.bfloat16:
        return KTMI_BF16
    if dtype == torch.float16:
        return KTMI_F16
    if dtype == torch.float32:
        return KTMI_F32
    raise TypeError(f"ktmi: unsupported activation dtype {dtype}")
