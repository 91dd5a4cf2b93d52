"""ctypes binding of libloractl_rocm.so (the C ABI in include/loractl_rocm.h).

Loading never falls back to anything: if the library is missing or does not
export a declared symbol, the import of the compute path fails loudly.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libloractl_rocm.so")

LRQ_OK = 0
LRQ_EINVAL = -1
LRQ_EUNSUPPORTED = -2
LRQ_EHIP = -3
LRQ_ENOMEM = -4
LRQ_FMT_INT4 = 1
LRQ_FMT_FP8 = 2
LRQ_FMT_INT8 = 3
LRQ_LAYOUT_ROWS = 0
LRQ_LAYOUT_BLOCKED = 1
LRQ_MAX_LORA_TOKENS = 259456  # include/loractl_rocm.h: tokens per LoRA call (m > 16)
LRQ_NOALLOC_SCRATCH_BYTES = 32 << 20

_ERRNAMES = {
    LRQ_EINVAL: "LRQ_EINVAL",
    LRQ_EUNSUPPORTED: "LRQ_EUNSUPPORTED",
    LRQ_EHIP: "LRQ_EHIP",
    LRQ_ENOMEM: "LRQ_ENOMEM",
}


class LrqWeight(ctypes.Structure):
    """Mirror of ``struct lrq_weight``."""

    _fields_ = [
        ("format", ctypes.c_int32),
        ("group", ctypes.c_int32),
        ("n", ctypes.c_int64),
        ("k", ctypes.c_int64),
        ("data", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("per_channel", ctypes.c_int32),
        ("layout", ctypes.c_int32),
        ("bias", ctypes.c_void_p),
    ]


class LrqError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{_ERRNAMES.get(code, code)}: {msg}")
        self.code = code


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_wp = ctypes.POINTER(LrqWeight)

# name -> (restype, argtypes); exactly the declarations of include/loractl_rocm.h
SIGNATURES = {
    "lrq_version": (_i32, []),
    "lrq_create": (_i32, [_i32, ctypes.POINTER(_vp)]),
    "lrq_destroy": (_i32, [_vp]),
    "lrq_set_stream": (_i32, [_vp, _vp]),
    "lrq_sync": (_i32, [_vp]),
    "lrq_last_error": (ctypes.c_char_p, [_vp]),
    "lrq_reserve": (_i32, [_vp, _i64, _i64, _i64, _i64]),
    "lrq_quantize_int4": (_i32, [_vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "lrq_quantize_int8": (_i32, [_vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "lrq_quantize_fp8": (_i32, [_vp, _vp, _i64, _i64, _i32, _vp, _vp]),
    "lrq_requantize_fp8_int4": (_i32, [_vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp, _vp]),
    "lrq_weight_blocked_size": (_i32, [_i32, _i64, _i64, _i64, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "lrq_weight_block": (_i32, [_vp, _wp, _vp, _vp]),
    "lrq_dequant": (_i32, [_vp, _wp, _vp]),
    "lrq_dequant_bf16": (_i32, [_vp, _wp, _vp]),
    "lrq_quant_matmul_t": (_i32, [_vp, _wp, _vp, _i64, _vp]),
    "lrq_quant_matmul_t_bwd": (_i32, [_vp, _wp, _vp, _i64, _vp]),
    "lrq_lora_fwd": (_i32, [_vp, _wp, _vp, _i64, _vp, _vp, _i64, _f32, _vp, _vp]),
    "lrq_lora_fwd_noalloc": (_i32, [_vp, _wp, _vp, _i64, _vp, _vp, _i64, _f32, _vp, _vp]),
    "lrq_lora_bwd": (_i32, [_vp, _wp, _vp, _vp, _i64, _vp, _vp, _i64, _f32, _vp, _vp, _vp, _vp]),
    "lrq_profile_enable": (_i32, [_vp, _i32]),
    "lrq_profile_reset": (_i32, [_vp]),
    "lrq_profile_count": (_i32, []),
    "lrq_profile_name": (ctypes.c_char_p, [_i32]),
    "lrq_profile_read": (_i32, [_vp, _i32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i64)]),
    "lrq_profile_relaunch": (_i32, [_vp, _i32, _i32]),
    "lrq_probe_stream_read": (_i32, [_vp, _vp, _i64]),
    "lrq_debug_force_wait_timeout": (_i32, [_i32]),
    "lrq_debug_gemm_path": (_i32, [_i32]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libloractl_rocm.so and bind every C-ABI entry point."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(there is no CPU fallback for the ROCm compute path)"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the symbol is missing
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
