"""ctypes binding of ``libhi_rocm.so`` (the hi-rocm C ABI, ``include/hi_rocm.h``).

Loading fails loudly when the library is missing: there is no CPU or
PyTorch fallback for any sampler entry point.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhi_rocm.so")

ROW_PARAMS_DTYPE = np.dtype(
    [
        ("temperature", "<f4"),
        ("top_p", "<f4"),
        ("min_p", "<f4"),
        ("repetition_penalty", "<f4"),
        ("frequency_penalty", "<f4"),
        ("presence_penalty", "<f4"),
        ("top_k", "<i4"),
        ("eos_id", "<u4"),
        ("flags", "<u4"),
        ("reserved", "<u4"),
    ]
)
assert ROW_PARAMS_DTYPE.itemsize == 40

OK, ERR_ARGS, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3
DTYPE_F32, DTYPE_BF16 = 0, 1
FLAG_REP_ONCE = 1
MAX_LOGPROBS = 1024

# Every function include/*.h declares, with its ctypes signature.
_vp, _i, _f, _i64, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_int64, ctypes.c_size_t
SIGNATURES = {
    # include/hi_rocm.h
    "hi_rocm_launch_argmax": (_i, [_vp, _vp, _i, _vp]),
    "hi_rocm_launch_dsv4_indexer_select": (_i, [_vp, _i, _i, _vp, _vp, _vp]),
    "hi_rocm_launch_argmax_last_row": (_i, [_vp, _vp, _i, _i, _vp]),
    "hi_rocm_launch_argmax_batched_last_token": (_i, [_vp, _vp, _i, _i, _i, _vp]),
    "hi_rocm_launch_sample_last_row": (_i, [_vp, _vp, _i, _i, _f, _f, _i, _f, _vp]),
    "hi_rocm_launch_sample_batched_last_token": (_i, [_vp, _vp, _vp, _i, _i, _i, _f, _f, _i, _i, _vp]),
    "hi_rocm_launch_select_batched_last_token_per_row": (
        _i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "hi_rocm_launch_select_batched_last_token_per_row_noalloc": (
        _i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "hi_rocm_sampler_reserve": (_i, [_i, _i, _i, _vp]),
    "hi_rocm_sampler_release": (_i, [_vp]),
    "hi_rocm_launch_moe_topk_router": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp]),
    "hi_rocm_lm_head_workspace_bytes": (_i, [_i, _i, ctypes.POINTER(_sz)]),
    "hi_rocm_lm_head_logits": (_i, [_vp, _vp, _vp, _f, _i, _i, _i, _vp, _vp]),
    "hi_rocm_sample_lm_head": (_i, [_vp, _vp, _vp, _f, _i, _i, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    "hi_rocm_sample_lm_head_ext": (_i, [_vp, _vp, _vp, _f, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                        _vp, _i, _vp, _sz, _vp]),
    "hi_rocm_spec_verify_greedy": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hi_rocm_history_append": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _i, _vp, _vp]),
    "hi_rocm_history_pack": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp]),
    "hi_rocm_rng_key_from_seed": (_i, [ctypes.c_uint64, _vp]),
    "hi_rocm_rng_uniforms": (_i, [_vp, _vp, _vp, _vp, _i, _vp]),
    "hi_rocm_decode_step_advance": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "hi_rocm_debug_chacha_block": (_i, [_vp, _vp, _i, _vp]),
    "hi_rocm_profile_begin": (_i, [_i]),
    "hi_rocm_profile_end": (_i, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                 ctypes.POINTER(_i)]),
    "hi_rocm_sampler_workspace_bytes": (_i, [_i, _i, _i, ctypes.POINTER(_sz)]),
    "hi_rocm_sample": (_i, [_vp, _i, _i, _i, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                            _vp, _i, _vp, _sz, _vp]),
    "hi_rocm_debug_distribution": (_i, [_vp, _i, _i, _i, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                        _vp]),
    "hi_rocm_debug_expf": (_i, [_vp, _vp, _i64, _vp]),
    "hi_rocm_debug_fold": (_i, [_vp, _vp, _i, ctypes.c_float, _vp, _vp, _vp]),
    "hi_rocm_debug_wide_paths": (_i, [_vp, _sz, _i, _i, _vp, _vp]),
    "hi_rocm_debug_wide_totals": (_i, [_vp, _sz, _i, _i, _vp, _vp]),
    "hi_rocm_last_error": (ctypes.c_char_p, []),
    "hi_rocm_version": (ctypes.c_char_p, []),
    # include/hi_rocm_host.h
    "hi_rocm_host_select_batched_last_token_per_row": (
        _i, [_vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _sz, _vp, ctypes.c_char_p, _sz,
             _vp]),
    "hi_rocm_host_sample_batched_last_token": (
        _i, [_vp, _sz, _sz, _sz, _sz, _f, _f, _i64, _vp, _sz, _vp, ctypes.c_char_p, _sz, _vp]),
    "hi_rocm_host_argmax_batched_last_token": (
        _i, [_vp, _sz, _sz, _sz, _sz, _vp, ctypes.c_char_p, _sz, _vp]),
    "hi_rocm_host_sample_last_row_with_sample": (
        _i, [_vp, _sz, _sz, _f, _f, _i64, _f, _vp, ctypes.c_char_p, _sz, _vp]),
}

_lib = None


class HiRocmError(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, status: int, message: str):
        super().__init__(f"hi-rocm status {status}: {message}")
        self.status = status


def load() -> ctypes.CDLL:
    """Load libhi_rocm.so (built by ``hi_amd._build.build()``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with hi_amd._build.build() "
                "(the sampler has no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status != OK:
        raise HiRocmError(status, load().hi_rocm_last_error().decode())
