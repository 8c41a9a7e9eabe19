"""CPU checks of the C ABI: the library loads, exports every function the
public headers declare, and rejects bad arguments before touching a GPU."""
import ctypes
import os
import re

import numpy as np

from hi_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("hi_rocm.h", "hi_rocm_host.h")]


def declared_functions():
    names = []
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(hi_rocm_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_every_declared_symbol_is_exported():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 17
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_version_and_row_params_layout():
    lib = _lib.load()
    assert b"gfx950" in lib.hi_rocm_version()
    assert _lib.ROW_PARAMS_DTYPE.itemsize == 40
    from oracle.oracle import ROW_PARAMS_DTYPE as ORACLE_DT
    assert ORACLE_DT == _lib.ROW_PARAMS_DTYPE


def test_workspace_bytes():
    lib = _lib.load()
    out = ctypes.c_size_t()
    assert lib.hi_rocm_sampler_workspace_bytes(256, 129280, 0, ctypes.byref(out)) == 0
    b256 = out.value
    assert lib.hi_rocm_sampler_workspace_bytes(1, 129280, 0, ctypes.byref(out)) == 0
    assert 0 < out.value < b256
    assert lib.hi_rocm_sampler_workspace_bytes(0, 10, 0, ctypes.byref(out)) == _lib.ERR_ARGS
    assert lib.hi_rocm_sampler_workspace_bytes(1, 10, 5000, ctypes.byref(out)) == _lib.ERR_UNSUPPORTED
    assert lib.hi_rocm_sampler_workspace_bytes(1, 1 << 30, 0, ctypes.byref(out)) == _lib.ERR_UNSUPPORTED


def test_launchers_reject_bad_arguments_without_a_gpu():
    """kernels.cu:14737-14880 argument checks (status 1), run before any HIP call."""
    lib = _lib.load()
    p = ctypes.c_void_p(0x1000)
    s = ctypes.c_void_p(0x2000)
    assert lib.hi_rocm_launch_argmax(None, p, 8, s) == 1
    assert lib.hi_rocm_launch_argmax(p, p, 0, s) == 1
    assert lib.hi_rocm_launch_argmax(p, p, 8, None) == 1
    assert lib.hi_rocm_launch_argmax_last_row(p, p, 0, 8, s) == 1
    assert lib.hi_rocm_launch_argmax_batched_last_token(p, p, 2, 0, 8, s) == 1
    assert lib.hi_rocm_launch_sample_last_row(p, p, 1, 8, 1.0, 0.9, -1, 0.5, s) == 1
    assert lib.hi_rocm_launch_sample_batched_last_token(p, p, None, 1, 1, 8, 1.0, 0.9, 4, 0, s) == 1
    assert lib.hi_rocm_launch_select_batched_last_token_per_row(p, p, p, p, p, None, 1, 1, 8, 0, s) == 1
    assert b"invalid" in lib.hi_rocm_last_error()
    # kernels.cu:2698-2701: null pointers, n_blocks <= 0, top_k <= 0, null stream
    assert lib.hi_rocm_launch_dsv4_indexer_select(None, 8, 2, p, p, s) == 1
    assert lib.hi_rocm_launch_dsv4_indexer_select(p, 8, 2, None, p, s) == 1
    assert lib.hi_rocm_launch_dsv4_indexer_select(p, 8, 2, p, None, s) == 1
    assert lib.hi_rocm_launch_dsv4_indexer_select(p, 0, 2, p, p, s) == 1
    assert lib.hi_rocm_launch_dsv4_indexer_select(p, 8, 0, p, p, s) == 1
    assert lib.hi_rocm_launch_dsv4_indexer_select(p, 8, 2, p, p, None) == 1
    # hi_rocm_sample: bad dtype, stride below vocab, history without counts
    params = np.zeros(40, np.uint8)
    assert lib.hi_rocm_sample(p, 7, 1, 8, 8, params.ctypes.data, p, None, None, None, None, p,
                              None, None, None, 0, p, 1 << 30, s) == 1
    assert lib.hi_rocm_sample(p, 0, 1, 8, 4, params.ctypes.data, p, None, None, None, None, p,
                              None, None, None, 0, p, 1 << 30, s) == 1
    assert lib.hi_rocm_sample(p, 0, 1, 8, 8, params.ctypes.data, p, p, p, None, None, p,
                              None, None, None, 0, p, 1 << 30, s) == 1
    # workspace too small
    assert lib.hi_rocm_sample(p, 0, 1, 8, 8, params.ctypes.data, p, None, None, None, None, p,
                              None, None, None, 0, p, 16, s) == 1
    # logprobs requested without outputs
    assert lib.hi_rocm_sample(p, 0, 1, 8, 8, params.ctypes.data, p, None, None, None, None, p,
                              None, None, None, 4, p, 1 << 30, s) == 1
