"""ctypes front end of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg use
this module, and only as the checker.  The product path (``hi_amd``) never
imports it.  The C restatement it loads is ``oracle/sampler_oracle.c``; see
that file for the reference citations of each function.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

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

GREEDY, RANKED, TEMP_ONLY, EOS, FALLBACK = 0, 1, 2, 3, 4


class _Batch(ctypes.Structure):
    _fields_ = [
        ("logits", ctypes.c_void_p),
        ("dtype", ctypes.c_int),
        ("batch", ctypes.c_int64),
        ("vocab", ctypes.c_int64),
        ("row_stride", ctypes.c_int64),
        ("params", ctypes.c_void_p),
        ("uniforms", ctypes.c_void_p),
        ("hist_offsets", ctypes.c_void_p),
        ("hist_ids", ctypes.c_void_p),
        ("hist_counts", ctypes.c_void_p),
        ("mask_words", ctypes.c_void_p),
        ("n_logprobs", ctypes.c_int),
        ("out_tokens", ctypes.c_void_p),
        ("out_logprobs", ctypes.c_void_p),
        ("out_logprob_ids", ctypes.c_void_p),
        ("out_token_logprobs", ctypes.c_void_p),
        ("out_path", ctypes.c_void_p),
        ("out_cdf_margin", ctypes.c_void_p),
        ("out_cutoff_margin", ctypes.c_void_p),
        ("out_n_candidates", ctypes.c_void_p),
    ]


class _RankedInfo(ctypes.Structure):
    _fields_ = [
        ("path", ctypes.c_int32),
        ("n_candidates", ctypes.c_int64),
        ("total", ctypes.c_float),
        ("candidate_total", ctypes.c_float),
        ("max_scaled", ctypes.c_float),
        ("cdf_margin", ctypes.c_double),
        ("cutoff_margin", ctypes.c_double),
    ]


_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    # make rebuilds when sampler_oracle.c is newer than the library
    args = ["make", "-s"] + (["-B"] if force else []) + ["-C", _HERE]
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        f32p = ctypes.POINTER(ctypes.c_float)
        L.hro_argmax_total.restype = ctypes.c_int64
        L.hro_argmax_total.argtypes = [ctypes.c_void_p, ctypes.c_int64]
        L.hro_argmax_ieee.restype = ctypes.c_int64
        L.hro_argmax_ieee.argtypes = [ctypes.c_void_p, ctypes.c_int64]
        L.hro_argmax_finite_lane.restype = ctypes.c_int64
        L.hro_argmax_finite_lane.argtypes = [ctypes.c_void_p, ctypes.c_int64, f32p]
        L.hro_ranked_sample.restype = ctypes.c_int64
        L.hro_ranked_sample.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_float,
                                        ctypes.c_float, ctypes.c_int32, ctypes.c_float,
                                        ctypes.c_float, ctypes.POINTER(_RankedInfo)]
        L.hro_ranked_sample_brute.restype = ctypes.c_int64
        L.hro_ranked_sample_brute.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_float,
                                              ctypes.c_float, ctypes.c_int32, ctypes.c_float,
                                              ctypes.c_float]
        L.hro_temp_only_sample.restype = ctypes.c_int64
        L.hro_temp_only_sample.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_float,
                                           ctypes.c_float]
        L.hro_process_row.restype = ctypes.c_int
        L.hro_process_row.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                      ctypes.c_void_p, ctypes.c_void_p]
        L.hro_sample_rows.restype = ctypes.c_int
        L.hro_sample_rows.argtypes = [ctypes.POINTER(_Batch), ctypes.c_int]
        L.hro_expf_array.restype = None
        L.hro_expf_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.hro_indexer_select.restype = ctypes.c_int64
        L.hro_indexer_select.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                         ctypes.c_void_p, ctypes.c_void_p]
        L.hro_fold_f32.restype = ctypes.c_float
        L.hro_fold_f32.argtypes = [ctypes.c_void_p, ctypes.c_int64]
        L.hro_spec_verify_greedy.restype = None
        L.hro_spec_verify_greedy.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                             ctypes.c_void_p]
        L.hro_moe_router.restype = None
        L.hro_moe_router.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_float]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def argmax_total(x) -> int:
    x = _f32(x)
    return int(lib().hro_argmax_total(_ptr(x), x.size))


def argmax_ieee(x) -> int:
    x = _f32(x)
    return int(lib().hro_argmax_ieee(_ptr(x), x.size))


def argmax_finite_lane(x):
    x = _f32(x)
    m = ctypes.c_float()
    i = lib().hro_argmax_finite_lane(_ptr(x), x.size, ctypes.byref(m))
    return int(i), float(m.value)


def ranked_sample(logits, temperature, top_p, top_k=None, sample=0.0, min_p=0.0, info=False):
    """gpu.rs:753-900 (sample_host_ranked_logits_with_uniform); top_k None/0 = unset."""
    x = _f32(logits)
    inf = _RankedInfo()
    k = 0 if top_k is None else int(top_k)
    tok = int(lib().hro_ranked_sample(_ptr(x), x.size, float(temperature), float(top_p), k,
                                      float(min_p), float(sample), ctypes.byref(inf)))
    if info:
        return tok, {f: getattr(inf, f) for f, _ in _RankedInfo._fields_}
    return tok


def ranked_sample_brute(logits, temperature, top_p, top_k=None, sample=0.0, min_p=0.0) -> int:
    """gpu.rs:29505-29580 (reference_ranked_sample)."""
    x = _f32(logits)
    k = 0 if top_k is None else int(top_k)
    return int(lib().hro_ranked_sample_brute(_ptr(x), x.size, float(temperature),
                                             float(top_p), k, float(min_p), float(sample)))


def temp_only_sample(logits, temperature, sample) -> int:
    x = _f32(logits)
    return int(lib().hro_temp_only_sample(_ptr(x), x.size, float(temperature), float(sample)))


def expf(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().hro_expf_array(_ptr(x), _ptr(y), x.size)
    return y


def fold_f32(x) -> float:
    x = _f32(x)
    return float(np.float32(lib().hro_fold_f32(_ptr(x), x.size)))


def process_row(raw, params, hist_ids=None, hist_counts=None, mask_words=None):
    raw = _f32(raw)
    p = np.asarray(params, dtype=ROW_PARAMS_DTYPE).reshape(1)
    out = np.empty_like(raw)
    hi = None if hist_ids is None else np.ascontiguousarray(hist_ids, dtype=np.uint32)
    hc = None if hist_counts is None else np.ascontiguousarray(hist_counts, dtype=np.uint32)
    mw = None if mask_words is None else np.ascontiguousarray(mask_words, dtype=np.uint32)
    any_finite = lib().hro_process_row(_ptr(raw), raw.size, _ptr(p), _ptr(hi), _ptr(hc),
                                       0 if hi is None else hi.size, _ptr(mw), _ptr(out))
    return out, bool(any_finite)


def sample_rows(logits, params, uniforms, hist_offsets=None, hist_ids=None, hist_counts=None,
                mask_words=None, n_logprobs=0, threads=1, want_token_logprobs=False):
    """Whole-batch oracle mirroring ``hi_rocm_sample``.

    ``logits`` is [B, V] float32, or uint16 holding bf16 bits.  Returns a dict
    of numpy arrays: tokens, path, cdf_margin, cutoff_margin, n_candidates and,
    when requested, logprobs / logprob_ids / token_logprobs.
    """
    logits = np.ascontiguousarray(logits)
    if logits.dtype == np.uint16:
        dtype = 1
    else:
        logits = _f32(logits)
        dtype = 0
    B, V = logits.shape
    params = np.ascontiguousarray(params, dtype=ROW_PARAMS_DTYPE).reshape(B)
    uniforms = _f32(uniforms).reshape(B)
    out = {
        "tokens": np.zeros(B, np.uint32),
        "path": np.zeros(B, np.int32),
        "cdf_margin": np.zeros(B, np.float64),
        "cutoff_margin": np.zeros(B, np.float64),
        "n_candidates": np.zeros(B, np.int64),
    }
    keep = []
    b = _Batch()
    b.logits = _ptr(logits)
    b.dtype = dtype
    b.batch, b.vocab, b.row_stride = B, V, V
    b.params = _ptr(params)
    b.uniforms = _ptr(uniforms)
    if hist_offsets is not None:
        ho = np.ascontiguousarray(hist_offsets, dtype=np.uint32)
        hi = np.ascontiguousarray(hist_ids, dtype=np.uint32)
        hc = np.ascontiguousarray(hist_counts, dtype=np.uint32)
        keep += [ho, hi, hc]
        b.hist_offsets, b.hist_ids, b.hist_counts = _ptr(ho), _ptr(hi), _ptr(hc)
    if mask_words is not None:
        mw = np.ascontiguousarray(mask_words, dtype=np.uint32)
        keep.append(mw)
        b.mask_words = _ptr(mw)
    b.n_logprobs = int(n_logprobs)
    b.out_tokens = _ptr(out["tokens"])
    if n_logprobs > 0:
        out["logprobs"] = np.zeros((B, n_logprobs), np.float32)
        out["logprob_ids"] = np.zeros((B, n_logprobs), np.uint32)
        b.out_logprobs = _ptr(out["logprobs"])
        b.out_logprob_ids = _ptr(out["logprob_ids"])
    if n_logprobs > 0 or want_token_logprobs:
        out["token_logprobs"] = np.zeros(B, np.float32)
        b.out_token_logprobs = _ptr(out["token_logprobs"])
    b.out_path = _ptr(out["path"])
    b.out_cdf_margin = _ptr(out["cdf_margin"])
    b.out_cutoff_margin = _ptr(out["cutoff_margin"])
    b.out_n_candidates = _ptr(out["n_candidates"])
    rc = lib().hro_sample_rows(ctypes.byref(b), int(threads))
    if rc != 0:
        raise ValueError(f"oracle rejected the batch (status {rc})")
    return out


def indexer_select(scores, top_k):
    """DSV4 indexer block selection (dsv4_cpu.rs:3258-3270): the kept block
    indices, ascending, and the uint8 marks."""
    x = _f32(scores)
    n = x.size
    marks = np.zeros(n, dtype=np.uint8)
    sel = np.zeros(max(1, min(int(top_k), n)), dtype=np.int32)
    took = lib().hro_indexer_select(_ptr(x), n, int(top_k), _ptr(marks), _ptr(sel))
    if took < 0:
        raise ValueError("indexer_select: n and top_k must be positive")
    return sel[:took], marks


def moe_router(scores, top_k, bias=None, norm_topk=False, gating_sigmoid=False, weights_scale=1.0):
    """MoE router top-k (kernels.cu:536-684, glibc expf): ids u32 and weights
    f32, each [rows, top_k]."""
    x = np.ascontiguousarray(scores, dtype=np.float32)
    rows, experts = x.shape
    ids = np.zeros((rows, top_k), np.uint32)
    w = np.zeros((rows, top_k), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().hro_moe_router(_ptr(x), _ptr(ids), _ptr(w), _ptr(b), rows, experts, int(top_k), int(bool(norm_topk)),
                         int(bool(gating_sigmoid)), float(weights_scale))
    return ids, w


def spec_verify_greedy(logits, draft, draft_len=None):
    """Greedy speculative verification (gpu.rs:10725-10762): logits
    [B, K+1, V] f32, draft [B, K] u32.  Returns (greedy [B, K+1],
    tokens [B, K+1] (valid up to count), count [B])."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    B, K1, V = x.shape
    K = K1 - 1
    d = np.ascontiguousarray(draft, dtype=np.uint32).reshape(B, K) if K > 0 else np.zeros((B, 1), np.uint32)
    dl = None if draft_len is None else np.ascontiguousarray(draft_len, dtype=np.int32)
    g = np.zeros((B, K1), np.uint32)
    t = np.zeros((B, K1), np.uint32)
    c = np.zeros(B, np.int32)
    lib().hro_spec_verify_greedy(_ptr(x), B, K, V, _ptr(d), _ptr(dl), _ptr(g), _ptr(t), _ptr(c))
    return g, t, c
