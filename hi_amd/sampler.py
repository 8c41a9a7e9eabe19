"""Python front end of the hi-rocm sampler.

Two layers, both over the C ABI in ``libhi_rocm.so``:

* the reference's per-step Rust API (crates/hi-cuda/src/gpu.rs:15542-15967)
  through its C++ mirror: ``RowSampling``, ``argmax_batched_last_token``,
  ``sample_batched_last_token``, ``select_batched_last_token_per_row``,
  ``sample_last_row_with_sample`` (host parameter lists, device logits,
  blocking like the Rust functions);
* the extended decode-step pipeline ``Sampler.sample`` (penalties, mask,
  min-p, logprobs, bf16), asynchronous on a stream, no allocation per call.

PyTorch only provides device memory and streams here.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import ROW_PARAMS_DTYPE, HiRocmError, check, load


class SamplerError(RuntimeError):
    """Error raised by the host layer (the Rust functions' ``bail!``)."""


@dataclass(frozen=True)
class RowSampling:
    """CudaRowSampling (gpu.rs:55-65): ``greedy`` or a sampled config."""

    greedy: bool
    temperature: float = 0.0
    top_p: float = 1.0
    top_k: Optional[int] = None

    @staticmethod
    def Greedy() -> "RowSampling":  # noqa: N802 - mirrors the Rust variant name
        return RowSampling(True)

    @staticmethod
    def Sampled(temperature: float, top_p: float, top_k: Optional[int] = None) -> "RowSampling":  # noqa: N802
        return RowSampling(False, float(temperature), float(top_p), top_k)


_host_streams = {}


def _stream_ptr(stream: Optional[torch.cuda.Stream]) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _host_stream(stream: Optional[torch.cuda.Stream]) -> int:
    """A non-null stream for the reference-mirror layer, which (like the
    reference's launchers) rejects the null stream.  When the caller gives
    none, a per-device stream ordered after the current stream is used."""
    if stream is not None and stream.cuda_stream != 0:
        return int(stream.cuda_stream)
    cur = torch.cuda.current_stream()
    if cur.cuda_stream != 0:
        return int(cur.cuda_stream)
    dev = torch.cuda.current_device()
    if dev not in _host_streams:
        _host_streams[dev] = torch.cuda.Stream(device=dev)
    hs = _host_streams[dev]
    hs.wait_stream(cur)
    return int(hs.cuda_stream)


def _check_logits(logits: torch.Tensor) -> None:
    if not logits.is_cuda or logits.dtype != torch.float32 or logits.dim() != 2 or not logits.is_contiguous():
        raise ValueError("logits must be a contiguous 2-D float32 CUDA tensor")


def _err_buf():
    return ctypes.create_string_buffer(512)


def argmax_batched_last_token(logits: torch.Tensor, batch_count: int, seq_len: int,
                              stream: Optional[torch.cuda.Stream] = None) -> list:
    _check_logits(logits)
    out = np.zeros(batch_count, np.uint32)
    err = _err_buf()
    rc = load().hi_rocm_host_argmax_batched_last_token(
        logits.data_ptr(), logits.shape[0], logits.shape[1], batch_count, seq_len,
        out.ctypes.data, err, len(err), _host_stream(stream))
    if rc != 0:
        raise SamplerError(err.value.decode())
    return out.tolist()


def sample_batched_last_token(logits: torch.Tensor, batch_count: int, seq_len: int,
                              temperature: float, top_p: float, top_k: Optional[int],
                              samples: Sequence[float],
                              stream: Optional[torch.cuda.Stream] = None) -> list:
    _check_logits(logits)
    sm = np.ascontiguousarray(samples, np.float32)
    out = np.zeros(batch_count, np.uint32)
    err = _err_buf()
    rc = load().hi_rocm_host_sample_batched_last_token(
        logits.data_ptr(), logits.shape[0], logits.shape[1], batch_count, seq_len,
        float(temperature), float(top_p), -1 if top_k is None else int(top_k),
        sm.ctypes.data, sm.size, out.ctypes.data, err, len(err), _host_stream(stream))
    if rc != 0:
        raise SamplerError(err.value.decode())
    return out.tolist()


def select_batched_last_token_per_row(logits: torch.Tensor, batch_count: int, seq_len: int,
                                      row_sampling: Sequence[RowSampling],
                                      samples: Sequence[float],
                                      stream: Optional[torch.cuda.Stream] = None) -> list:
    _check_logits(logits)
    n = len(row_sampling)
    kinds = np.array([0 if r.greedy else 1 for r in row_sampling] or [0], np.int32)
    temps = np.array([r.temperature for r in row_sampling] or [0], np.float32)
    tps = np.array([r.top_p for r in row_sampling] or [1], np.float32)
    tks = np.array([-1 if r.top_k is None else int(r.top_k) for r in row_sampling] or [-1], np.int64)
    sm = np.ascontiguousarray(list(samples) or [0.0], np.float32)
    out = np.zeros(max(batch_count, 1), np.uint32)
    err = _err_buf()
    rc = load().hi_rocm_host_select_batched_last_token_per_row(
        logits.data_ptr(), logits.shape[0], logits.shape[1], batch_count, seq_len, n,
        kinds.ctypes.data, temps.ctypes.data, tps.ctypes.data, tks.ctypes.data,
        sm.ctypes.data, len(samples), out.ctypes.data, err, len(err), _host_stream(stream))
    if rc != 0:
        raise SamplerError(err.value.decode())
    return out[:batch_count].tolist()


def sample_last_row_with_sample(logits: torch.Tensor, temperature: float, top_p: float,
                                top_k: Optional[int], sample: float,
                                stream: Optional[torch.cuda.Stream] = None) -> int:
    _check_logits(logits)
    out = np.zeros(1, np.uint32)
    err = _err_buf()
    rc = load().hi_rocm_host_sample_last_row_with_sample(
        logits.data_ptr(), logits.shape[0], logits.shape[1], float(temperature), float(top_p),
        -1 if top_k is None else int(top_k), float(sample), out.ctypes.data, err, len(err),
        _host_stream(stream))
    if rc != 0:
        raise SamplerError(err.value.decode())
    return int(out[0])


def row_params(batch: int, temperature=0.0, top_p=1.0, top_k=0, min_p=0.0,
               repetition_penalty=1.0, frequency_penalty=0.0, presence_penalty=0.0,
               eos_id=0, flags=0) -> np.ndarray:
    """Structured array of ``hi_rocm_row_params``; scalars broadcast over rows."""
    p = np.zeros(batch, ROW_PARAMS_DTYPE)
    p["temperature"] = temperature
    p["top_p"] = top_p
    p["top_k"] = top_k
    p["min_p"] = min_p
    p["repetition_penalty"] = repetition_penalty
    p["frequency_penalty"] = frequency_penalty
    p["presence_penalty"] = presence_penalty
    p["eos_id"] = eos_id
    p["flags"] = flags
    return p


def sampler_release(stream: Optional[torch.cuda.Stream] = None) -> None:
    """Free the library workspace of ``stream`` on the current device
    (``hi_rocm_sampler_release``); the mirrors allocate it again on demand."""
    s = stream if stream is not None else torch.cuda.current_stream()
    check(load().hi_rocm_sampler_release(int(s.cuda_stream)))


def params_to_device(params: np.ndarray, device="cuda") -> torch.Tensor:
    raw = np.ascontiguousarray(params, ROW_PARAMS_DTYPE).view(np.uint8)
    return torch.from_numpy(raw.copy()).to(device)


class Sampler:
    """The extended decode-step sampler (``hi_rocm_sample``) with its own workspace.

    The workspace is allocated once, for up to ``max_batch`` rows of ``vocab``
    logits; ``sample`` allocates nothing and only enqueues kernels.
    """

    def __init__(self, max_batch: int, vocab: int, n_logprobs: int = 0, device="cuda"):
        lib = load()
        nbytes = ctypes.c_size_t()
        check(lib.hi_rocm_sampler_workspace_bytes(max_batch, vocab, n_logprobs, ctypes.byref(nbytes)))
        self.max_batch, self.vocab, self.n_logprobs = max_batch, vocab, n_logprobs
        self.workspace = torch.zeros(nbytes.value, dtype=torch.uint8, device=device)

    def sample(self, logits: torch.Tensor, params: torch.Tensor, uniforms: torch.Tensor,
               hist_offsets: Optional[torch.Tensor] = None, hist_ids: Optional[torch.Tensor] = None,
               hist_counts: Optional[torch.Tensor] = None, mask_words: Optional[torch.Tensor] = None,
               n_logprobs: int = 0, token_logprobs: bool = False,
               out: Optional[dict] = None, stream: Optional[torch.cuda.Stream] = None) -> dict:
        """Enqueue one sampling step; returns device tensors (tokens, logprobs ...)."""
        if logits.dim() != 2:
            raise ValueError("logits must be [batch, vocab]")
        B, V = logits.shape
        if logits.dtype == torch.float32:
            dtype = _lib.DTYPE_F32
        elif logits.dtype == torch.bfloat16:
            dtype = _lib.DTYPE_BF16
        else:
            raise ValueError("logits must be float32 or bfloat16")
        if B > self.max_batch or V > self.vocab or n_logprobs > self.n_logprobs:
            raise ValueError("shape exceeds the workspace this Sampler was built for")
        dev = logits.device
        if out is None:
            out = {"tokens": torch.empty(B, dtype=torch.int32, device=dev)}
            if n_logprobs > 0:
                out["logprobs"] = torch.empty(B, n_logprobs, dtype=torch.float32, device=dev)
                out["logprob_ids"] = torch.empty(B, n_logprobs, dtype=torch.int32, device=dev)
            if token_logprobs:
                out["token_logprobs"] = torch.empty(B, dtype=torch.float32, device=dev)

        def p(t):
            return 0 if t is None else t.data_ptr()

        status = load().hi_rocm_sample(
            logits.data_ptr(), dtype, B, V, logits.stride(0), params.data_ptr(), uniforms.data_ptr(),
            p(hist_offsets), p(hist_ids), p(hist_counts), p(mask_words),
            out["tokens"].data_ptr(), p(out.get("logprobs")), p(out.get("logprob_ids")),
            p(out.get("token_logprobs")), n_logprobs, self.workspace.data_ptr(),
            self.workspace.numel(), _stream_ptr(stream))
        check(status)
        return out


WIDE_PATHS = {0: "other", 1: "wide", 2: "no-stats", 3: "chunk-full", 4: "total", 5: "merge-full",
              6: "no-cutoff", 7: "draw-fail", 8: "row-minp", 9: "row-lists", 10: "row-general"}


def debug_wide_paths(smp: "Sampler", batch: int, vocab: int,
                     stream: Optional[torch.cuda.Stream] = None) -> np.ndarray:
    """How the last ``smp.sample`` call finished each row: top-p rows on the
    chunked path, every row of the row kernel (``hi_rocm_debug_wide_paths``;
    codes in WIDE_PATHS)."""
    out = np.zeros(batch, np.uint32)
    check(load().hi_rocm_debug_wide_paths(smp.workspace.data_ptr(), smp.workspace.numel(), batch, vocab,
                                          out.ctypes.data, _stream_ptr(stream)))
    return out & 0xff


def debug_wide_totals(smp: "Sampler", batch: int, vocab: int,
                      stream: Optional[torch.cuda.Stream] = None) -> np.ndarray:
    """The wide pass's normaliser and candidate total of each top-p row it
    finished in the last ``smp.sample`` call (float32[batch][2];
    ``hi_rocm_debug_wide_totals``; other rows hold stale values)."""
    out = np.zeros((batch, 2), np.float32)
    check(load().hi_rocm_debug_wide_totals(smp.workspace.data_ptr(), smp.workspace.numel(), batch, vocab,
                                           out.ctypes.data, _stream_ptr(stream)))
    return out


MINP_MISSES = {0: "none", 1: "array", 2: "top-k", 3: "draw"}


def debug_row_minp_misses(smp: "Sampler", batch: int, vocab: int,
                          stream: Optional[torch.cuda.Stream] = None) -> np.ndarray:
    """Why the row kernel's min-p finish left each row to the candidate lists'
    finish in the last ``smp.sample`` call (codes in MINP_MISSES)."""
    out = np.zeros(batch, np.uint32)
    check(load().hi_rocm_debug_wide_paths(smp.workspace.data_ptr(), smp.workspace.numel(), batch, vocab,
                                          out.ctypes.data, _stream_ptr(stream)))
    return out >> 8


def debug_distribution(logits: torch.Tensor, params: torch.Tensor,
                       hist_offsets=None, hist_ids=None, hist_counts=None, mask_words=None,
                       stream: Optional[torch.cuda.Stream] = None):
    """Processed logits and full-vocabulary probabilities (``hi_rocm_debug_distribution``)."""
    B, V = logits.shape
    dtype = _lib.DTYPE_BF16 if logits.dtype == torch.bfloat16 else _lib.DTYPE_F32
    proc = torch.empty(B, V, dtype=torch.float32, device=logits.device)
    probs = torch.empty(B, V, dtype=torch.float32, device=logits.device)

    def p(t):
        return 0 if t is None else t.data_ptr()

    check(load().hi_rocm_debug_distribution(
        logits.data_ptr(), dtype, B, V, logits.stride(0), params.data_ptr(), p(hist_offsets),
        p(hist_ids), p(hist_counts), p(mask_words), proc.data_ptr(), probs.data_ptr(),
        _stream_ptr(stream)))
    return proc, probs


def debug_expf(x: torch.Tensor, stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    y = torch.empty_like(x)
    check(load().hi_rocm_debug_expf(x.data_ptr(), y.data_ptr(), x.numel(), _stream_ptr(stream)))
    return y


__all__ = [
    "RowSampling", "SamplerError", "HiRocmError", "Sampler", "row_params", "params_to_device",
    "argmax_batched_last_token", "sample_batched_last_token", "select_batched_last_token_per_row",
    "sample_last_row_with_sample", "debug_distribution", "debug_expf", "debug_wide_paths",
    "debug_row_minp_misses", "sampler_release",
]
