"""Python front end of the DSV4 indexer block selection.

Mirrors the reference's Rust wrapper ``launch_dsv4_indexer_select``
(crates/hi-cuda/src/kernels.rs:3455-3481): the same argument meaning, the
same capacity checks (raised as ``ValueError`` where the wrapper bails),
and a ``HiRocmError`` for a non-zero status from the C ABI.  Everything
stays on the device: scores in, kept indices (ascending) and marks out.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib

_side_streams = {}


def launch_dsv4_indexer_select(scores: torch.Tensor, n_blocks: int, top_k: int,
                               marks: torch.Tensor, sel_out: torch.Tensor,
                               stream: Optional[torch.cuda.Stream] = None) -> None:
    """Write the min(top_k, n_blocks) kept block indices into ``sel_out``
    (int32, ascending) and 1/0 per block into ``marks`` (uint8)."""
    if n_blocks <= 0 or n_blocks > 2**31 - 1:
        raise ValueError("dsv4 indexer select blocks out of range")
    if n_blocks > 2**31 - 1 - 2**20:
        raise ValueError("dsv4 indexer select: n_blocks above 2^31 - 2^20 is not supported")
    if top_k <= 0 or top_k > 2**31 - 1:
        raise ValueError("dsv4 indexer select top_k out of range")
    if scores.dtype != torch.float32 or not scores.is_cuda or not scores.is_contiguous():
        raise ValueError("dsv4 indexer select scores: a contiguous f32 CUDA tensor")
    if scores.numel() < n_blocks:
        raise ValueError("dsv4 indexer select scores too small")
    if marks.dtype != torch.uint8 or not marks.is_cuda or marks.numel() < n_blocks:
        raise ValueError("dsv4 indexer select marks scratch too small")
    if sel_out.dtype != torch.int32 or not sel_out.is_cuda or sel_out.numel() < min(top_k, n_blocks):
        raise ValueError("dsv4 indexer select output too small")
    lib = _lib.load()
    side = None
    if stream is None or stream.cuda_stream == 0:
        cur = torch.cuda.current_stream()
        if cur.cuda_stream == 0:
            # the C ABI (like kernels.cu:2696) rejects the null stream: run on
            # a side stream ordered after the current one, then order the
            # current stream after the launch so its later reads see the
            # results, and keep the caching allocator from reusing the
            # tensors while the side stream still uses them
            dev = scores.device.index if scores.device.index is not None else torch.cuda.current_device()
            side = _side_streams.get(dev)
            if side is None:
                side = _side_streams[dev] = torch.cuda.Stream(device=dev)
            side.wait_stream(cur)
            stream = side
        else:
            stream = cur
    _lib.check(lib.hi_rocm_launch_dsv4_indexer_select(
        scores.data_ptr(), int(n_blocks), int(top_k), marks.data_ptr(), sel_out.data_ptr(),
        int(stream.cuda_stream)))
    if side is not None:
        torch.cuda.current_stream().wait_stream(side)
        for t in (scores, marks, sel_out):
            t.record_stream(side)


def dsv4_indexer_select(scores: torch.Tensor, top_k: int,
                        stream: Optional[torch.cuda.Stream] = None):
    """Allocating convenience form: returns (sel int32[take], marks uint8[n])."""
    n = scores.numel()
    marks = torch.empty(n, dtype=torch.uint8, device=scores.device)
    sel = torch.empty(max(1, min(top_k, n)), dtype=torch.int32, device=scores.device)
    launch_dsv4_indexer_select(scores, n, top_k, marks, sel, stream)
    return sel[:min(top_k, n)], marks
