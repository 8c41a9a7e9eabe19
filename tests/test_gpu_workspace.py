"""The library-owned workspace of the reference-shaped launchers: growth is
refused (status 2, nothing enqueued) while the stream is being captured,
a reserve before capture makes the same call capturable, and
hi_rocm_sampler_release gives a stream's buffer back."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32 = np.float32


def _per_row_inputs(torch, B, V, seed):
    rng = np.random.default_rng(seed)
    logits = torch.from_numpy(rng.normal(0, 3, (B, V)).astype(F32)).cuda()
    temps = torch.full((B,), 0.8, dtype=torch.float32, device="cuda")
    top_ps = torch.full((B,), 0.9, dtype=torch.float32, device="cuda")
    top_ks = torch.full((B,), 40, dtype=torch.int32, device="cuda")
    samples = torch.from_numpy(rng.random(B).astype(F32)).cuda()
    out = torch.zeros(B, dtype=torch.int32, device="cuda")
    return logits, temps, top_ps, top_ks, samples, out


def _launch(lib, args, B, V, stream):
    logits, temps, top_ps, top_ks, samples, out = args
    return lib.hi_rocm_launch_select_batched_last_token_per_row(
        logits.data_ptr(), out.data_ptr(), samples.data_ptr(), temps.data_ptr(), top_ps.data_ptr(),
        top_ks.data_ptr(), B, 1, V, 1, int(stream.cuda_stream))


def test_growth_under_capture_is_refused(hip):
    import torch
    from hi_amd import _lib
    lib = _lib.load()
    B, V = 8, 151936
    args = _per_row_inputs(torch, B, V, 5)
    stream = torch.cuda.Stream()  # a fresh stream: no workspace yet
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    rc = None
    with torch.cuda.graph(g, stream=stream):
        rc = _launch(lib, args, B, V, stream)
    torch.cuda.synchronize()
    assert rc == _lib.ERR_UNSUPPORTED, rc
    assert b"hi_rocm_sampler_reserve" in lib.hi_rocm_last_error()
    # nothing was enqueued: the captured graph replays without touching out
    args[5].fill_(-7)
    g.replay()
    torch.cuda.synchronize()
    assert (args[5] == -7).all()
    # reserved first, the same call captures and replays like the eager call
    _lib.check(lib.hi_rocm_sampler_reserve(B, V, 0, ctypes.c_void_p(int(stream.cuda_stream))))
    with torch.cuda.stream(stream):
        _lib.check(_launch(lib, args, B, V, stream))
    torch.cuda.synchronize()
    eager = args[5].clone()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=stream):
        rc2 = _launch(lib, args, B, V, stream)
    assert rc2 == _lib.OK, lib.hi_rocm_last_error()
    args[5].fill_(-7)
    for _ in range(3):
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(args[5], eager)
    # release is refused during capture, then frees the buffer
    g3 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g3, stream=stream):
        rc3 = lib.hi_rocm_sampler_release(ctypes.c_void_p(int(stream.cuda_stream)))
    assert rc3 == _lib.ERR_UNSUPPORTED
    _lib.check(lib.hi_rocm_sampler_release(ctypes.c_void_p(int(stream.cuda_stream))))


def test_release_gives_memory_back(hip):
    """Streams made and dropped one per request keep no buffer once released."""
    import torch
    from hi_amd import _lib
    from hi_amd import sampler as S
    lib = _lib.load()
    B, V = 64, 151936
    args = _per_row_inputs(torch, B, V, 6)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    streams = [torch.cuda.Stream() for _ in range(6)]
    for s in streams:
        with torch.cuda.stream(s):
            _lib.check(_launch(lib, args, B, V, s))
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    # (the device commits a buffer's pages as they are first touched, so the
    # drop is below the buffers' sizes; it is still one buffer per stream)
    assert free0 - free1 >= len(streams) * (32 << 20), (free0, free1)
    for s in streams:
        S.sampler_release(s)
    S.sampler_release(streams[0])  # a second release of a stream is a no-op
    torch.cuda.synchronize()
    free2 = torch.cuda.mem_get_info()[0]
    assert free2 >= free1 + 0.9 * (free0 - free1), (free0, free1, free2)
    # a released stream allocates again on its next call
    with torch.cuda.stream(streams[1]):
        _lib.check(_launch(lib, args, B, V, streams[1]))
    torch.cuda.synchronize()
    S.sampler_release(streams[1])
