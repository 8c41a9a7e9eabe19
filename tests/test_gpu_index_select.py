"""GPU parity of the DSV4 indexer block selection: the HIP kernel, called
through the C ABI (hi_rocm_launch_dsv4_indexer_select), against the CPU
oracle on the same scores.  Index and mark output must be bit-exact.

Cases: the reference test's own shapes and tie-heavy scores
(crates/hi-cuda/src/dsv4_gpu.rs:7277-7312), total_cmp special values, all
scores equal, k >= n, n = 1, and large n (up to 2^22 with k = 2048) on
both the one-workgroup and the many-workgroup kernels, with output buffers
pre-filled so that a missed or stray write shows."""
import ctypes
import sys

import numpy as np
import pytest

from hi_amd.workloads import INDEXER_TEST_SHAPES, indexer_test_scores

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def env():
    import torch
    from hi_amd import _lib
    from oracle import oracle
    assert torch.cuda.is_available()
    _STREAM.append(torch.cuda.Stream())  # the launcher rejects the null stream, as the reference's
    return torch, _lib.load(), oracle


_STREAM = []


def _run(env, x, k):
    torch, lib, _ = env
    n = x.size
    take = min(k, n)
    d_x = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()
    d_marks = torch.full((n,), 0xAB, dtype=torch.uint8, device="cuda")
    d_sel = torch.full((take + 64,), -7, dtype=torch.int32, device="cuda")
    stream = _STREAM[0]
    torch.cuda.synchronize()
    st = lib.hi_rocm_launch_dsv4_indexer_select(d_x.data_ptr(), n, k, d_marks.data_ptr(),
                                                d_sel.data_ptr(), ctypes.c_void_p(stream.cuda_stream))
    assert st == 0, lib.hi_rocm_last_error()
    torch.cuda.synchronize()
    sel = d_sel.cpu().numpy()
    assert (sel[take:] == -7).all(), "write past the kept count"
    return sel[:take], d_marks.cpu().numpy()


def _check(env, x, k, label):
    _, _, oracle = env
    say(f"indexer select: {label} n={x.size} k={k}")
    sel, marks = _run(env, x, k)
    want_sel, want_marks = oracle.indexer_select(x, k)
    assert np.array_equal(sel, want_sel), label
    assert np.array_equal(marks, want_marks), label


def test_reference_shapes(env):
    for n, k in INDEXER_TEST_SHAPES:
        _check(env, indexer_test_scores(n), k, "reference test scores")


def test_special_values_and_ties(env):
    nan = np.float32(np.nan)
    neg_nan = np.frombuffer(np.uint32(0xFFC00000).tobytes(), dtype=np.float32)[0]
    _check(env, np.array([-0.0, 0.0], np.float32), 1, "signed zeros")
    _check(env, np.array([np.inf, nan, 1.0], np.float32), 1, "+nan over +inf")
    _check(env, np.array([-np.inf, neg_nan, -1.0], np.float32), 2, "-nan under -inf")
    _check(env, np.array([0.5], np.float32), 3, "n=1, k>n")
    _check(env, np.full(5000, 0.25, np.float32), 1234, "all equal")
    _check(env, np.full(5000, 0.25, np.float32), 5000, "all equal, k=n")
    rng = np.random.default_rng(5)
    x = rng.integers(-2, 3, 70001).astype(np.float32)
    at = rng.integers(0, x.size, 300)
    x[at] = rng.choice(np.array([nan, neg_nan, np.inf, -np.inf, -0.0], np.float32), at.size)
    for k in (1, 63, 64, 65, 2048, 30000, 70001, 90000):
        _check(env, x, k, "five levels with specials")


def test_random_sizes(env):
    rng = np.random.default_rng(7)
    for n in (1, 2, 63, 64, 65, 1000, 1023, 1024, 1025, 16383, 16385, 100003, (1 << 18) + 1):
        x = rng.standard_normal(n).astype(np.float32)
        for k in sorted({1, max(1, n // 3), min(2048, n), n}):
            _check(env, x, k, "normal")


def test_repeated_launches_reuse_buffers(env):
    """One set of buffers over several layers' launches (the decode step
    reuses its marks scratch, dsv4_gpu.rs:4555-4576): every launch leaves
    marks and the output complete for its own scores."""
    torch, lib, oracle = env
    rng = np.random.default_rng(3)
    n_max, k = 4096, 512
    d_marks = torch.full((n_max,), 0xAB, dtype=torch.uint8, device="cuda")
    d_sel = torch.full((k,), -7, dtype=torch.int32, device="cuda")
    s = ctypes.c_void_p(_STREAM[0].cuda_stream)
    for layer, n in enumerate((4096, 1162, 700, 4096)):
        x = rng.standard_normal(n).astype(np.float32)
        d_x = torch.from_numpy(x).cuda()
        say(f"indexer select: layer {layer} n={n} k={k}")
        assert lib.hi_rocm_launch_dsv4_indexer_select(d_x.data_ptr(), n, k, d_marks.data_ptr(),
                                                      d_sel.data_ptr(), s) == 0
        torch.cuda.synchronize()
        want_sel, want_marks = oracle.indexer_select(x, k)
        assert np.array_equal(d_sel.cpu().numpy()[:min(k, n)], want_sel)
        assert np.array_equal(d_marks.cpu().numpy()[:n], want_marks)


def test_python_front_end(env):
    torch, _, oracle = env
    from hi_amd.index_select import dsv4_indexer_select, launch_dsv4_indexer_select
    x = indexer_test_scores(1162)
    want_sel, want_marks = oracle.indexer_select(x, 512)
    # no device-wide synchronisation: the results are read through the
    # current (null) stream, which the front end orders after its launch
    for _ in range(3):
        sel, marks = dsv4_indexer_select(torch.from_numpy(x).cuda(), 512)
        assert np.array_equal((sel + 0).cpu().numpy(), want_sel)
        assert np.array_equal(marks.cpu().numpy(), want_marks)
    with pytest.raises(ValueError):
        launch_dsv4_indexer_select(torch.from_numpy(x).cuda(), 1162, 512,
                                   torch.empty(10, dtype=torch.uint8, device="cuda"),
                                   torch.empty(512, dtype=torch.int32, device="cuda"))


def test_unaligned_buffers(env):
    """Scores and marks that start off a 16-byte / 4-byte boundary, and n not
    a multiple of 4: the element-by-element load and store path."""
    torch, lib, oracle = env
    rng = np.random.default_rng(9)
    s = ctypes.c_void_p(_STREAM[0].cuda_stream)
    for n, k in ((4096, 300), (65536, 2048), (65535, 2048), (16385, 100)):
        x = rng.standard_normal(n).astype(np.float32)
        big = torch.from_numpy(np.concatenate([[np.float32(7)], x])).cuda()
        marks_big = torch.full((n + 1,), 0xAB, dtype=torch.uint8, device="cuda")
        d_sel = torch.full((min(k, n),), -7, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        say(f"indexer select: unaligned n={n} k={k}")
        assert lib.hi_rocm_launch_dsv4_indexer_select(big.data_ptr() + 4, n, k, marks_big.data_ptr() + 1,
                                                      d_sel.data_ptr(), s) == 0
        torch.cuda.synchronize()
        want_sel, want_marks = oracle.indexer_select(x, k)
        assert np.array_equal(d_sel.cpu().numpy(), want_sel)
        m = marks_big.cpu().numpy()
        assert m[0] == 0xAB and np.array_equal(m[1:], want_marks)


def test_many_workgroups_ties_and_reuse(env):
    """The many-workgroup form (n above 8192): every score equal (the
    boundary bin holds all n, more than the output kernel keeps in LDS, so
    the threshold is selected over global memory), three levels, and
    repeated launches of different n and k on one stream (the histogram the
    calls share must be back at zero after each)."""
    rng = np.random.default_rng(11)
    _check(env, np.full(70000, 0.25, np.float32), 1234, "all equal, many workgroups")
    _check(env, np.full(70000, -3.0, np.float32), 70000, "all equal, many workgroups, k=n")
    x = rng.integers(0, 3, 50000).astype(np.float32)
    for k in (1, 4096, 16667, 33334, 49999):
        _check(env, x, k, "three levels, many workgroups")
    for n, k in ((65536, 2048), (20000, 2048), (65536, 512), (4194304, 2048), (8193, 8193), (12289, 1)):
        _check(env, rng.standard_normal(n).astype(np.float32), k, "repeated launches")


def test_capture_without_buffer_takes_one_workgroup(env):
    """A first call on a stream inside graph capture cannot allocate the
    many-workgroup buffer: it takes the one-workgroup kernel, and the
    captured graph replays to the oracle's result."""
    torch, lib, oracle = env
    rng = np.random.default_rng(13)
    n, k = 65536, 2048
    x = rng.standard_normal(n).astype(np.float32)
    d_x = torch.from_numpy(x).cuda()
    d_marks = torch.full((n,), 0xAB, dtype=torch.uint8, device="cuda")
    d_sel = torch.full((k,), -7, dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()  # no buffer yet
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    say(f"indexer select: captured on a fresh stream n={n} k={k}")
    with torch.cuda.graph(g, stream=stream):
        st = lib.hi_rocm_launch_dsv4_indexer_select(d_x.data_ptr(), n, k, d_marks.data_ptr(), d_sel.data_ptr(),
                                                    ctypes.c_void_p(stream.cuda_stream))
    assert st == 0, lib.hi_rocm_last_error()
    want_sel, want_marks = oracle.indexer_select(x, k)
    for _ in range(3):
        d_marks.fill_(0xAB)
        d_sel.fill_(-7)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(d_sel.cpu().numpy(), want_sel)
        assert np.array_equal(d_marks.cpu().numpy(), want_marks)
