"""GPU: the workgroup form of the sequential f32 fold (hi_rocm_debug_fold)
against a literal left-to-right float32 fold (numpy's float32 cumsum
accumulates sequentially in float32; tests/test_exact_fold.py pins the
integer emulation itself on the host)."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32 = np.float32


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def seq_starts(terms, counts, a0):
    """Value before every run and the final value, by a sequential fold."""
    x = np.repeat(terms, counts)
    c = np.cumsum(np.concatenate([np.array([a0], F32), x]), dtype=F32)
    ends = np.cumsum(counts.astype(np.int64))
    starts = np.concatenate([np.zeros(1, np.int64), ends[:-1]])
    return c[starts], c[-1]


def gpu_fold(hip, terms, counts, a0):
    import torch
    lib = hip.load()
    t = torch.from_numpy(np.ascontiguousarray(terms, F32)).cuda()
    m = torch.from_numpy(np.ascontiguousarray(counts, np.uint32).view(np.int32)).cuda()
    out = torch.empty(len(terms), dtype=torch.float32, device="cuda")
    fin = torch.empty(1, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    hip.check(lib.hi_rocm_debug_fold(t.data_ptr(), m.data_ptr(), len(terms), float(a0), out.data_ptr(),
                                     fin.data_ptr(), s.cuda_stream))
    s.synchronize()
    return out.cpu().numpy(), float(fin.cpu().numpy()[0])


def cases(rng):
    # vocab-order weights: exp of normals, many tiny terms
    for n in (1, 2, 63, 64, 65, 1000, 4096, 20000, 65536):
        yield f"weights n={n}", np.exp(rng.normal(-4, 3, n)).astype(F32), np.ones(n, np.uint32), -0.0
    # rank order: descending weights, then divided by a total (cum_p)
    for n in (100, 1024, 4096):
        w = np.sort(np.exp(rng.normal(0, 1.5, n)).astype(F32))[::-1]
        w = (w / w[0]).astype(F32)
        yield f"rank-order n={n}", w, np.ones(n, np.uint32), -0.0
        tot = np.cumsum(w, dtype=F32)[-1]
        yield f"cum_p n={n}", (w / tot).astype(F32), np.ones(n, np.uint32), 0.0
    # runs of equal terms (bf16-like weights with multiplicities)
    for n in (10, 180, 2000):
        v = np.sort(np.exp(rng.normal(-6, 3, n)).astype(F32))[::-1]
        c = rng.integers(1, 2000, n).astype(np.uint32)
        yield f"runs n={n}", v, c, -0.0
    # exact halves: short-mantissa terms, both parities
    for n in (500, 5000):
        v = np.ldexp(rng.integers(1, 8, n), -rng.integers(0, 30, n)).astype(F32)
        yield f"halves n={n}", v, rng.integers(1, 50, n).astype(np.uint32), np.float32(rng.random())
    # subnormal start and terms, zeros, large jumps
    sub = (rng.integers(0, 1 << 23, 3000).astype(np.uint32)).view(F32)
    yield "subnormals", sub, np.ones(3000, np.uint32), 0.0
    z = np.exp(rng.normal(-2, 4, 3000)).astype(F32)
    z[rng.integers(0, 3000, 600)] = 0.0
    z[rng.integers(0, 3000, 5)] = 1e6
    yield "zeros and jumps", z, rng.integers(1, 4, 3000).astype(np.uint32), 1e-30


def test_fold_matches_sequential_float32(hip):
    rng = np.random.default_rng(7)
    for name, terms, counts, a0 in cases(rng):
        say(f"fold case {name}")
        want_s, want_f = seq_starts(terms, counts, a0)
        got_s, got_f = gpu_fold(hip, terms, counts, a0)
        bad = np.flatnonzero(got_s.view(np.uint32) != want_s.view(np.uint32))
        # -0 vs +0 only at a zero start
        bad = [b for b in bad if not (got_s[b] == 0 and want_s[b] == 0)]
        assert not bad, (name, bad[:5], got_s[bad[:5]], want_s[bad[:5]])
        assert np.float32(got_f).view(np.uint32) == np.float32(want_f).view(np.uint32) or \
            (got_f == 0 and want_f == 0), (name, got_f, want_f)


def test_fold_rejects_bad_arguments(hip):
    import torch
    lib = hip.load()
    s = torch.cuda.Stream()
    t = torch.zeros(4, device="cuda")
    assert lib.hi_rocm_debug_fold(t.data_ptr(), t.data_ptr(), 0, 0.0, t.data_ptr(), t.data_ptr(),
                                  s.cuda_stream) == 1
    assert lib.hi_rocm_debug_fold(t.data_ptr(), t.data_ptr(), 65537, 0.0, t.data_ptr(), t.data_ptr(),
                                  s.cuda_stream) == 1
