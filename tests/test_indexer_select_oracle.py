"""CPU tests that pin the oracle's DSV4 indexer block selection
(oracle/sampler_oracle.c hro_indexer_select, following
crates/hi-cuda/src/dsv4_cpu.rs:3258-3270) before the GPU tests trust it.

Checks that would catch a plausible slip: an independent pure-Python
restatement (tuple sort on total_cmp keys built with struct), the
reference test's own shapes and score generator (dsv4_gpu.rs:7277-7312),
the total_cmp special cases (-0 < +0, +NaN above +inf, -NaN below -inf),
and the invariants that fix the answer (count, separation of kept and
dropped keys, lower index first on the boundary key)."""
import struct

import numpy as np
import pytest

from hi_amd.workloads import INDEXER_TEST_SHAPES, indexer_test_scores


@pytest.fixture(scope="module")
def oracle():
    from oracle import oracle as o
    return o


def _py_total_key(v: float) -> int:
    u = struct.unpack("<I", struct.pack("<f", v))[0]
    return (~u & 0xFFFFFFFF) if u & 0x80000000 else (u | 0x80000000)


def _py_select(scores, k):
    """host_select of dsv4_gpu.rs:7260-7275, restated with Python's sort."""
    ranked = sorted(range(len(scores)), key=lambda i: (-_py_total_key(float(scores[i])), i))
    return sorted(ranked[:k])


def _check_invariants(scores, k, sel, marks):
    n = len(scores)
    take = min(k, n)
    keys = np.array([_py_total_key(float(x)) for x in scores], dtype=np.uint64)
    assert len(sel) == take
    assert list(sel) == sorted(set(int(i) for i in sel))
    assert int(marks.sum()) == take and all(marks[i] == 1 for i in sel)
    kept = marks.astype(bool)
    if take < n:
        lo, hi = keys[kept].min(), keys[~kept].max()
        assert lo >= hi
        if lo == hi:  # the boundary key: kept ones have the lower indices
            eq_kept = np.nonzero(kept & (keys == lo))[0]
            eq_drop = np.nonzero(~kept & (keys == lo))[0]
            assert eq_kept.max() < eq_drop.min()


def test_reference_test_shapes(oracle):
    for n, k in INDEXER_TEST_SHAPES:
        x = indexer_test_scores(n)
        sel, marks = oracle.indexer_select(x, k)
        assert list(sel) == _py_select(x, k), (n, k)
        _check_invariants(x, k, sel, marks)


def test_reference_score_generator():
    # first values of the hashed generator, computed by hand in u32:
    # idx 0 -> 0x85ebca6b >> 8 = 0x85ebca, % 64 = 10 -> 10/64
    x = indexer_test_scores(2)
    assert x[0] == np.float32(((0x85EBCA6B >> 8) % 64) / 64.0)
    m1 = (0x9E3779B9 + 0x85EBCA6B) & 0xFFFFFFFF
    assert x[1] == np.float32(((m1 >> 8) % 64) / 64.0)


def test_total_cmp_special_values(oracle):
    nan = np.float32(np.nan)
    neg_nan = np.frombuffer(np.uint32(0xFFC00000).tobytes(), dtype=np.float32)[0]
    cases = [
        ([-0.0, 0.0], 1, [1]),            # +0 ranks above -0
        ([0.0, -0.0], 1, [0]),
        ([np.inf, nan], 1, [1]),          # +NaN above +inf
        ([-np.inf, neg_nan], 1, [0]),     # -NaN below -inf
        ([1.0, 1.0, 1.0], 2, [0, 1]),     # ties: lower index first
        ([2.0, 5.0, 5.0, 1.0], 2, [1, 2]),
        ([3.0], 7, [0]),                  # k > n keeps everything
    ]
    for xs, k, want in cases:
        sel, marks = oracle.indexer_select(np.array(xs, dtype=np.float32), k)
        assert list(sel) == want, (xs, k)


def test_random_against_python(oracle):
    rng = np.random.default_rng(11)
    specials = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0], dtype=np.float32)
    for trial in range(60):
        n = int(rng.integers(1, 400))
        k = int(rng.integers(1, n + 20))
        if trial % 3 == 0:
            x = rng.integers(-3, 4, n).astype(np.float32)          # heavy ties
        else:
            x = rng.standard_normal(n).astype(np.float32)
        if trial % 4 == 0:
            at = rng.integers(0, n, max(1, n // 10))
            x[at] = rng.choice(specials, at.size)
        sel, marks = oracle.indexer_select(x, k)
        assert list(sel) == _py_select(x, k), (trial, n, k)
        _check_invariants(x, k, sel, marks)


def test_rejects_bad_sizes(oracle):
    with pytest.raises(ValueError):
        oracle.indexer_select(np.zeros(0, dtype=np.float32), 1)
    with pytest.raises(ValueError):
        oracle.indexer_select(np.zeros(4, dtype=np.float32), 0)
