"""The streaming selects' group-maximum bound has two forms in
hi_amd/csrc/sampler_kernels.hip (wave_prefix_reach): a 20-step bit-by-bit
search for the largest key prefix (low 12 bits clear) that at least `need`
of a wave's 256 group-maximum keys reach, and, for need <= 16, the need-th
largest key with its low 12 bits cleared.  The device code takes the second
form for small `need`; this checks on the CPU that both forms give the same
prefix on random, tied, tiny and saturated key sets (the GPU parity tests run
the device code itself)."""
import numpy as np


def bit_search(keys, need):
    prefix = 0
    for bit in range(31, 11, -1):
        probe = prefix | (1 << bit)
        if int(np.count_nonzero(keys >= probe)) >= need:
            prefix = probe
    return prefix


def kth_largest(keys, need):
    s = np.sort(keys)[::-1]
    return int(s[need - 1]) & 0xFFFFF000


def test_forms_agree():
    rng = np.random.default_rng(7)
    cases = []
    for _ in range(400):
        kind = rng.integers(0, 5)
        if kind == 0:
            k = rng.integers(0, 2**32, 256, dtype=np.uint64)
        elif kind == 1:  # many ties
            k = rng.choice(rng.integers(0, 2**32, 5, dtype=np.uint64), 256)
        elif kind == 2:  # keys below the 12-bit prefix granularity
            k = rng.integers(0, 0x1000, 256, dtype=np.uint64)
        elif kind == 3:  # unused groups read as zero
            k = rng.integers(0, 2**32, 256, dtype=np.uint64)
            k[rng.random(256) < 0.9] = 0
        else:  # keys of a few f32 logits (order-preserving map of positive floats)
            x = rng.normal(0, 3, 256).astype(np.float32)
            b = x.view(np.uint32).astype(np.uint64)
            k = np.where(x >= 0, b | 0x80000000, (~b) & 0xFFFFFFFF)
        cases.append(k.astype(np.uint64))
    for k in cases:
        for need in range(1, 17):
            assert bit_search(k, need) == kth_largest(k, need), (need, k[:8])
