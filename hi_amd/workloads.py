"""Seeded synthetic sampler workloads: the five configurations of the
benchmark definition, and the reference test's LCG logits.

Every generator is deterministic (numpy PCG64 streams from fixed seeds), so
the GPU and the CPU oracle see identical inputs.  Nothing here is a model:
logits are drawn directly.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from ._lib import ROW_PARAMS_DTYPE


@dataclass
class Workload:
    name: str
    logits: np.ndarray                  # [B, V] float32, or uint16 bf16 bits
    params: np.ndarray                  # [B] ROW_PARAMS_DTYPE
    uniforms: np.ndarray                # [B] float32
    hist_offsets: Optional[np.ndarray] = None
    hist_ids: Optional[np.ndarray] = None
    hist_counts: Optional[np.ndarray] = None
    mask_words: Optional[np.ndarray] = None
    n_logprobs: int = 0
    notes: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return self.logits.shape[0]

    @property
    def vocab(self) -> int:
        return self.logits.shape[1]

    @property
    def is_bf16(self) -> bool:
        return self.logits.dtype == np.uint16

    def algorithmic_bytes(self) -> int:
        """Bytes one step must move at least once: logits, history pairs,
        mask, params, uniforms, outputs (tokens, logprobs)."""
        B, V = self.logits.shape
        n = self.logits.nbytes
        if self.hist_ids is not None:
            n += self.hist_ids.nbytes + self.hist_counts.nbytes + self.hist_offsets.nbytes
        if self.mask_words is not None:
            n += self.mask_words.nbytes
        n += self.params.nbytes + self.uniforms.nbytes + 4 * B
        n += B * self.n_logprobs * 8
        return int(n)


def _params(B):
    p = np.zeros(B, ROW_PARAMS_DTYPE)
    p["top_p"] = 1.0
    p["repetition_penalty"] = 1.0
    return p


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (nearest even); returns the uint16 bits."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def _zipf_logits(rng, B, V, s=1.1, noise=0.5):
    """log of a Zipf(s) distribution over a seeded permutation of the vocab,
    plus N(0, noise^2) per element."""
    ranks = np.arange(1, V + 1, dtype=np.float64)
    logp = -s * np.log(ranks)
    logp -= np.log(np.exp(logp - logp.max()).sum()) + logp.max()
    out = np.empty((B, V), np.float32)
    for b in range(B):
        perm = rng.permutation(V)
        row = np.empty(V, np.float64)
        row[perm] = logp
        out[b] = (row + rng.normal(0.0, noise, V)).astype(np.float32)
    return out


def _zipf_ids(rng, n, V, s=1.1, perm=None):
    """n token ids drawn from a Zipf(s) law over ranks 1..V (inverse CDF)."""
    ranks = np.arange(1, V + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** (-s))
    cdf /= cdf[-1]
    r = np.searchsorted(cdf, rng.random(n), side="right")
    r = np.minimum(r, V - 1)
    return (perm[r] if perm is not None else r).astype(np.uint32)


def _history_csr(per_row_ids):
    """Aggregate each row's id list into (id, count) pairs in CSR form."""
    offs = [0]
    ids, cnts = [], []
    for row in per_row_ids:
        u, c = np.unique(row, return_counts=True)
        ids.append(u.astype(np.uint32))
        cnts.append(c.astype(np.uint32))
        offs.append(offs[-1] + len(u))
    return (np.array(offs, np.uint32), np.concatenate(ids) if ids else np.zeros(0, np.uint32),
            np.concatenate(cnts) if cnts else np.zeros(0, np.uint32))


def config1(seed: int = 0, V: int = 151936) -> Workload:
    """C1: single-row ranked sampling, B=1, fp32 N(0, 3^2) with 8 ids raised
    by +10; T 0.7, top-k 40, top-p 0.9, repetition penalty 1.1; 64-token
    uniform history; top-40 logprobs."""
    rng = np.random.default_rng(seed)
    logits = rng.normal(0.0, 3.0, (1, V)).astype(np.float32)
    spikes = rng.choice(V, 8, replace=False)
    logits[0, spikes] += np.float32(10.0)
    hist = rng.integers(0, V, 64)
    p = _params(1)
    p["temperature"] = 0.7
    p["top_k"] = 40
    p["top_p"] = 0.9
    p["repetition_penalty"] = 1.1
    offs, ids, cnts = _history_csr([hist])
    u = rng.random(1).astype(np.float32)
    return Workload("c1_b1_v151936_topk40", logits, p, u, offs, ids, cnts, None, 40,
                    {"history_has_duplicates": bool(len(np.unique(hist)) < 64)})


def config2(seed: int = 2, B: int = 64, V: int = 151936) -> Workload:
    """C2: bf16 Zipf(1.1)-shaped logits; rows 0..B/2-1 greedy, the rest
    T 1.0, top-p 0.95, no top-k, no penalties."""
    rng = np.random.default_rng(seed)
    logits = f32_to_bf16_bits(_zipf_logits(rng, B, V))
    p = _params(B)
    p["temperature"][B // 2:] = 1.0
    p["top_p"][B // 2:] = 0.95
    u = rng.random(B).astype(np.float32)
    return Workload("c2_b64_v151936_bf16_greedy_topp", logits, p, u)


def config3(seed: int = 3, B: int = 256, V: int = 129280, hist_len: int = 2048) -> Workload:
    """C3: fp32 N(0, 2.5^2) with 16 per-row spikes of +8; per-row T in
    [0.3, 1.2], top-k in {20, 50, 100}, top-p in [0.8, 0.99], min-p 0.05,
    frequency 0.2, presence 0.3; 2048-token Zipf history per row."""
    rng = np.random.default_rng(seed)
    logits = rng.normal(0.0, 2.5, (B, V)).astype(np.float32)
    for b in range(B):
        logits[b, rng.choice(V, 16, replace=False)] += np.float32(8.0)
    p = _params(B)
    p["temperature"] = rng.uniform(0.3, 1.2, B).astype(np.float32)
    p["top_k"] = rng.choice([20, 50, 100], B)
    p["top_p"] = rng.uniform(0.8, 0.99, B).astype(np.float32)
    p["min_p"] = 0.05
    p["frequency_penalty"] = 0.2
    p["presence_penalty"] = 0.3
    perm = rng.permutation(V)
    offs, ids, cnts = _history_csr([_zipf_ids(rng, hist_len, V, 1.1, perm) for _ in range(B)])
    u = rng.random(B).astype(np.float32)
    return Workload("c3_b256_v129280_full_pipeline", logits, p, u, offs, ids, cnts)


def config4(seed: int = 4, B: int = 128, V: int = 256000) -> Workload:
    """C4: flat fp32 N(0, 0.5^2); top-k 1024 then top-p 0.99, T 1.0; top-20 logprobs."""
    rng = np.random.default_rng(seed)
    logits = rng.normal(0.0, 0.5, (B, V)).astype(np.float32)
    p = _params(B)
    p["temperature"] = 1.0
    p["top_k"] = 1024
    p["top_p"] = 0.99
    u = rng.random(B).astype(np.float32)
    return Workload("c4_b128_v256000_topk1024", logits, p, u, n_logprobs=20)


def config5(seed: int = 5, B: int = 32, V: int = 151936, eos_id: int = 2,
            n_fully_masked: int = 2) -> Workload:
    """C5: fp32 Zipf-shaped logits with a per-row allowed-token bitmask of
    density 0.5%, 5% or 50%; T 0.8, top-p 0.9; the last rows are fully
    masked and must return EOS."""
    rng = np.random.default_rng(seed)
    logits = _zipf_logits(rng, B, V)
    W = (V + 31) // 32
    dens = rng.choice([0.005, 0.05, 0.5], B)
    bits = rng.random((B, W * 32)) < dens[:, None]
    bits[:, V:] = False
    if n_fully_masked:
        bits[B - n_fully_masked:] = False
    words = np.packbits(bits.reshape(B, W, 32)[:, :, ::-1], axis=2).view(">u4").reshape(B, W)
    words = words.astype(np.uint32)
    p = _params(B)
    p["temperature"] = 0.8
    p["top_p"] = 0.9
    p["eos_id"] = eos_id
    u = rng.random(B).astype(np.float32)
    return Workload("c5_b32_v151936_masked", logits, p, u, mask_words=words,
                    notes={"densities": dens.tolist()})


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


def lcg_logits(seed: int, n: int, spread: float) -> np.ndarray:
    """The reference test's deterministic logits (gpu.rs:29585-29597):
    s = seed*0x9E3779B97F4A7C15 + 1; s = s*6364136223846793005 +
    1442695040888963407; u = (s >> 40) / 2^24; logit = (u - 0.5) * spread."""
    M = (1 << 64) - 1
    s = (seed * 0x9E3779B97F4A7C15 + 1) & M
    out = np.empty(n, np.float32)
    for i in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) & M
        u = np.float32(s >> 40) / np.float32(1 << 24)
        out[i] = (u - np.float32(0.5)) * np.float32(spread)
    return out


def indexer_test_scores(n: int) -> np.ndarray:
    """The scores of the reference's indexer-select test
    (crates/hi-cuda/src/dsv4_gpu.rs:7282-7289): a hash of the index folded to
    64 levels in [0, 1), so most scores tie.  u32 wrapping arithmetic."""
    idx = np.arange(n, dtype=np.uint64)
    mixed = (idx * np.uint64(0x9E3779B9) + np.uint64(0x85EBCA6B)) & np.uint64(0xFFFFFFFF)
    return (((mixed >> np.uint64(8)) % np.uint64(64)).astype(np.float32) / np.float32(64.0))


# The (n_blocks, top_k) shapes of that test; 1162 is its 4.6k-token
# production shape.
INDEXER_TEST_SHAPES = [(3, 1), (513, 512), (700, 512), (1162, 512), (4096, 512)]
