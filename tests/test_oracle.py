"""CPU tests that pin the oracle (oracle/sampler_oracle.c) before it is trusted.

Each check is chosen so that a plausible restatement mistake (a wrong fold
order, a dropped tie rule, a swapped comparison) fails it:
  * the reference's own test grid and tie surface (gpu.rs:29505-29760),
  * its known answers (qwen_cpu.rs:4463-4485, hi-mlx generate.rs:193-197,
    lib.rs:18509-18575),
  * a second, independent Python restatement on small vocabularies,
  * closed forms (top_k = 1, top_p = 0, u = 0, penalties on tiny inputs),
  * inverse-CDF invariants (lib.rs:25972-26054),
  * the committed golden vectors in tests/golden/.
"""
import json
import os

import numpy as np
import pytest

from hi_amd.workloads import lcg_logits

F32 = np.float32
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")

GRID_VOCABS = [64, 200, 1500, 4096]
GRID_TEMPS = [0.7, 1.0, 1.3]
GRID_TOP_PS = [float("inf"), 0.5, 0.9, 0.95, 0.999]
GRID_TOP_KS = [None, 1, 10, 40, 2000]
GRID_SAMPLES = [0.0, 0.13, 0.5, 0.77, 0.999]


def test_reference_grid_windowed_equals_full_sort(oracle):
    """gpu.rs:29582-29633: 1500 cases, windowed sampler == full-sort baseline."""
    cases = 0
    for vi, n in enumerate(GRID_VOCABS):
        logits = lcg_logits(0x1234 + vi, n, 4.0)
        for t in GRID_TEMPS:
            for tp in GRID_TOP_PS:
                for tk in GRID_TOP_KS:
                    for sm in GRID_SAMPLES:
                        got = oracle.ranked_sample(logits, t, tp, tk, sm)
                        want = oracle.ranked_sample_brute(logits, t, tp, tk, sm)
                        assert got == want, (n, t, tp, tk, sm)
                        cases += 1
    assert cases >= 1500


def test_golden_reference_grid(oracle):
    """Committed expected tokens for the reference grid and its tie surface."""
    with open(os.path.join(GOLDEN, "reference_grid.json")) as f:
        gold = json.load(f)
    assert len(gold["cases"]) >= 1500
    cache = {}
    for c in gold["cases"]:
        key = (c["kind"], c["seed"], c["n"])
        if key not in cache:
            if c["kind"] == "lcg":
                cache[key] = lcg_logits(c["seed"], c["n"], 4.0)
            else:
                cache[key] = np.array([[1.5, 0.25, -2.0][i % 3] for i in range(c["n"])], F32)
        tp = float("inf") if c["top_p"] is None else c["top_p"]
        got = oracle.ranked_sample(cache[key], c["temperature"], tp, c["top_k"], c["sample"])
        assert got == c["token"], c


def test_tie_surface_matches_bruteforce(oracle):
    """gpu.rs:29700-29706: three distinct values, ties resolved by index."""
    for n in (200, 1500, 4096):
        ties = np.array([[1.5, 0.25, -2.0][i % 3] for i in range(n)], F32)
        for t in (0.7, 1.0):
            for tp in (float("inf"), 0.5, 0.9, 0.999):
                for tk in (None, 1, 10, 40, 2000):
                    for sm in GRID_SAMPLES:
                        assert oracle.ranked_sample(ties, t, tp, tk, sm) == \
                            oracle.ranked_sample_brute(ties, t, tp, tk, sm)
    # with k = 10 over ties every candidate has weight 1: the draw is uniform
    # over the 10 lowest indices holding 1.5, i.e. 0, 3, ..., 27
    ties = np.array([[1.5, 0.25, -2.0][i % 3] for i in range(300)], F32)
    got = {oracle.ranked_sample(ties, 1.0, float("inf"), 10, u) for u in np.linspace(0, 0.999, 200)}
    assert got == set(range(0, 30, 3))


def test_known_answers(oracle):
    # qwen_cpu.rs:4463-4474: top-k 2 of [0,1,2,3] only yields 2 or 3
    got = {oracle.ranked_sample([0, 1, 2, 3], 0.8, 1.0, 2, u) for u in np.linspace(0, 1, 64)}
    assert got == {2, 3}
    # qwen_cpu.rs:4477-4485: top_p 0 selects the top candidate
    assert all(oracle.ranked_sample([0, 3, 1, 2], 1.0, 0.0, None, u) == 1 for u in np.linspace(0, 1, 9))
    # hi-mlx generate.rs:193-197: greedy picks index 1
    assert oracle.argmax_ieee([0.1, 3.0, 2.9]) == 1
    assert oracle.argmax_total([0.1, 3.0, 2.9]) == 1
    # lib.rs:18509-18575: top_p = 0 sampled equals greedy
    for seed in range(5):
        x = lcg_logits(seed, 500, 6.0)
        assert oracle.ranked_sample(x, 0.9, 0.0, None, 0.7) == oracle.argmax_total(x)
    # temperature <= 0 or non-finite is greedy (gpu.rs:760-765)
    x = lcg_logits(9, 100, 4.0)
    for t in (0.0, -1.0, float("nan"), float("inf")):
        assert oracle.ranked_sample(x, t, 0.5, 5, 0.3) == oracle.argmax_total(x)


def _py_ranked(expf, logits, T, top_p, top_k, u, min_p=0.0):
    """Independent restatement of gpu.rs:753-900 (full sort; Python floats
    only through numpy float32 scalars)."""
    lg = np.asarray(logits, F32)
    T = F32(T)
    scaled = np.array([F32(l / T) if np.isfinite(l) else F32(-np.inf) for l in lg], F32)
    mx = F32(-np.inf)
    for v in scaled:
        mx = v if v > mx else mx
    w = expf((scaled - mx).astype(F32))
    if min_p > 0:
        w = np.where(w < F32(min_p), F32(0), w).astype(F32)
    order = sorted(range(len(lg)), key=lambda i: (-float(w[i]), i))
    if top_k:
        order = order[:min(top_k, len(order))]
        total = F32(-0.0)
        for i in order:
            total = F32(total + w[i])
    else:
        total = F32(-0.0)
        for v in w:
            total = F32(total + v)
    cutoff = F32(min(max(top_p, 0.0), 1.0)) if np.isfinite(top_p) else F32(1.0)
    cands, cum = [], F32(0.0)
    for i in order:
        if w[i] <= 0:
            continue
        cands.append(i)
        cum = F32(cum + F32(w[i] / total))
        if cutoff < 1 and cum >= cutoff:
            break
    ct = F32(-0.0)
    for i in cands:
        ct = F32(ct + w[i])
    uu = F32(min(max(u, 0.0), 0.99999994)) if np.isfinite(u) else F32(0)
    target = F32(uu * ct)
    c = F32(0.0)
    for i in cands:
        c = F32(c + w[i])
        if target < c:
            return i
    return cands[-1]


def test_independent_python_restatement(oracle):
    rng = np.random.default_rng(7)
    n_cases = 0
    for trial in range(120):
        n = int(rng.integers(2, 90))
        kind = trial % 4
        if kind == 0:
            x = rng.normal(0, 3, n).astype(F32)
        elif kind == 1:
            x = rng.integers(-3, 3, n).astype(F32)  # heavy ties
        elif kind == 2:
            x = (rng.normal(0, 40, n)).astype(F32)  # underflowing weights
        else:
            x = rng.normal(0, 1, n).astype(F32)
            x[rng.integers(0, n, 3)] = -np.inf
        T = float(rng.choice([0.3, 0.7, 1.0, 1.7]))
        tp = float(rng.choice([0.0, 0.3, 0.9, 0.999, 1.0, np.inf]))
        tk = int(rng.choice([0, 1, 3, 10, 1000]))
        mp = float(rng.choice([0.0, 0.0, 0.05, 0.5]))
        for u in (0.0, 0.25, 0.5, 0.999, 0.99999994):
            want = _py_ranked(oracle.expf, x, T, tp, tk or None, u, mp)
            got = oracle.ranked_sample(x, T, tp, tk or None, u, min_p=mp)
            assert got == want, (trial, n, T, tp, tk, mp, u)
            n_cases += 1
    assert n_cases == 600


def test_closed_forms(oracle):
    rng = np.random.default_rng(11)
    for _ in range(50):
        n = int(rng.integers(5, 3000))
        x = rng.normal(0, 2, n).astype(F32)
        w = oracle.expf((x / F32(0.8)) - (x / F32(0.8)).max())
        wmax = w.max()
        first = int(np.flatnonzero(w == wmax)[0])
        # top_k = 1: the weight argmax, lowest index among equal weights
        assert oracle.ranked_sample(x, 0.8, 1.0, 1, float(rng.random())) == first
        # u = 0: the first candidate in rank order
        assert oracle.ranked_sample(x, 0.8, 0.9, 50, 0.0) == first
        # min_p = 1 keeps only weight 1
        assert oracle.ranked_sample(x, 0.8, 1.0, None, 0.99, min_p=1.0) == first
        # a finite, non-clamped uniform above 1 behaves like 0.99999994
        assert oracle.ranked_sample(x, 0.8, 0.95, 30, 5.0) == oracle.ranked_sample(x, 0.8, 0.95, 30, 0.99999994)
        # NaN uniform behaves like 0 (gpu.rs:882-886)
        assert oracle.ranked_sample(x, 0.8, 0.95, 30, float("nan")) == first


def test_top_p_normaliser_closed_forms(oracle):
    """gpu.rs:834-838: with top_k set, the top-p normaliser is the kept mass;
    without it, the whole vocabulary's mass.  Equal logits give equal
    weights 1, so the nucleus is fixed by counting: n equal weights, top_p
    0.5 and a normaliser of m keep the first ceil(m / 2) ranks (cum_p of
    rank r is (r + 1) / m, exact for these m)."""
    x = np.zeros(4, F32)
    # no top_k: total 4, cum_p 0.25, 0.5 -> ranks {0, 1}
    assert oracle.ranked_sample(x, 1.0, 0.5, None, 0.4) == 0
    assert oracle.ranked_sample(x, 1.0, 0.5, None, 0.75) == 1
    # top_k 2: total 2 (the kept mass), cum_p 0.5 at rank 0 -> {0}
    for u in (0.0, 0.4, 0.75, 0.99999994):
        assert oracle.ranked_sample(x, 1.0, 0.5, 2, u) == 0
    # top_k 3: total 3, cum_p 1/3, 2/3 -> {0, 1}
    assert oracle.ranked_sample(x, 1.0, 0.5, 3, 0.75) == 1
    # top_k 4 = V: total 4 again -> {0, 1}
    assert oracle.ranked_sample(x, 1.0, 0.5, 4, 0.75) == 1
    # eight equal weights, top_p 0.25: without top_k {0, 1}; top_k 4 keeps
    # mass 4, so cum_p 0.25 at rank 0 -> {0}
    y = np.zeros(8, F32)
    assert oracle.ranked_sample(y, 1.0, 0.25, None, 0.9) == 1
    assert oracle.ranked_sample(y, 1.0, 0.25, 4, 0.9) == 0
    # the full sort gives the same answers
    assert oracle.ranked_sample_brute(y, 1.0, 0.25, 4, 0.9) == 0
    assert oracle.ranked_sample_brute(x, 1.0, 0.5, 2, 0.75) == 0


def test_inverse_cdf_invariants(oracle):
    """lib.rs:25972-26054: each pick lies in its CDF bin, picks monotone in u."""
    rng = np.random.default_rng(5)
    for trial in range(6):
        n = 2000
        x = rng.normal(0, 2, n).astype(F32)
        T = 1.0
        us = np.sort(rng.random(200).astype(F32))
        # temperature-only path: CDF in index order
        picks = [oracle.temp_only_sample(x, T, u) for u in us]
        assert all(a <= b for a, b in zip(picks, picks[1:]))
        w = np.exp(x.astype(np.float64) - x.max())
        cdf = np.cumsum(w)
        total = cdf[-1]
        for u, p in zip(us, picks):
            lo = cdf[p - 1] if p > 0 else 0.0
            assert lo - 1e-3 * total <= u * total <= cdf[p] + 1e-3 * total
        # ranked path: monotone in rank position
        order = sorted(range(n), key=lambda i: (-w[i], i))
        pos = {i: r for r, i in enumerate(order)}
        rp = [pos[oracle.ranked_sample(x, T, 0.9, None, u)] for u in us]
        assert all(a <= b for a, b in zip(rp, rp[1:]))


def _py_temp_only(expf, x, T, u):
    """Independent restatement of kernels.cu:7803-7867 (index-order CDF)."""
    x = np.asarray(x, F32)
    n = len(x)
    fin = np.isfinite(x)
    best, bi, have = F32(-np.inf), 0, False
    for i in range(n):
        if fin[i] and (not have or x[i] > best or (x[i] == best and i % 256 < bi % 256)):
            best, bi, have = x[i], i, True
    ms = F32(best / F32(T))
    if not np.isfinite(ms):
        return bi

    def wgt(i):
        if not fin[i]:
            return F32(0)
        s = F32(x[i] / F32(T))
        if not np.isfinite(s):
            return F32(0)
        return expf(np.array([F32(s - ms)], F32))[0]

    chunk = (n + 255) // 256
    cs = []
    for t in range(256):
        s = F32(0)
        for i in range(t * chunk, min(t * chunk + chunk, n)):
            s = F32(s + wgt(i))
        cs.append(s)
    pre, acc = [], F32(0)
    for c in cs:
        pre.append(acc)
        acc = F32(acc + c)
    uu = F32(min(max(u, 0.0), 0.99999994)) if np.isfinite(u) else F32(0)
    target = F32(uu * acc)
    tok = None
    for t in range(256):
        st, en = t * chunk, min(t * chunk + chunk, n)
        lo = pre[t]
        hi = F32(lo + cs[t])
        if st < en and target >= lo and (target < hi or t == 255):
            c, ch = lo, -1
            for i in range(st, en):
                wv = wgt(i)
                if wv <= 0:
                    continue
                ch = i
                c = F32(c + wv)
                if target < c:
                    break
            if ch >= 0:
                tok = ch if tok is None else min(tok, ch)
    return tok if tok is not None else bi


def test_temp_only_independent(oracle):
    rng = np.random.default_rng(3)
    for trial in range(8):
        n = int(rng.integers(1, 1200))
        x = rng.normal(0, 2, n).astype(F32)
        if trial % 3 == 0:
            x[rng.integers(0, n, max(1, n // 10))] = -np.inf
        for u in (0.0, 0.3, 0.77, 0.99999994):
            assert oracle.temp_only_sample(x, 0.9, u) == _py_temp_only(oracle.expf, x, 0.9, u)


def _bitrev8(r):
    return int(f"{r & 255:08b}"[::-1], 2)


def test_finite_lane_argmax_rule(oracle):
    # kernels.cu:7780-7801: lane t of 256 keeps its first maximum; the tree
    # (strides 128 .. 1, strict >) decides bit 0 of the lane last, so tied
    # maxima go to the smallest bit reversal of (idx mod 256), then the
    # smallest idx.  Maxima at 300 (residue 44, reversed 52) and 5 (residue
    # 5, reversed 160): 300 wins.  Adding 260 (residue 4, reversed 32): 260.
    x = np.zeros(600, F32)
    x[300] = x[5] = 3.0
    assert oracle.argmax_finite_lane(x)[0] == 300
    x[260] = 3.0
    assert oracle.argmax_finite_lane(x)[0] == 260
    assert oracle.argmax_ieee(x) == 5
    # residues 1 (reversed 128) and 2 (reversed 64): 2 wins; 0 beats both
    z = np.zeros(8, F32)
    z[1] = z[2] = 1.0
    assert oracle.argmax_finite_lane(z)[0] == 2
    z[0] = 1.0
    assert oracle.argmax_finite_lane(z)[0] == 0
    # same residue: the lower index (lane t keeps its first maximum)
    y2 = np.zeros(1000, F32)
    y2[7 + 512] = y2[7 + 256] = 2.0
    assert oracle.argmax_finite_lane(y2)[0] == 7 + 256
    # every tie pattern on random inputs equals the closed form
    rng = np.random.default_rng(11)
    for trial in range(300):
        n = int(rng.integers(1, 2000))
        v = rng.integers(0, 4, n).astype(F32)
        if trial % 5 == 0:
            v[rng.integers(0, n, max(1, n // 7))] = np.nan
        if trial % 7 == 0:
            v[rng.integers(0, n, max(1, n // 9))] = np.inf
        fin = np.isfinite(v)
        if not fin.any():
            assert oracle.argmax_finite_lane(v)[0] == 0
            continue
        m = v[fin].max()
        ties = np.flatnonzero(fin & (v == m))
        want = min(ties, key=lambda i: (_bitrev8(int(i)), int(i)))
        assert oracle.argmax_finite_lane(v)[0] == want, trial
    # non-finite values never win the finite argmax; IEEE argmax keeps +inf
    y = np.array([1.0, np.inf, 2.0, np.nan], F32)
    assert oracle.argmax_finite_lane(y)[0] == 2
    assert oracle.argmax_ieee(y) == 1
    assert oracle.argmax_total(y) == 3  # total_cmp: positive NaN is largest
    assert oracle.argmax_ieee(np.full(4, -np.inf, F32)) == 0


def test_penalty_closed_forms(oracle):
    from oracle.oracle import ROW_PARAMS_DTYPE
    p = np.zeros(1, ROW_PARAMS_DTYPE)
    p["temperature"] = 1.0
    p["top_p"] = 1.0
    p["repetition_penalty"] = 1.3
    p["frequency_penalty"] = 0.2
    p["presence_penalty"] = 0.5
    raw = np.array([2.0, -2.0, 0.0, 1.5, 7.0], F32)
    ids = np.array([0, 1, 2, 3, 0, 99], np.uint32)   # id 0 twice, 99 out of range
    cnt = np.array([2, 3, 1, 0, 1, 4], np.uint32)
    out, any_f = oracle.process_row(raw, p, ids, cnt)
    assert any_f
    want = raw.copy()
    c = [3, 3, 1, 0, 0]
    for i in range(5):
        l = F32(raw[i])
        if c[i]:
            for _ in range(c[i]):
                l = F32(l * F32(1.3)) if l < 0 else F32(l / F32(1.3))
            l = F32(l - F32(F32(0.2) * F32(c[i])))
            l = F32(l - F32(0.5))
        want[i] = l
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))
    # the REP_ONCE flag applies the repetition penalty once per token
    p["flags"] = 1
    out2, _ = oracle.process_row(raw, p, ids, cnt)
    assert out2[0] == F32(F32(F32(2.0) / F32(1.3)) - F32(F32(0.2) * F32(3))) - F32(0.5)
    # |p - 1| <= FLT_EPSILON switches the repetition penalty off (generate.rs:60)
    p["flags"] = 0
    p["repetition_penalty"] = np.nextafter(F32(1.0), F32(2.0))
    p["frequency_penalty"] = 0.0
    p["presence_penalty"] = 0.0
    out3, _ = oracle.process_row(raw, p, ids, cnt)
    assert np.array_equal(out3, raw - F32(0.0))


def test_mask_and_eos(oracle):
    from oracle.oracle import ROW_PARAMS_DTYPE
    B, V = 3, 70
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (B, V)).astype(F32)
    W = (V + 31) // 32
    mask = np.zeros((B, W), np.uint32)
    mask[0, 0] = 1 << 7            # only token 7 allowed
    mask[1, 2] = 1 << (65 - 64)    # only token 65 allowed
    p = np.zeros(B, ROW_PARAMS_DTYPE)
    p["temperature"] = [0.0, 0.8, 0.8]
    p["top_p"] = [1.0, 0.9, 0.9]
    p["eos_id"] = 42
    r = oracle.sample_rows(x, p, np.array([0.3, 0.9, 0.5], F32), mask_words=mask, n_logprobs=3)
    assert r["tokens"].tolist() == [7, 65, 42]
    assert r["path"].tolist()[2] == oracle.EOS
    assert r["logprob_ids"][0, 0] == 7 and r["logprobs"][0, 0] == 0.0
    assert np.all(r["logprob_ids"][2] == 0xFFFFFFFF) and r["token_logprobs"][2] == 0.0


def test_logprobs_match_float64(oracle):
    from oracle.oracle import ROW_PARAMS_DTYPE
    rng = np.random.default_rng(2)
    B, V = 4, 3000
    x = rng.normal(0, 3, (B, V)).astype(F32)
    p = np.zeros(B, ROW_PARAMS_DTYPE)
    p["temperature"] = [0.0, 0.7, 1.3, 0.9]
    p["top_p"] = [1.0, 0.9, 1.0, 0.8]
    p["top_k"] = [0, 40, 0, 7]
    r = oracle.sample_rows(x, p, rng.random(B).astype(F32), n_logprobs=20)
    for b in range(B):
        T = p["temperature"][b] if p["temperature"][b] > 0 else 1.0
        s = (x[b] / F32(T)).astype(np.float64)
        lp = s - s.max() - np.log(np.exp(s - s.max()).sum())
        order = np.lexsort((np.arange(V), -lp))[:20]
        assert r["logprob_ids"][b].tolist() == order.tolist()
        np.testing.assert_allclose(r["logprobs"][b], lp[order], rtol=1e-6)
        np.testing.assert_allclose(r["token_logprobs"][b], lp[r["tokens"][b]], rtol=1e-6)


def test_expf_port_matches_glibc_exhaustively(tmp_path):
    """The weight function the kernels use (hi_amd/csrc/exact_expf.h), built
    for the host, equals glibc expf on every float in [-104, 0] and on a
    stride sample of the rest."""
    import subprocess
    src = os.path.join(os.path.dirname(__file__), "native", "expf_port_check.cpp")
    inc = os.path.join(os.path.dirname(os.path.dirname(__file__)), "hi_amd", "csrc")
    exe = tmp_path / "expf_port_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-pthread", "-I", inc, src,
                    "-o", str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    assert "mismatches 0" in out, out


def test_glibc_expf_monotone_on_negatives(oracle):
    """Ranking by scaled logit is consistent with ranking by weight only if
    expf is non-decreasing; check it on a dense sample of (-104, 0]."""
    x = -np.linspace(0, 104, 2_000_001).astype(F32)[::-1]
    x = np.unique(x)
    y = oracle.expf(x)
    assert np.all(np.diff(y.astype(np.float64)) >= 0)
