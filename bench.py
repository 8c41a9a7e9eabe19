"""Benchmark of the hi-rocm batched token sampler on one MI355X.

Headline metric: sampled rows/s for the full pipeline at
B=256, V=129280 fp32 (config 3: penalties + top-k + top-p + min-p + draw),
plus µs/step at B=1 (config 1, hipGraph-captured) and the fraction of the
HBM roofline.  A "step" is one sampler call over one batch of synthetic
logits already resident in HBM.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Prints one JSON line.  The CPU baselines (the oracle on a bounded sample
of the same rows: single thread, rows serial; and rows split over every
usable core) are timed on this host in the same run.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "sampled rows/s @B=256 V=129280; µs/step @B=1; % of HBM peak BW"

# Passes over row-sized data per step, by row class and kernel shape:
# reads and writes of the logits or of per-logit workspace arrays (4 B per
# logit), each counted once; everything else a row's finish touches is
# O(candidates).  "l2" names the passes whose data was written in the same
# step and is normally re-read from the on-die caches (L2 / the 256 MB
# Infinity Cache) rather than from HBM.
PASSES = {
    "row_kernel (B >= 192 f32, no logprobs; C3)": {
        "top-k <= 256 (incl. min-p, penalties, mask)": {"reads": 1, "writes": 0},
        "other classes, or a fallback (general path, 8192-logit chunks)":
            {"reads": "1 + 1 of s for top-p / temperature-only / top-k > 1024", "writes": "0, or 1 of s",
             "l2": "the s re-read"},
    },
    "select + finish (C1 one launch; C2, C4, C5 two)": {
        "greedy, top-k <= 1024 (C1, C2's greedy half, C4)": {"reads": 1, "writes": 0},
        "top-p without top-k (wide pass; C2, C5)": {
            "reads": "1 (logits) + 1 (s, finish grid) + the refolded chunks' w (a few per row)",
            "writes": "2 (s by the select pass, w by the finish grid)", "l2": "the s and w re-reads"},
        "temperature only, top-k > 1024": {"reads": "1 + 1 of s", "writes": "1 of s", "l2": "the s re-read"},
    },
}


def _dev(torch, x):
    x = np.ascontiguousarray(x)
    if x.dtype == np.uint32:
        x = x.view(np.int32)
    if x.dtype == np.uint16:  # bf16 bit patterns
        return torch.from_numpy(x.view(np.int16)).to("cuda").view(torch.bfloat16)
    return torch.from_numpy(x).to("cuda")


def _prepare(torch, w):
    from hi_amd import sampler as S
    args = dict(
        logits=_dev(torch, w.logits),
        params=S.params_to_device(w.params),
        uniforms=_dev(torch, w.uniforms),
        hist=[_dev(torch, a) for a in (w.hist_offsets, w.hist_ids, w.hist_counts)]
        if w.hist_offsets is not None else [None, None, None],
        mask=_dev(torch, w.mask_words) if w.mask_words is not None else None,
    )
    smp = S.Sampler(w.batch, w.vocab, w.n_logprobs)
    return smp, args


def _step(smp, a, w, out, stream):
    return smp.sample(a["logits"], a["params"], a["uniforms"], *a["hist"], a["mask"],
                      n_logprobs=w.n_logprobs, out=out, stream=stream)


def time_large_batch(torch, w, steps, warmup):
    """K eager steps on one stream, bracketed by two events (the host
    enqueues faster than the GPU runs a C3 step, so the GPU sets the pace).
    A second pass records an event after every step for the p50/p99 spread;
    those events add a few microseconds to each step."""
    smp, a = _prepare(torch, w)
    stream = torch.cuda.Stream()
    out = None
    with torch.cuda.stream(stream):
        for _ in range(max(warmup, 1)):
            out = _step(smp, a, w, out, stream)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        ev0.record(stream)
        for _ in range(steps):
            out = _step(smp, a, w, out, stream)
        ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = ev0.elapsed_time(ev1)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    with torch.cuda.stream(stream):
        evs[0].record(stream)
        for i in range(steps):
            out = _step(smp, a, w, out, stream)
            evs[i + 1].record(stream)
    torch.cuda.synchronize()
    per = np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(steps)])
    return total_ms / steps, per, wall


def time_config(torch, w, steps, warmup, cfg):
    """One of the other configurations (C2, C4, C5): K eager steps of the
    whole pipeline on one stream between two HIP events on that stream, then
    a second pass with an event after every step for the p50 / p99 spread
    (those events add a few microseconds to each step).  Algorithmic bytes
    per step are the workload's input and output bytes, each counted once;
    the fraction is of the 8 TB/s HBM peak.  `roofline` prices the step's
    kernels together (the select pass and the finish grid, two launches):
    the HBM bytes they move per step come from the committed counter
    summary of this configuration when it was measured on this build."""
    smp, a = _prepare(torch, w)
    stream = torch.cuda.Stream()
    out = None
    with torch.cuda.stream(stream):
        for _ in range(max(warmup, 1)):
            out = _step(smp, a, w, out, stream)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        ev0.record(stream)
        for _ in range(steps):
            out = _step(smp, a, w, out, stream)
        ev1.record(stream)
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1000.0 / steps
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    with torch.cuda.stream(stream):
        evs[0].record(stream)
        for i in range(steps):
            out = _step(smp, a, w, out, stream)
            evs[i + 1].record(stream)
    torch.cuda.synchronize()
    per = np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]) * 1000.0
    alg = w.algorithmic_bytes()
    gbs = alg / (us * 1e-6) / 1e9
    traffic, tag = traffic_from_profile(f"config{cfg}_hbm_traffic.md")
    current = traffic is not None and tag == source_hash()
    return {"workload": w.name, "us_per_step": us, "rows_per_s": w.batch / (us * 1e-6),
            "us_per_step_p50_with_step_events": float(np.percentile(per, 50)),
            "us_per_step_p99_with_step_events": float(np.percentile(per, 99)),
            "algorithmic_bytes": alg, "gbs": gbs, "hbm_frac": gbs / HBM_PEAK_GBS,
            "floor_us": alg / (HBM_PEAK_GBS * 1e9) * 1e6,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": traffic if current else None,
                         "traffic_summary": {"file": f"profiles/config{cfg}_hbm_traffic.md", "bytes": traffic,
                                             "source_hash": tag, "matches_this_build": current},
                         "kernels": "the step's launches together (select pass + finish grid)"}}


def time_parts(torch, w, steps):
    """Per-part device time of a step: the library records hipEvents on the
    launch stream before the pass over the logits, between it and the
    finish, and after the finish (hi_rocm_profile_begin / _end)."""
    import ctypes
    from hi_amd import _lib
    lib = _lib.load()
    smp, a = _prepare(torch, w)
    stream = torch.cuda.Stream()
    out = None
    with torch.cuda.stream(stream):
        for _ in range(5):
            out = _step(smp, a, w, out, stream)
    torch.cuda.synchronize()
    _lib.check(lib.hi_rocm_profile_begin(steps))
    with torch.cuda.stream(stream):
        for _ in range(steps):
            out = _step(smp, a, w, out, stream)
    p, f, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int()
    _lib.check(lib.hi_rocm_profile_end(ctypes.byref(p), ctypes.byref(f), ctypes.byref(n)))
    assert n.value == steps, (n.value, steps)
    return p.value * 1000.0 / steps, f.value * 1000.0 / steps


def pmc_probe(torch, w, steps, copy_mib=512):
    """Workload for the rocprofv3 --pmc passes: steps of one configuration,
    then one plain device copy of copy_mib MiB whose FETCH_SIZE / WRITE_SIZE
    calibrate the counters (a copy reads and writes exactly its size)."""
    smp, a = _prepare(torch, w)
    stream = torch.cuda.Stream()
    out = None
    with torch.cuda.stream(stream):
        for _ in range(steps):
            out = _step(smp, a, w, out, stream)
    torch.cuda.synchronize()
    n = copy_mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_probe": w.name, "steps": steps, "copy_bytes": n * 4}))


def source_hash():
    """SHA-256 of the library's HIP sources and headers (hi_amd/csrc, include),
    which identifies the build a counter summary was measured on."""
    import hashlib
    h = hashlib.sha256()
    for d in (os.path.join(ROOT, "hi_amd", "csrc"), os.path.join(ROOT, "include")):
        for name in sorted(os.listdir(d)):
            if name.endswith((".hip", ".h")):
                h.update(name.encode())
                with open(os.path.join(d, name), "rb") as f:
                    h.update(f.read())
    return h.hexdigest()


def traffic_from_profile(name="row_kernel_c3_hbm_traffic.md"):
    """HBM bytes per launch (per step for a configuration summary) from a
    committed rocprofv3 --pmc summary under profiles/ (FETCH_SIZE +
    WRITE_SIZE, scaled by a copy of known size), with the source hash the
    summary was measured on.  Returns (bytes or None, summary hash or None):
    the caller reports the bytes only when the hash is this build's."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None, None
    traffic = tag = None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            traffic = float(line.split(":", 1)[1].strip())
        if line.startswith("source_hash:"):
            tag = line.split(":", 1)[1].strip()
    return traffic, tag


def time_graph_b1(torch, w, steps, warmup):
    """B=1: one hipGraph replay per step (the step has no host sync)."""
    smp, a = _prepare(torch, w)
    stream = torch.cuda.Stream()
    out = None
    with torch.cuda.stream(stream):
        for _ in range(3):
            out = _step(smp, a, w, out, stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        _step(smp, a, w, out, stream)
    torch.cuda.synchronize()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        g.replay()
    ev1.record()
    torch.cuda.synchronize()
    graph_us = ev0.elapsed_time(ev1) * 1000.0 / steps
    # the step's cost inside a larger graph (as in a decode step whose graph
    # also holds the model's forward pass): `inner` steps captured in one
    # graph, so the per-replay launch is spread over them
    inner = 20
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=stream):
        for _ in range(inner):
            _step(smp, a, w, out, stream)
    torch.cuda.synchronize()
    for _ in range(max(1, warmup // inner)):
        g2.replay()
    torch.cuda.synchronize()
    reps = max(1, steps // inner)
    ev0.record()
    for _ in range(reps):
        g2.replay()
    ev1.record()
    torch.cuda.synchronize()
    in_graph_us = ev0.elapsed_time(ev1) * 1000.0 / (reps * inner)
    # eager for comparison (launch overhead included)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for _ in range(steps):
            out = _step(smp, a, w, out, stream)
    torch.cuda.synchronize()
    eager_us = (time.perf_counter() - t0) * 1e6 / steps
    return graph_us, in_graph_us, eager_us


def time_indexer_select(torch, shapes=((1162, 512), (65536, 2048)), launches=200, cpu=True):
    """DSV4 indexer block selection (hi_rocm_launch_dsv4_indexer_select):
    us per launch over back-to-back launches on one stream, bracketed by HIP
    events on that stream.  Algorithmic bytes per launch: n scores f32 read,
    n marks u8 and min(k, n) int32 indices written.  One workgroup up to
    8192 scores, else one per 4096 scores in three kernels: the bound is
    latency (kernel launches and dependent global round trips), not HBM.
    CPU baseline: the host
    selection the reference's CPU path runs, on the same scores."""
    import ctypes
    from hi_amd import _lib
    from hi_amd.workloads import indexer_test_scores
    lib = _lib.load()
    out = []
    stream = torch.cuda.Stream()
    for n, k in shapes:
        x = torch.from_numpy(indexer_test_scores(n) if n <= 4096 else
                             np.random.default_rng(1).standard_normal(n).astype(np.float32)).cuda()
        marks = torch.empty(n, dtype=torch.uint8, device="cuda")
        sel = torch.empty(min(n, k), dtype=torch.int32, device="cuda")
        s = ctypes.c_void_p(stream.cuda_stream)
        args = (x.data_ptr(), n, k, marks.data_ptr(), sel.data_ptr(), s)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for _ in range(20):
                _lib.check(lib.hi_rocm_launch_dsv4_indexer_select(*args))
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(launches):
                _lib.check(lib.hi_rocm_launch_dsv4_indexer_select(*args))
            e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1000.0 / launches
        alg = n * 4 + n + min(n, k) * 4
        rec = {"n_blocks": n, "top_k": k, "us_per_launch": us, "algorithmic_bytes": alg, "gbs": alg / us / 1e3}
        if cpu:
            # the reference's host path (dsv4_cpu.rs:3258-3270: rank by
            # total_cmp, keep the first k, sort the kept indices), restated
            # in C with qsort, one thread
            from oracle import oracle
            oracle.build()
            xs = x.cpu().numpy()
            calls, t0 = 0, time.perf_counter()
            while calls < 3 or time.perf_counter() - t0 < 0.5:
                oracle.indexer_select(xs, k)
                calls += 1
            rec["cpu_baseline"] = {"us_per_call": (time.perf_counter() - t0) / calls * 1e6, "cores": 1,
                                   "kind": "port", "sample": f"{calls} calls on the same scores"}
        out.append(rec)
    return out


def time_router(torch, rows=4096, experts=256, top_k=8, launches=100, cpu=True):
    """MoE router top-k (hi_rocm_launch_moe_topk_router), DeepSeek-V3-style
    sigmoid gating with a selection bias and normalised weights: us per
    launch over back-to-back launches between HIP events on the launch
    stream.  Algorithmic bytes: scores read once, ids and weights written.
    CPU baseline: the oracle's literal restatement of the reference kernel's
    per-row loops (one thread), on a bounded sample of the rows."""
    import ctypes
    from hi_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(3)
    xs = rng.standard_normal((rows, experts)).astype(np.float32)
    bs = (rng.standard_normal(experts) * 0.1).astype(np.float32)
    x, b = torch.from_numpy(xs).cuda(), torch.from_numpy(bs).cuda()
    ids = torch.empty((rows, top_k), dtype=torch.int32, device="cuda")
    w = torch.empty((rows, top_k), dtype=torch.float32, device="cuda")
    stream = torch.cuda.Stream()
    args = (x.data_ptr(), ids.data_ptr(), w.data_ptr(), b.data_ptr(), rows, experts, top_k, 1, 1, 2.5,
            ctypes.c_void_p(stream.cuda_stream))
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(10):
            _lib.check(lib.hi_rocm_launch_moe_topk_router(*args))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(launches):
            _lib.check(lib.hi_rocm_launch_moe_topk_router(*args))
        e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / launches
    alg = rows * experts * 4 + experts * 4 + rows * top_k * 8
    rec = {"rows": rows, "experts": experts, "top_k": top_k, "gating": "sigmoid+bias, normalised",
           "us_per_launch": us, "rows_per_s": rows / (us * 1e-6), "algorithmic_bytes": alg, "gbs": alg / us / 1e3}
    if cpu:
        from oracle import oracle
        oracle.build()
        n, t0 = 0, time.perf_counter()
        while n < rows and (n < 64 or time.perf_counter() - t0 < 1.0):
            oracle.moe_router(xs[n:n + 64], top_k, bias=bs, norm_topk=True, gating_sigmoid=True, weights_scale=2.5)
            n += 64
        dt = time.perf_counter() - t0
        rec["cpu_baseline"] = {"rows_per_s": n / dt, "cores": 1, "kind": "port",
                               "sample": f"{n} of the {rows} rows"}
    return rec


def time_lm_head(torch, B=32, H=4096, V=151936, cap=30.0, launches=10, rounds=6):
    """The LM-head projection + softcap fused into the sampler's first pass
    (hi_rocm_sample_lm_head) against the unfused pair (hi_rocm_lm_head_logits
    writing the logits, then hi_rocm_sample on them), both timed by HIP events
    on the launch stream over back-to-back calls, in alternating rounds (the
    median round of each is reported: the box's HBM throughput drifts by a
    few percent between rounds).  Rows: top-k 40, top-p 0.9, T 0.8; the
    fused and unfused paths are also timed with greedy rows, and the projection alone
    (hi_rocm_lm_head_logits, the logits written).  Algorithmic bytes per call:
    the bf16 weight V*H*2 and hidden B*H*2 read, tokens written (the
    projection reads every weight once)."""
    import ctypes
    from hi_amd import _lib
    from hi_amd import sampler as S
    lib = _lib.load()
    g = torch.Generator(device="cpu").manual_seed(5)
    h = (torch.randn((B, H), generator=g)).to(torch.bfloat16).cuda()
    w = (torch.randn((V, H), device="cuda") * (1.0 / H ** 0.5)).to(torch.bfloat16)
    params = np.zeros(B, _lib.ROW_PARAMS_DTYPE)
    params["temperature"] = 0.8
    params["top_p"] = 0.9
    params["top_k"] = 40
    dp = S.params_to_device(params)
    params["temperature"] = 0.0
    dg = S.params_to_device(params)
    du = torch.from_numpy(np.random.default_rng(6).random(B).astype(np.float32)).cuda()
    n = ctypes.c_size_t()
    _lib.check(lib.hi_rocm_lm_head_workspace_bytes(B, V, ctypes.byref(n)))
    ws = torch.zeros(n.value, dtype=torch.uint8, device="cuda")
    tok = torch.empty(B, dtype=torch.int32, device="cuda")
    logits = torch.empty((B, V), dtype=torch.float32, device="cuda")
    smp = S.Sampler(B, V, 0)
    stream = torch.cuda.Stream()
    s = ctypes.c_void_p(stream.cuda_stream)

    def fused(params_dev):
        _lib.check(lib.hi_rocm_sample_lm_head(h.data_ptr(), w.data_ptr(), None, cap, B, H, V, params_dev.data_ptr(),
                                              du.data_ptr(), tok.data_ptr(), ws.data_ptr(), n.value, s))

    def unfused(params_dev):
        _lib.check(lib.hi_rocm_lm_head_logits(h.data_ptr(), w.data_ptr(), None, cap, B, H, V, logits.data_ptr(), s))
        smp.sample(logits, params_dev, du, out={"tokens": tok}, stream=stream)

    def twin():
        _lib.check(lib.hi_rocm_lm_head_logits(h.data_ptr(), w.data_ptr(), None, cap, B, H, V, logits.data_ptr(), s))

    cases = (("fused", lambda: fused(dp)), ("unfused", lambda: unfused(dp)), ("fused_greedy", lambda: fused(dg)),
             ("unfused_greedy", lambda: unfused(dg)), ("projection", twin))
    times = {name: [] for name, _ in cases}
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _, fn in cases:
            for _ in range(3):
                fn()
    for _ in range(rounds):
        for name, fn in cases:
            with torch.cuda.stream(stream):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(launches):
                    fn()
                e1.record(stream)
            e1.synchronize()
            times[name].append(e0.elapsed_time(e1) * 1000.0 / launches)
    res = {"batch": B, "hidden": H, "vocab": V, "softcap": cap, "rows": "top-k 40, top-p 0.9, T 0.8"}
    for name, v in times.items():
        res[f"{name}_us"] = round(float(np.median(v)), 2)
    alg = V * H * 2 + B * H * 2 + B * 4
    res["algorithmic_bytes"] = alg
    res["fused_gbs"] = round(alg / res["fused_us"] / 1e3, 1)
    res["fused_hbm_frac"] = round(res["fused_gbs"] / HBM_PEAK_GBS, 4)
    res["projection_gbs"] = round(alg / res["projection_us"] / 1e3, 1)
    res["projection_hbm_frac"] = round(res["projection_gbs"] / HBM_PEAK_GBS, 4)
    return res


def cpu_baseline(w, budget_s=15.0):
    """The oracle (a C restatement of the reference CPU sampler plus the
    extension stages), single thread, rows processed serially like the
    reference's host loop.  Bounded sample: rows of the same workload until
    the time budget is used."""
    from oracle import oracle
    oracle.build()
    B = w.batch
    rows_done = 0
    t0 = time.perf_counter()
    b = 0
    while time.perf_counter() - t0 < budget_s:
        sel = slice(b, b + 1)
        h = None
        if w.hist_offsets is not None:
            h0, h1 = int(w.hist_offsets[b]), int(w.hist_offsets[b + 1])
            h = (np.array([0, h1 - h0], np.uint32), w.hist_ids[h0:h1], w.hist_counts[h0:h1])
        oracle.sample_rows(w.logits[sel], w.params[sel], w.uniforms[sel],
                           *(h if h else (None, None, None)),
                           None if w.mask_words is None else w.mask_words[sel],
                           w.n_logprobs, threads=1)
        rows_done += 1
        b = (b + 1) % B
    el = time.perf_counter() - t0
    return {"value": rows_done / el, "unit": "rows/s", "cores": 1, "kind": "port",
            "sample": f"{rows_done} rows of {w.name} (oracle, 1 thread, serial rows), {el:.1f} s",
            **host_cpu()}


def host_cpu():
    """The host's CPU model and C library, for the CPU baselines' record
    (the oracle's expf is the host glibc's)."""
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        libc = os.confstr("CS_GNU_LIBC_VERSION")
    except (ValueError, OSError):
        libc = None
    return {"cpu_model": model, "libc": libc}


def host_cores():
    """Cores this process may use: its CPU affinity, capped by
    OMP_NUM_THREADS where the environment sets it."""
    n = len(os.sched_getaffinity(0))
    try:
        n = min(n, int(os.environ.get("OMP_NUM_THREADS", n)))
    except ValueError:
        pass
    return max(1, n)


def cpu_baseline_all_cores(w, budget_s=8.0):
    """The same oracle with the batch's rows split over every usable core
    (the second CPU figure of the measurement plan): whole batches until the
    time budget is used."""
    from oracle import oracle
    oracle.build()
    cores = host_cores()
    rows_done = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        oracle.sample_rows(w.logits, w.params, w.uniforms, w.hist_offsets, w.hist_ids, w.hist_counts,
                           w.mask_words, w.n_logprobs, threads=cores)
        rows_done += w.batch
    el = time.perf_counter() - t0
    return {"value": rows_done / el, "unit": "rows/s", "cores": cores, "kind": "port",
            "sample": f"{rows_done} rows of {w.name} (oracle, rows split over {cores} threads), {el:.1f} s",
            **host_cpu()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--pmc-probe", action="store_true",
                    help="run C3 steps then a plain copy of known size, for rocprofv3 --pmc")
    ap.add_argument("--pmc-config", type=int, choices=(1, 2, 3, 4, 5),
                    help="the same probe with configuration N's steps")
    ap.add_argument("--lm-head-only", action="store_true",
                    help="time only the LM-head projection, fused and unfused (for rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}): the sampler's rows are "
              "independent, so a multi-GPU run is data-parallel over the batch and scales by "
              "construction; see DESIGN.md for how the path would shard.", file=sys.stderr)
        sys.exit(2)

    import torch
    from hi_amd.workloads import config1, config3

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.lm_head_only:
        print(json.dumps({"lm_head_fused": time_lm_head(torch),
                          "lm_head_fused_b64": time_lm_head(torch, B=64, rounds=3)}))
        return
    if args.pmc_config:
        from hi_amd.workloads import CONFIGS
        pmc_probe(torch, CONFIGS[args.pmc_config](), args.steps)
        return
    w3 = config3()
    if args.pmc_probe:
        pmc_probe(torch, w3, args.steps)
        return
    ms, per, wall = time_large_batch(torch, w3, args.steps, args.warmup)
    rows_per_s = w3.batch / (ms / 1000.0)
    alg_bytes = w3.algorithmic_bytes()
    achieved = alg_bytes / (ms / 1000.0) / 1e9
    pass_us, _ = time_parts(torch, w3, args.steps)
    w1 = config1()
    b1_graph_us, b1_in_graph_us, b1_eager_us = time_graph_b1(torch, w1, max(args.steps, 100), 20)
    b1_pass_us, _ = time_parts(torch, w1, max(args.steps, 100))
    # the dominant kernel of the C3 step: at B >= 192 (no logprobs) the step
    # is one row_kernel launch, which reads every algorithmic byte and also
    # finishes the rows.  Its average duration is the timed region's (K
    # launches back to back on one stream between two events); the
    # library's own events around single launches (pass_us) add their own
    # overhead and are reported beside it.
    kernel_us = ms * 1000.0
    kernel_gbs = alg_bytes / (kernel_us * 1e-6) / 1e9
    traffic, traffic_tag = traffic_from_profile()
    traffic_current = traffic is not None and traffic_tag == source_hash()

    res = {
        "metric": METRIC,
        "value": rows_per_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": w3.name, "batch": w3.batch, "vocab": w3.vocab,
                   "logits": "f32 N(0,2.5^2) + 16 spikes/row", "top_k": "{20,50,100}",
                   "top_p": "[0.8,0.99]", "min_p": 0.05, "frequency_penalty": 0.2,
                   "presence_penalty": 0.3, "history": "2048 Zipf ids/row"},
        "timing": "K eager steps on one stream between two events",
        "us_per_step_p50_with_step_events": float(np.percentile(per, 50) * 1000),
        "us_per_step_p99_with_step_events": float(np.percentile(per, 99) * 1000),
        "b1_us_per_step_graph": b1_graph_us,
        "b1_us_per_step_in_graph": b1_in_graph_us,
        "b1_us_per_step_eager": b1_eager_us,
        "b1_workload": w1.name,
        # C1 runs as one fused launch (select_finish_kernel): the library's
        # first event interval is that launch, the second holds no kernel
        "b1_kernel_us": {"select_finish_kernel": b1_pass_us},
        "step_hbm_fraction": achieved / HBM_PEAK_GBS,
        # one row_kernel launch per C3 step; the library's third event follows
        # the second directly there, so only the first interval is a kernel
        "step_kernel_us": {"row_kernel": pass_us},
        "roofline": {"bound": "hbm", "achieved": kernel_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": kernel_gbs / HBM_PEAK_GBS, "traffic": traffic if traffic_current else None,
                     "traffic_summary": {"file": "profiles/row_kernel_c3_hbm_traffic.md", "bytes": traffic,
                                         "source_hash": traffic_tag, "matches_this_build": traffic_current},
                     "kernel": "hi_rocm::row_kernel<false> (C3: one workgroup per row, whole step)",
                     "kernel_avg_us": kernel_us,
                     "kernel_avg_us_library_events": pass_us,
                     "algorithmic_bytes_per_launch": alg_bytes},
    }
    from hi_amd.workloads import config2, config4, config5
    res["other_configs"] = {f"c{i}": time_config(torch, mk(), args.steps, args.warmup, i)
                            for i, mk in ((2, config2), (4, config4), (5, config5))}
    res["passes"] = PASSES
    res["dsv4_indexer_select"] = time_indexer_select(torch, cpu=not args.no_cpu_baseline)
    res["moe_router"] = time_router(torch, cpu=not args.no_cpu_baseline)
    res["lm_head_fused"] = time_lm_head(torch)
    res["lm_head_fused_b64"] = time_lm_head(torch, B=64, rounds=3)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(w3, args.cpu_budget)
        res["cpu_baseline_all_cores"] = cpu_baseline_all_cores(w3)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
