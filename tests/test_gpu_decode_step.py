"""GPU checks of the decode-step upkeep kernels against the restatement in
oracle/decode_step_oracle.py:

* hi_rocm_history_append / _pack over a prompt seeding and several decode
  steps (duplicates, a slot reset, a slot overflow), eagerly and replayed
  from a captured graph; the packed CSR then drives hi_rocm_sample's
  penalties and the tokens equal the sampler oracle's on the host-built CSR;
* hi_rocm_rng_uniforms over 40 steps (crossing ChaCha block boundaries),
  with greedy requests drawing nothing.
"""
import ctypes

import numpy as np
import pytest

from oracle import decode_step_oracle as D

pytestmark = pytest.mark.gpu


def _t(torch, a, dtype=None):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    if a.dtype == np.uint64:
        a = a.view(np.int64)
    return torch.from_numpy(a).to("cuda")


class DevHistory:
    def __init__(self, torch, lib, hip, batch, cap):
        self.torch, self.lib, self.hip = torch, lib, hip
        self.B, self.cap = batch, cap
        z = lambda n: torch.zeros(n, dtype=torch.int32, device="cuda")
        self.ids, self.cnt, self.lens = z(batch * cap), z(batch * cap), z(batch)
        self.overflow = z(1)
        self.offsets, self.hids, self.hcnt = z(batch + 1), z(batch * cap), z(batch * cap)

    def append(self, rows, tokens, n, stream):
        self.hip.check(self.lib.hi_rocm_history_append(
            self.ids.data_ptr(), self.cnt.data_ptr(), self.lens.data_ptr(), self.B, self.cap,
            0 if rows is None else rows.data_ptr(), tokens.data_ptr(), n, self.overflow.data_ptr(),
            stream.cuda_stream))

    def pack(self, stream):
        self.hip.check(self.lib.hi_rocm_history_pack(
            self.ids.data_ptr(), self.cnt.data_ptr(), self.lens.data_ptr(), self.B, self.cap,
            self.offsets.data_ptr(), self.hids.data_ptr(), self.hcnt.data_ptr(), stream.cuda_stream))

    def read(self):
        off = self.offsets.cpu().numpy().view(np.uint32)
        n = int(off[-1])
        return (off.tolist(), self.hids[:n].cpu().numpy().view(np.uint32).tolist(),
                self.hcnt[:n].cpu().numpy().view(np.uint32).tolist(), int(self.overflow.item()))


def test_history_append_pack_and_penalised_sampling(hip, oracle):
    import torch
    from hi_amd import sampler as S
    from hi_amd._lib import ROW_PARAMS_DTYPE
    lib = hip.load()
    stream = torch.cuda.Stream()
    rng = np.random.default_rng(77)
    B, cap, V = 6, 48, 5000
    dh = DevHistory(torch, lib, hip, B, cap)
    ref = D.History(B, cap)
    # prompt seeding: (slot, token) pairs, small vocabulary (repeats), slot 5
    # gets more distinct ids than it can hold
    rows, toks = [], []
    for r in range(B):
        n = int(rng.integers(0, 60))
        t = rng.integers(0, 40, n) if r != 5 else np.arange(1000, 1000 + 60)
        rows += [r] * len(t)
        toks += [int(x) for x in t]
    rows += [-1, B + 3]
    toks += [1, 2]  # skipped: no such slot
    print(f"history prompt pairs={len(rows)}", flush=True)
    rt, tt = _t(torch, np.array(rows, np.int32)), _t(torch, np.array(toks, np.uint32))
    torch.cuda.synchronize()
    dh.append(rt, tt, len(rows), stream)
    dh.pack(stream)
    stream.synchronize()
    ref.append(rows, toks)
    assert dh.read() == (*ref.csr(), ref.overflow)
    # decode steps: one token per slot (no rows array), a reset at step 4
    params = np.zeros(B, ROW_PARAMS_DTYPE)
    params["temperature"] = 0.9
    params["top_p"] = np.inf
    params["top_k"] = 50
    params["repetition_penalty"] = 1.3
    params["frequency_penalty"] = 0.25
    params["presence_penalty"] = 0.5
    dparams = S.params_to_device(params)
    smp = S.Sampler(B, V, 0)
    for step in range(8):
        if step == 4:
            rr, rtok = [2, 2], [D.RESET, 17]
            torch.cuda.synchronize()
            dh.append(_t(torch, np.array(rr, np.int32)), _t(torch, np.array(rtok, np.uint32)), 2, stream)
            dh.pack(stream)
            ref.append(rr, rtok)
        logits = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
        logits[:, :40] += 3.0  # the history tokens compete
        u = rng.random(B).astype(np.float32)
        offsets, ids, counts = ref.csr()
        want = oracle.sample_rows(logits, params, u, np.array(offsets, np.uint32), np.array(ids, np.uint32),
                                  np.array(counts, np.uint32))["tokens"]
        dl, du = _t(torch, logits), _t(torch, u)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            out = smp.sample(dl, dparams, du, dh.offsets, dh.hids, dh.hcnt, stream=stream)
            dh.append(None, out["tokens"], B, stream)
            dh.pack(stream)
        stream.synchronize()
        got = out["tokens"].cpu().numpy().view(np.uint32)
        print(f"history step {step} tokens={got.tolist()}", flush=True)
        assert np.array_equal(got, want), (step, got, want)
        ref.append(list(range(B)), [int(x) for x in got])
        assert dh.read() == (*ref.csr(), ref.overflow), step


def test_history_graph_replays(hip):
    import torch
    lib = hip.load()
    B, cap = 5, 16
    dh = DevHistory(torch, lib, hip, B, cap)
    ref = D.History(B, cap)
    tokens = torch.zeros(B, dtype=torch.int32, device="cuda")
    rng = np.random.default_rng(5)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        dh.append(None, tokens, B, torch.cuda.current_stream())
        dh.pack(torch.cuda.current_stream())
    torch.cuda.synchronize()
    # capture does not run the kernels
    assert int(dh.lens.sum().item()) == 0
    for rep in range(6):
        t = rng.integers(0, 12, B).astype(np.uint32)
        tokens.copy_(torch.from_numpy(t.view(np.int32)))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref.append(list(range(B)), [int(x) for x in t])
        assert dh.read() == (*ref.csr(), ref.overflow), rep


def test_rng_uniforms_match_stdrng(hip):
    import torch
    lib = hip.load()
    seeds = [0, 1, 0x2503_01, 2**63 + 5, 42, 7]
    sampled = np.array([1, 0, 1, 1, 0, 1], np.uint8)
    B = len(seeds)
    keys = np.zeros((B, 8), np.uint32)
    for b, s in enumerate(seeds):
        k = (ctypes.c_uint32 * 8)()
        hip.check(lib.hi_rocm_rng_key_from_seed(ctypes.c_uint64(s), k))
        keys[b] = list(k)
        assert keys[b].tolist() == D.stdrng_key_from_seed(s)
    rngs = [D.StdRng(keys[b]) for b in range(B)]
    raw = [D.StdRng(keys[b]) for b in range(B)]  # the keystream words themselves
    dk = _t(torch, keys.reshape(-1))
    used = torch.zeros(B, dtype=torch.int64, device="cuda")
    used[3] = (1 << 32) * 16 - 2  # crosses the low counter word within the run
    rngs[3] = D.StdRng(keys[3], words_used=(1 << 32) * 16 - 2)
    raw[3] = D.StdRng(keys[3], words_used=(1 << 32) * 16 - 2)
    ds = torch.from_numpy(sampled).to("cuda")
    out = torch.zeros(B, dtype=torch.float32, device="cuda")
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    for step in range(40):
        hip.check(lib.hi_rocm_rng_uniforms(dk.data_ptr(), used.data_ptr(), ds.data_ptr(), out.data_ptr(), B,
                                           stream.cuda_stream))
        stream.synchronize()
        got = out.cpu().numpy()
        want = np.array([rngs[b].uniform_f32() if sampled[b] else 0.0 for b in range(B)], np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (step, got, want)
        # the closed form of gen_range(0.0f32..1.0f32) on the device's values:
        # u * 2^23 is the integer (w >> 9) of the next keystream word w (the
        # ChaCha12 core is pinned by RFC 8439's vectors), so 0 <= u < 1
        for b in range(B):
            if sampled[b]:
                w = raw[b].next_u32()
                assert float(got[b]) * float(1 << 23) == float(w >> 9) and 0.0 <= got[b] < 1.0, (step, b)
    u = used.cpu().numpy()
    assert u[1] == 0 and u[0] == 40 and u[3] == (1 << 32) * 16 - 2 + 40


def test_decode_step_graph_loop(hip, oracle):
    """A whole decode step's upkeep captured once and replayed: uniforms from
    each request's StdRng, the sampler on the packed history, the sampled
    tokens appended, the history packed, and the next step's token and
    position inputs written from the samples (hi_rocm_decode_step_advance,
    the device form of upload_batch_graph_inputs).  Between replays only the
    logits change, as a forward pass would write them; every replay must
    equal the host chain: StdRng uniforms, the oracle on the host-built
    history, the host history and the reference's pad-row rule."""
    import torch
    from hi_amd import sampler as S
    from hi_amd._lib import ROW_PARAMS_DTYPE
    lib = hip.load()
    rng = np.random.default_rng(91)
    B, n_active, cap, V = 6, 5, 64, 3000
    seeds = [11, 12, 13, 14, 15, 0]
    sampled = np.array([1, 1, 0, 1, 1, 0], np.uint8)  # request 2 greedy, row 5 a pad row
    keys = np.zeros((B, 8), np.uint32)
    for b, sd in enumerate(seeds):
        k = (ctypes.c_uint32 * 8)()
        hip.check(lib.hi_rocm_rng_key_from_seed(ctypes.c_uint64(sd), k))
        keys[b] = list(k)
    rngs = [D.StdRng(keys[b]) for b in range(B)]
    params = np.zeros(B, ROW_PARAMS_DTYPE)
    params["temperature"] = np.where(sampled == 1, 0.85, 0.0)
    params["top_p"] = 0.95
    params["top_k"] = 40
    params["repetition_penalty"] = 1.2
    params["frequency_penalty"] = 0.3
    params["presence_penalty"] = 0.2
    dparams = S.params_to_device(params)
    dh = DevHistory(torch, lib, hip, B, cap)
    ref = D.History(B, cap)
    prompt_rows, prompt_toks = [], []
    for r in range(n_active):
        t = rng.integers(0, 60, int(rng.integers(3, 20)))
        prompt_rows += [r] * len(t)
        prompt_toks += [int(x) for x in t]
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    dh.append(_t(torch, np.array(prompt_rows, np.int32)), _t(torch, np.array(prompt_toks, np.uint32)),
              len(prompt_rows), stream)
    dh.pack(stream)
    stream.synchronize()
    ref.append(prompt_rows, prompt_toks)
    dk = _t(torch, keys.reshape(-1))
    used = torch.zeros(B, dtype=torch.int64, device="cuda")
    ds = torch.from_numpy(sampled).to("cuda")
    unif = torch.zeros(B, dtype=torch.float32, device="cuda")
    logits = torch.zeros((B, V), dtype=torch.float32, device="cuda")
    tokens = _t(torch, np.array([7, 8, 9, 10, 11, 0], np.uint32))
    pos0 = np.array([20, 31, 5, 17, 3, 0], np.uint32)
    positions = _t(torch, pos0)
    smp = S.Sampler(B, V, 0)
    with torch.cuda.stream(stream):
        out = smp.sample(logits, dparams, unif, dh.offsets, dh.hids, dh.hcnt, stream=stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        cs = torch.cuda.current_stream()
        hip.check(lib.hi_rocm_rng_uniforms(dk.data_ptr(), used.data_ptr(), ds.data_ptr(), unif.data_ptr(), B,
                                           cs.cuda_stream))
        smp.sample(logits, dparams, unif, dh.offsets, dh.hids, dh.hcnt, out=out, stream=cs)
        dh.append(None, out["tokens"], n_active, cs)
        dh.pack(cs)
        hip.check(lib.hi_rocm_decode_step_advance(out["tokens"].data_ptr(), tokens.data_ptr(),
                                                  positions.data_ptr(), n_active, B, cs.cuda_stream))
    torch.cuda.synchronize()
    # capture runs nothing
    assert int(used.sum().item()) == 0
    want_pos = pos0.astype(np.int64).copy()
    for step in range(6):
        lg = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
        lg[:, :60] += 2.5  # the history tokens compete
        logits.copy_(torch.from_numpy(lg))
        torch.cuda.synchronize()
        u = np.array([rngs[b].uniform_f32() if sampled[b] else 0.0 for b in range(B)], np.float32)
        offsets, ids, counts = ref.csr()
        want = oracle.sample_rows(lg, params, u, np.array(offsets, np.uint32), np.array(ids, np.uint32),
                                  np.array(counts, np.uint32))["tokens"]
        print(f"decode-step graph replay {step}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(unif.cpu().numpy().view(np.uint32), u.view(np.uint32)), step
        got = out["tokens"].cpu().numpy().view(np.uint32)
        assert np.array_equal(got, want), (step, got, want)
        ref.append(list(range(n_active)), [int(x) for x in got[:n_active]])
        assert dh.read() == (*ref.csr(), ref.overflow), step
        want_pos[:n_active] += 1
        want_pos[n_active:] = 0
        want_tok = np.concatenate([want[:n_active], np.zeros(B - n_active, np.uint32)])
        assert np.array_equal(tokens.cpu().numpy().view(np.uint32), want_tok), step
        assert np.array_equal(positions.cpu().numpy().view(np.uint32), want_pos.astype(np.uint32)), step
