"""GPU checks of the LM-head projection fused into the sampler's first pass
(hi_rocm_sample_lm_head; reference gpu.rs:20999-21009 + the softcap of
gpu.rs:23232-23249 + the sampler).

* The unfused twin (hi_rocm_lm_head_logits) against a float64 product of
  the same bf16 operands, with bias and softcap: this checks the MFMA
  operand layout and the epilogue (tolerance: f32 accumulation, 1e-5 of
  the magnitude sum, and the softcap's tanh to 2e-6).
* The fused tokens against the sampler oracle run on the twin's logits,
  row by row, bit-exact, for every row: greedy and top-k <= 64 rows in the
  fused finish, rows of other classes (top-p only, temperature only,
  top-k above 64) and cuts between distinct logits of equal weight through
  the general per-row path over the workspace's copy of the row.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32 = np.float32


def _bf16(torch, shape, scale, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)
    return x.cuda(), x.float().numpy().astype(np.float64)


def _twin(hip, torch, h, w, bias, cap, B, H, V):
    lib = hip.load()
    out = torch.zeros((B, V), dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    hip.check(lib.hi_rocm_lm_head_logits(h.data_ptr(), w.data_ptr(), 0 if bias is None else bias.data_ptr(),
                                         cap, B, H, V, out.data_ptr(), s.cuda_stream))
    s.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("B,H,V,cap", [(5, 64, 2000, 0.0), (32, 256, 3001, 5.0), (17, 4096, 1024, 30.0),
                                       (9, 96, 777, 2.0), (48, 256, 3001, 5.0), (64, 160, 1500, 0.0)])
def test_twin_logits_match_float64(hip, B, H, V, cap):
    import torch
    h, hn = _bf16(torch, (B, H), 1.0, 1)
    w, wn = _bf16(torch, (V, H), 1.0 / np.sqrt(H), 2)
    bn = (np.random.default_rng(3).standard_normal(V) * 0.5).astype(F32)
    bias = torch.from_numpy(bn).cuda()
    print(f"lm head twin B={B} H={H} V={V} cap={cap}", flush=True)
    got = _twin(hip, torch, h, w, bias, cap, B, H, V).astype(np.float64)
    acc = hn @ wn.T
    mag = np.abs(hn) @ np.abs(wn).T
    pre = acc + bn
    if cap > 0:
        want = cap * np.tanh(pre / cap)
        # d(cap tanh(x/cap))/dx <= 1: the accumulation error carries through
        tol = 1e-5 * mag + 2e-6 * np.abs(want) + 1e-6
    else:
        want = pre
        tol = 1e-5 * mag + 1e-6
    bad = np.abs(got - want) > tol
    assert not bad.any(), (np.argwhere(bad)[:5], got[bad][:5], want[bad][:5])


# (32, 512, 50000): more tiles than k (the tile-top bound); (20, 96, 3000):
# fewer tiles than most k (every tile scanned) and a trailing 32-wide K
# block; (8, 64, 50): one tile shorter than k; (64, 512, 20000) and
# (40, 96, 5000): two row groups of 32 per tile.
@pytest.mark.parametrize("B,H,V,cap,seed", [(32, 512, 50000, 8.0, 11), (20, 96, 3000, 0.0, 21), (8, 64, 50, 3.0, 31),
                                            (64, 512, 20000, 8.0, 61), (40, 96, 5000, 2.0, 71)])
def test_fused_tokens_match_oracle_on_twin_logits(hip, oracle, B, H, V, cap, seed):
    import torch
    from hi_amd import sampler as S
    from hi_amd._lib import ROW_PARAMS_DTYPE
    lib = hip.load()
    print(f"lm head fused B={B} H={H} V={V} cap={cap}", flush=True)
    h, _ = _bf16(torch, (B, H), 1.0, seed)
    w, _ = _bf16(torch, (V, H), 3.0 / np.sqrt(H), seed + 1)
    bias = torch.from_numpy((np.random.default_rng(seed + 2).standard_normal(V) * 0.3).astype(F32)).cuda()
    logits = _twin(hip, torch, h, w, bias, cap, B, H, V)
    rng = np.random.default_rng(seed + 3)
    params = np.zeros(B, ROW_PARAMS_DTYPE)
    params["temperature"] = rng.uniform(0.5, 1.3, B)
    params["top_p"] = rng.choice(np.array([1.0, 0.9, 0.5], F32), B)
    params["top_k"] = rng.choice(np.array([1, 5, 20, 40, 64], np.int32), B)
    params["min_p"] = np.where(rng.random(B) < 0.3, F32(0.05), F32(0.0))
    params["temperature"][:4] = 0.0           # greedy
    # rows the fused finish does not take: the general per-row path
    params["top_k"][4] = 0                     # top-p only
    params["top_p"][4] = 0.9
    params["top_k"][5], params["top_p"][5], params["min_p"][5] = 0, 1.0, 0.0  # temperature only
    params["top_k"][6] = 100                   # top-k above the fused finish's 64
    params["top_k"][7], params["top_p"][7] = 300, 0.8
    u = rng.random(B).astype(F32)
    want = oracle.sample_rows(logits, params, u)["tokens"]
    ws_n = ctypes.c_size_t()
    hip.check(lib.hi_rocm_lm_head_workspace_bytes(B, V, ctypes.byref(ws_n)))
    ws = torch.zeros(ws_n.value, dtype=torch.uint8, device="cuda")
    dp = S.params_to_device(params)
    du = torch.from_numpy(u).cuda()
    out = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    for rep in range(2):
        hip.check(lib.hi_rocm_sample_lm_head(h.data_ptr(), w.data_ptr(), bias.data_ptr(), cap, B, H, V,
                                             dp.data_ptr(), du.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                             ws_n.value, s.cuda_stream))
        s.synchronize()
        got = out.cpu().numpy().view(np.uint32)
        print(f"lm head fused rep {rep}: {got[:8].tolist()}", flush=True)
        assert np.array_equal(got, want), (np.flatnonzero(got != want)[:8])


def test_fused_duplicate_vocabulary_rows(hip, oracle):
    """Every weight row repeated 48 times in a row: tiles of ties, where no
    logit threshold keeps between k and 64 keys (top-k 50 and 64 take the
    exact one-wave select), and top-k cuts inside a run of equal logits (the
    finish resolves them by index, as the reference's (weight, index) rank
    does).  A cut whose next lower logit key weighs the same (small |l/T|,
    or T > 1) goes through the general per-row path: every row gets the
    oracle's token."""
    import torch
    from hi_amd import sampler as S
    from hi_amd._lib import ROW_PARAMS_DTYPE
    lib = hip.load()
    B, H, V, cap = 12, 128, 6000, 4.0
    g = torch.Generator(device="cpu").manual_seed(41)
    base = (torch.randn(((V + 47) // 48, H), generator=g) * (2.0 / np.sqrt(H))).to(torch.bfloat16)
    w = base.repeat_interleave(48, dim=0)[:V].contiguous().cuda()
    h = torch.randn((B, H), generator=g).to(torch.bfloat16).cuda()
    logits = _twin(hip, torch, h, w, None, cap, B, H, V)
    rng = np.random.default_rng(42)
    params = np.zeros(B, ROW_PARAMS_DTYPE)
    params["temperature"] = rng.uniform(0.55, 1.0, B)
    params["temperature"][-3:] = [1.3, 1.7, 2.5]
    params["top_p"] = 1.0
    params["top_k"] = np.array([50, 64, 40, 5, 64, 50, 1, 20, 64, 50, 33, 48], np.int32)
    params["temperature"][0] = 0.0
    u = rng.random(B).astype(F32)
    want = oracle.sample_rows(logits, params, u)["tokens"]
    ws_n = ctypes.c_size_t()
    hip.check(lib.hi_rocm_lm_head_workspace_bytes(B, V, ctypes.byref(ws_n)))
    ws = torch.zeros(ws_n.value, dtype=torch.uint8, device="cuda")
    dp = S.params_to_device(params)
    du = torch.from_numpy(u).cuda()
    out = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    print(f"lm head fused duplicate rows B={B} H={H} V={V}", flush=True)
    torch.cuda.synchronize()
    hip.check(lib.hi_rocm_sample_lm_head(h.data_ptr(), w.data_ptr(), None, cap, B, H, V, dp.data_ptr(),
                                         du.data_ptr(), out.data_ptr(), ws.data_ptr(), ws_n.value, s.cuda_stream))
    s.synchronize()
    got = out.cpu().numpy().view(np.uint32)
    print(f"got {got.tolist()}\nwant {want.tolist()}", flush=True)
    assert np.array_equal(got, want), np.flatnonzero(got != want)


def test_fused_clustered_tiles(hip, oracle):
    """Weight rows equal to one of 400 base rows per 128-column tile plus 1%
    noise: every column of a high tile outranks the low tiles, so the
    tiles kept by the tile-top bound hold far more than 4096 keys above it
    and the finish selects over global memory."""
    import torch
    from hi_amd import sampler as S
    from hi_amd._lib import ROW_PARAMS_DTYPE
    lib = hip.load()
    B, H, V, cap = 8, 64, 128 * 400, 0.0
    g = torch.Generator(device="cpu").manual_seed(51)
    base = torch.randn((400, H), generator=g) * (2.0 / np.sqrt(H))
    w = (base.repeat_interleave(128, dim=0) + 0.01 * torch.randn((V, H), generator=g)).to(torch.bfloat16).cuda()
    h = torch.randn((B, H), generator=g).to(torch.bfloat16).cuda()
    logits = _twin(hip, torch, h, w, None, cap, B, H, V)
    rng = np.random.default_rng(52)
    params = np.zeros(B, ROW_PARAMS_DTYPE)
    params["temperature"] = rng.uniform(0.6, 1.0, B)
    params["top_p"] = 1.0
    params["top_k"] = np.array([64, 64, 40, 64, 50, 64, 1, 64], np.int32)
    u = rng.random(B).astype(F32)
    want = oracle.sample_rows(logits, params, u)["tokens"]
    ws_n = ctypes.c_size_t()
    hip.check(lib.hi_rocm_lm_head_workspace_bytes(B, V, ctypes.byref(ws_n)))
    ws = torch.zeros(ws_n.value, dtype=torch.uint8, device="cuda")
    dp = S.params_to_device(params)
    du = torch.from_numpy(u).cuda()
    out = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    print(f"lm head fused clustered tiles B={B} H={H} V={V}", flush=True)
    torch.cuda.synchronize()
    hip.check(lib.hi_rocm_sample_lm_head(h.data_ptr(), w.data_ptr(), None, cap, B, H, V, dp.data_ptr(),
                                         du.data_ptr(), out.data_ptr(), ws.data_ptr(), ws_n.value, s.cuda_stream))
    s.synchronize()
    got = out.cpu().numpy().view(np.uint32)
    print(f"got {got.tolist()}\nwant {want.tolist()}", flush=True)
    assert np.array_equal(got, want)


def test_twin_rows_do_not_depend_on_the_batch(hip):
    """A row's logits are the same bits whether the call has one row group
    (20 rows) or two (40 rows, the first 20 the same)."""
    import torch
    H, V, cap = 256, 2500, 6.0
    h, _ = _bf16(torch, (40, H), 1.0, 81)
    w, _ = _bf16(torch, (V, H), 1.0 / np.sqrt(H), 82)
    bias = torch.from_numpy((np.random.default_rng(83).standard_normal(V) * 0.5).astype(F32)).cuda()
    print("lm head twin batch independence", flush=True)
    big = _twin(hip, torch, h, w, bias, cap, 40, H, V)
    small = _twin(hip, torch, h[:20].contiguous(), w, bias, cap, 20, H, V)
    assert np.array_equal(big[:20].view(np.uint32), small.view(np.uint32))


def test_fused_with_penalties_mask_and_logprobs(hip, oracle):
    """hi_rocm_sample_lm_head_ext: histories with penalties, an allowed-token
    mask and logprobs, over mixed row classes (greedy, top-k <= 64, top-p
    only, top-k 100), against the oracle run on the twin's logits with the
    same inputs: tokens bit-exact, logprob ids exact, logprobs within 1e-5.
    Rows 0-3 keep neutral penalties on a history (the fused finish's plain
    rows would take them, but the call asks for logprobs: the general path),
    and a second call without mask or logprobs sends only the rows with
    live penalties there."""
    import torch
    from hi_amd import sampler as S
    from hi_amd._lib import ROW_PARAMS_DTYPE
    lib = hip.load()
    B, H, V, cap = 24, 128, 6001, 6.0
    h, _ = _bf16(torch, (B, H), 1.0, 81)
    w, _ = _bf16(torch, (V, H), 3.0 / np.sqrt(H), 82)
    logits = _twin(hip, torch, h, w, None, cap, B, H, V)
    rng = np.random.default_rng(83)
    params = np.zeros(B, ROW_PARAMS_DTYPE)
    params["temperature"] = rng.uniform(0.5, 1.3, B)
    params["top_p"] = rng.choice(np.array([1.0, 0.9], F32), B)
    params["top_k"] = rng.choice(np.array([1, 20, 40, 64], np.int32), B)
    params["min_p"] = np.where(rng.random(B) < 0.3, F32(0.05), F32(0.0))
    params["repetition_penalty"] = rng.choice(np.array([1.0, 1.2], F32), B)
    params["frequency_penalty"] = rng.choice(np.array([0.0, 0.3], F32), B)
    params["presence_penalty"] = rng.choice(np.array([0.0, 0.5], F32), B)
    params["temperature"][4:7] = 0.0                    # greedy
    params["top_k"][8], params["top_p"][8] = 0, 0.9      # top-p only
    params["top_k"][9] = 100                            # above the fused finish's 64
    params["repetition_penalty"][:4] = 1.0
    params["frequency_penalty"][:4] = 0.0
    params["presence_penalty"][:4] = 0.0
    u = rng.random(B).astype(F32)
    offs = np.zeros(B + 1, np.uint32)
    ids_l, cnt_l = [], []
    for b in range(B):
        r = np.minimum(rng.zipf(1.3, 40) - 1, V + 3).astype(np.uint32) if b % 5 != 2 else np.zeros(0, np.uint32)
        ids_l.append(r)
        cnt_l.append(rng.integers(1, 4, r.size).astype(np.uint32))
        offs[b + 1] = offs[b] + r.size
    ids, cnts = np.concatenate(ids_l), np.concatenate(cnt_l)
    W = (V + 31) // 32
    mask = np.full((B, W), 0xFFFFFFFF, np.uint32)
    mask[10:14] = rng.integers(0, 2 ** 32, (4, W), dtype=np.uint64).astype(np.uint32)
    mask[14] = 0                                         # fully masked: EOS
    params["eos_id"][14] = 3
    n_lp = 5
    want = oracle.sample_rows(logits, params, u, offs, ids, cnts, mask, n_lp, threads=8, want_token_logprobs=True)
    ws_n = ctypes.c_size_t()
    hip.check(lib.hi_rocm_lm_head_workspace_bytes(B, V, ctypes.byref(ws_n)))
    ws = torch.zeros(ws_n.value, dtype=torch.uint8, device="cuda")
    dp = S.params_to_device(params)
    dev = lambda x: torch.from_numpy(x.view(np.int32)).cuda()
    du, doff, dids, dcnt, dmask = torch.from_numpy(u).cuda(), dev(offs), dev(ids), dev(cnts), dev(mask)
    out = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    lp = torch.zeros((B, n_lp), dtype=torch.float32, device="cuda")
    lpi = torch.zeros((B, n_lp), dtype=torch.int32, device="cuda")
    tlp = torch.zeros(B, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    print(f"lm head fused with penalties, mask and logprobs B={B} H={H} V={V}", flush=True)
    torch.cuda.synchronize()
    hip.check(lib.hi_rocm_sample_lm_head_ext(h.data_ptr(), w.data_ptr(), None, cap, B, H, V, dp.data_ptr(),
                                             du.data_ptr(), doff.data_ptr(), dids.data_ptr(), dcnt.data_ptr(),
                                             dmask.data_ptr(), out.data_ptr(), lp.data_ptr(), lpi.data_ptr(),
                                             tlp.data_ptr(), n_lp, ws.data_ptr(), ws_n.value, s.cuda_stream))
    s.synchronize()
    got = out.cpu().numpy().view(np.uint32)
    print(f"got {got.tolist()}\nwant {want['tokens'].tolist()}", flush=True)
    assert np.array_equal(got, want["tokens"]), np.flatnonzero(got != want["tokens"])
    assert np.array_equal(lpi.cpu().numpy().view(np.uint32), want["logprob_ids"])
    gl, wl = lp.cpu().numpy(), want["logprobs"]
    fin = np.isfinite(wl)
    assert np.array_equal(fin, np.isfinite(gl))
    np.testing.assert_allclose(gl[fin], wl[fin], rtol=1e-5, atol=0)
    gt, wt = tlp.cpu().numpy(), want["token_logprobs"]
    fin = np.isfinite(wt)
    np.testing.assert_allclose(gt[fin], wt[fin], rtol=1e-5, atol=0)
    # no mask, no logprobs: the plain rows finish fused, the penalised ones
    # through the general path
    want2 = oracle.sample_rows(logits, params, u, offs, ids, cnts, None, 0, threads=8)
    out.fill_(-7)
    hip.check(lib.hi_rocm_sample_lm_head_ext(h.data_ptr(), w.data_ptr(), None, cap, B, H, V, dp.data_ptr(),
                                             du.data_ptr(), doff.data_ptr(), dids.data_ptr(), dcnt.data_ptr(),
                                             None, out.data_ptr(), None, None, None, 0, ws.data_ptr(), ws_n.value,
                                             s.cuda_stream))
    s.synchronize()
    got2 = out.cpu().numpy().view(np.uint32)
    assert np.array_equal(got2, want2["tokens"]), np.flatnonzero(got2 != want2["tokens"])
