"""GPU parity of hi_rocm_spec_verify_greedy against the oracle's literal
restatement of gpu.rs:10725-10762 (host argmax gpu.rs:6406-6435): per-row
argmax, accepted counts and emitted tokens bit for bit, over drafts that
are fully accepted, rejected at each position, per-request draft lengths,
K = 0, ties, NaN and infinities, and a 151,936-token vocabulary."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32 = np.float32


@pytest.mark.parametrize("B,K,V", [(8, 4, 151936), (33, 1, 5000), (5, 0, 777), (16, 7, 32000)])
def test_spec_verify_parity(hip, oracle, B, K, V):
    import torch
    lib = hip.load()
    rng = np.random.default_rng(B * 100 + K)
    x = (rng.standard_normal((B, K + 1, V)) * 2).astype(F32)
    x[0, :, :] = np.round(x[0, :, :])  # ties
    x[1 % B, 0, 0] = np.nan
    x[2 % B, -1, 5] = np.inf
    x[3 % B, 0, 7] = np.nan
    g_ref = np.argmax(np.nan_to_num(x, nan=-np.inf), axis=2)
    # drafts: copy the target's argmax for a prefix of random length, then differ
    d = np.zeros((B, max(K, 1)), np.uint32)
    for b in range(B):
        cut = rng.integers(0, K + 1)
        for i in range(K):
            d[b, i] = g_ref[b, i] if i < cut else (g_ref[b, i] + 1) % V
    d = d[:, :K]
    dl = rng.integers(0, K + 1, B).astype(np.int32)
    for use_len in (False, True):
        dx = torch.from_numpy(x).cuda()
        dd = torch.from_numpy(d.view(np.int32).copy() if K else np.zeros(1, np.int32)).cuda()
        ddl = torch.from_numpy(dl).cuda()
        g = torch.full((B, K + 1), -1, dtype=torch.int32, device="cuda")
        t = torch.full((B, K + 1), -1, dtype=torch.int32, device="cuda")
        c = torch.full((B,), -1, dtype=torch.int32, device="cuda")
        s = torch.cuda.Stream()
        torch.cuda.synchronize()
        print(f"spec verify B={B} K={K} V={V} lens={use_len}", flush=True)
        hip.check(lib.hi_rocm_spec_verify_greedy(dx.data_ptr(), B, K, V, dd.data_ptr(),
                                                 ddl.data_ptr() if use_len else 0, g.data_ptr(), t.data_ptr(),
                                                 c.data_ptr(), s.cuda_stream))
        s.synchronize()
        wg, wt, wc = oracle.spec_verify_greedy(x, d, dl if use_len else None)
        gg, tt, cc = g.cpu().numpy().view(np.uint32), t.cpu().numpy().view(np.uint32), c.cpu().numpy()
        assert np.array_equal(gg, wg)
        assert np.array_equal(cc, wc)
        for b in range(B):
            assert np.array_equal(tt[b, :cc[b]], wt[b, :wc[b]]), b
            assert (tt[b, cc[b]:] == 0xffffffff).all(), "write past the emitted tokens"
