"""GPU parity of hi_rocm_launch_moe_topk_router against the oracle's literal
restatement of kernels.cu:536-684 (same glibc expf): ids and weights bit for
bit, over expert counts from 8 to 2048, both gatings, bias, normalisation,
scale, and rows with ties, NaN and infinities."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32 = np.float32


def _rows(rng, rows, E):
    x = (rng.standard_normal((rows, E)) * 2.5).astype(F32)
    x[1] = np.round(x[1])            # many ties
    x[2, :] = 0.75                   # all equal
    x[3, E // 2] = np.nan            # softmax: NaN sum -> fallback
    x[4, 0] = np.inf                 # non-finite max
    x[5, :] = -np.inf
    x[6, :min(E, 7)] = -np.inf
    x[7, E - 1] = -0.0
    x[7, 0] = 0.0
    return x


@pytest.mark.parametrize("E,k", [(8, 2), (64, 8), (160, 6), (256, 8), (300, 17), (2048, 8), (97, 97)])
def test_router_parity(hip, oracle, E, k):
    import torch
    lib = hip.load()
    rng = np.random.default_rng(E * 31 + k)
    rows = 37
    x = _rows(rng, rows, E)
    bias = (rng.standard_normal(E) * 0.2).astype(F32)
    bias_nan = bias.copy()
    bias_nan[min(3, E - 1)] = np.nan
    dx = torch.from_numpy(x).to("cuda")
    ids = torch.zeros((rows, k), dtype=torch.int32, device="cuda")
    w = torch.zeros((rows, k), dtype=torch.float32, device="cuda")
    stream = torch.cuda.Stream()
    cases = [(False, None, False, 1.0), (False, None, True, 1.0), (False, None, True, 2.5),
             (True, None, False, 1.0), (True, bias, True, 1.0), (True, bias_nan, False, 0.5)]
    for sigmoid, b, norm, scale in cases:
        db = torch.from_numpy(b).to("cuda") if b is not None else None
        torch.cuda.synchronize()
        print(f"router E={E} k={k} sigmoid={sigmoid} bias={b is not None} norm={norm} scale={scale}", flush=True)
        hip.check(lib.hi_rocm_launch_moe_topk_router(
            dx.data_ptr(), ids.data_ptr(), w.data_ptr(), 0 if db is None else db.data_ptr(), rows, E, k,
            int(norm), int(sigmoid), scale, stream.cuda_stream))
        stream.synchronize()
        want_ids, want_w = oracle.moe_router(x, k, bias=b, norm_topk=norm, gating_sigmoid=sigmoid,
                                             weights_scale=scale)
        got_ids = ids.cpu().numpy().view(np.uint32)
        got_w = w.cpu().numpy()
        bad = np.flatnonzero((got_ids != want_ids).any(1) | (got_w.view(np.uint32) != want_w.view(np.uint32)).any(1))
        assert bad.size == 0, (sigmoid, norm, bad[:5], got_ids[bad[:2]], want_ids[bad[:2]], got_w[bad[:2]],
                               want_w[bad[:2]])


def test_router_rejects_like_the_reference(hip):
    lib = hip.load()
    import torch
    s = torch.cuda.Stream()
    x = torch.zeros(8, device="cuda")
    o = torch.zeros(8, device="cuda")
    assert lib.hi_rocm_launch_moe_topk_router(x.data_ptr(), o.data_ptr(), o.data_ptr(), 0, 1, 4, 5, 0, 0, 1.0,
                                              s.cuda_stream) == 1  # top_k > experts
    assert lib.hi_rocm_launch_moe_topk_router(x.data_ptr(), o.data_ptr(), o.data_ptr(), 0, 1, 4, 2, 0, 0, 1.0,
                                              0) == 1  # null stream
    assert lib.hi_rocm_launch_moe_topk_router(x.data_ptr(), o.data_ptr(), o.data_ptr(), 0, 1, 4096, 2, 0, 0, 1.0,
                                              s.cuda_stream) == 2  # beyond 2048 experts
