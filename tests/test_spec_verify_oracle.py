"""CPU pins of the greedy speculative verification restatement
(oracle hro_spec_verify_greedy: gpu.rs:10725-10762 with the host argmax of
gpu.rs:6406-6435): closed forms of the acceptance (all accepted -> K + 1
tokens with the bonus, first mismatch at i -> i + 1 tokens ending in the
target's token, K = 0, per-request draft lengths), the argmax rule's
special cases (ties to the first index, a NaN at index 0 keeps index 0,
NaNs elsewhere never win, -0 == +0), and numpy's first-maximum argmax on
random rows without NaN."""
import numpy as np

from oracle import oracle as O

F32 = np.float32


def _rows(tokens, V=7):
    x = np.zeros((1, len(tokens), V), F32)
    for r, t in enumerate(tokens):
        x[0, r, t] = 1.0
    return x


def test_acceptance_closed_forms():
    O.build()
    x = _rows([3, 5, 1, 6])
    g, t, c = O.spec_verify_greedy(x, np.array([[3, 5, 1]], np.uint32))
    assert g.tolist() == [[3, 5, 1, 6]] and c.tolist() == [4] and t[0, :4].tolist() == [3, 5, 1, 6]
    g, t, c = O.spec_verify_greedy(x, np.array([[3, 4, 1]], np.uint32))
    assert c.tolist() == [2] and t[0, :2].tolist() == [3, 5]
    g, t, c = O.spec_verify_greedy(x, np.array([[0, 5, 1]], np.uint32))
    assert c.tolist() == [1] and t[0, :1].tolist() == [3]
    g, t, c = O.spec_verify_greedy(_rows([2]), np.zeros((1, 0), np.uint32))
    assert c.tolist() == [1] and t[0, 0] == 2
    # a shorter draft: only its entries are checked, then its bonus row
    g, t, c = O.spec_verify_greedy(x, np.array([[3, 5, 0]], np.uint32), draft_len=np.array([2], np.int32))
    assert c.tolist() == [3] and t[0, :3].tolist() == [3, 5, 1]


def test_argmax_rule():
    nan = F32(np.nan)
    rows = np.array([[[1, 4, 4, 2]], [[nan, 9, 9, 1]], [[1, nan, 0.5, 1]], [[-0.0, 0.0, -1, -2]],
                     [[-np.inf, nan, nan, nan]], [[nan, nan, nan, nan]]], F32).reshape(6, 1, 4)
    g, _, _ = O.spec_verify_greedy(rows, np.zeros((6, 0), np.uint32))
    assert g[:, 0].tolist() == [1, 0, 0, 0, 0, 0]


def test_argmax_matches_numpy_first_max():
    rng = np.random.default_rng(4)
    x = np.round(rng.standard_normal((5, 4, 300)) * 3).astype(F32)  # many ties
    d = rng.integers(0, 300, (5, 3)).astype(np.uint32)
    g, t, c = O.spec_verify_greedy(x, d)
    assert np.array_equal(g, np.argmax(x, axis=2).astype(np.uint32))
    for b in range(5):
        acc = next((i for i in range(3) if d[b, i] != g[b, i]), 3)
        assert c[b] == acc + 1 and np.array_equal(t[b, :acc + 1], g[b, :acc + 1])
