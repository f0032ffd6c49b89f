"""CDF oracle: numpy's float32 row-sum order (pinned against numpy.sum itself),
the plan the GPU walks, invariants and special cases of cdf.py."""
import numpy as np
import pytest

from oracle import cdf as ocdf


@pytest.mark.parametrize("V", [1, 5, 8, 100, 128, 129, 1000, 8192, 8193, 8199, 20000, 50277])
def test_rowsum_order_is_numpys(V):
    rng = np.random.default_rng(V)
    rows = (rng.random((3, V)) ** 3).astype(np.float32)
    np_sums = rows.sum(axis=1, keepdims=True)[:, 0]
    for i in range(3):
        assert ocdf.rowsum_f32(rows[i]) == np_sums[i]


@pytest.mark.parametrize("V", [1, 7, 100, 1141, 8192, 8193, 50277])
def test_plan_reproduces_rowsum(V):
    """Walking pairwise_plan (leaves, then inner nodes in order, then the
    blocks left to right) gives rowsum_f32 bit for bit."""
    rng = np.random.default_rng(V + 1)
    row = rng.random(V).astype(np.float32)
    leaves, inner, roots = ocdf.pairwise_plan(V)
    assert sum(n for _, n in leaves) == V
    assert all(leaves[i][0] + leaves[i][1] == leaves[i + 1][0] for i in range(len(leaves) - 1))
    vals = [ocdf._pairwise(row[s:s + n]) for s, n in leaves]
    for l, r in inner:
        vals.append(np.float32(vals[l] + vals[r]))
    acc = np.float32(0.0)
    for r in roots:
        acc = np.float32(acc + vals[r])
    assert acc == ocdf.rowsum_f32(row)


def test_invariants_and_special_cases():
    rng = np.random.default_rng(5)
    p = rng.random((16, 300)).astype(np.float32)
    cdf = ocdf.probs_to_cdf(p)
    assert (cdf[:, 0] == 0).all() and (cdf[:, -1] == ocdf.T).all()
    assert (np.diff(cdf.astype(np.int64), axis=1) >= 1).all()
    # one-hot: every other bin gets MIN_PROB = 1, the hot bin takes the rest
    V = 1000
    onehot = np.zeros((1, V), dtype=np.float32)
    onehot[0, 123] = 1.0
    w = np.diff(ocdf.probs_to_cdf(onehot)[0].astype(np.int64))
    assert (np.delete(w, 123) == 1).all() and w[123] == ocdf.T - (V - 1)
    # uniform over V = 2^k: p*(T-V) = (T-V)/V exactly; floor + 1 each, index 0
    # (first maximum) absorbs the deficit
    V = 1024
    u = np.full((1, V), 1.0 / V, dtype=np.float32)
    w = np.diff(ocdf.probs_to_cdf(u)[0].astype(np.int64))
    base = (ocdf.T - V) // V + 1
    assert (w[1:] == base).all() and w[0] == ocdf.T - base * (V - 1)


def test_renormalisation_is_float32():
    """Scaling the input by a power of two leaves the CDF unchanged (exact in
    float32 while nothing underflows)."""
    rng = np.random.default_rng(9)
    p = rng.random((4, 777)).astype(np.float32)
    np.testing.assert_array_equal(ocdf.probs_to_cdf(p), ocdf.probs_to_cdf(p * np.float32(8)))
