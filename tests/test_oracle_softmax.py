"""Softmax oracle: the deterministic exp against float64 exp, exact points,
monotonicity; softmax probabilities against float64 softmax."""
import numpy as np

from oracle import softmax as osm


def _ulp_err(got, ref):
    ref32 = ref.astype(np.float32)
    spacing = np.spacing(np.abs(ref32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - ref) / spacing


def test_kexp_accuracy_dense_grid():
    """Faithful on a dense grid: the degree-6 minimax polynomial is within
    0.053 ulp of e^r in exact arithmetic; with the float32 roundings of the
    reduction and the Horner steps the result stays below 1 ulp (0.87 max)."""
    x = np.linspace(-86.99, 0.0, 2_000_001, dtype=np.float32)
    got = osm.kexp(x)
    assert _ulp_err(got, np.exp(x.astype(np.float64))).max() < 1.0
    assert (np.diff(got.astype(np.float64)) >= 0).all()          # monotone


def test_kexp_exact_points_and_floor():
    assert osm.kexp(np.float32(0.0)) == np.float32(1.0)
    for n in range(1, 120):
        x = np.float32(-n * np.log(2.0))
        assert _ulp_err(osm.kexp(x), np.exp(np.float64(x))) <= 2.0
    assert osm.kexp(np.float32(-87.5)) == 0.0
    assert osm.kexp(np.float32(-np.inf)) == 0.0
    tiny = osm.kexp(np.float32(-87.0))
    assert tiny >= np.finfo(np.float32).tiny                       # never subnormal


def test_softmax_close_to_float64():
    rng = np.random.default_rng(3)
    logits = (rng.standard_normal((8, 50277)) * 3).astype(np.float16)
    q = osm.softmax_probs(logits)
    x = logits.astype(np.float64)
    ref = np.exp(x - x.max(axis=1, keepdims=True))
    ref /= ref.sum(axis=1, keepdims=True)
    np.testing.assert_allclose(q, ref, rtol=2e-6, atol=1e-12)
    cdf = osm.logits_to_cdf(logits)
    assert (np.diff(cdf.astype(np.int64), axis=1) >= 1).all() and (cdf[:, -1] == 1 << 24).all()
