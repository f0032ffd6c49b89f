"""Seeded random shapes through the engine: stream counts 1, 17, 129, 300,
347 and 420, random ragged lengths, a random window of 64 or 128 tokens,
both codecs. The tile choices of the stepped products, the decode head's row
groups, the K/V/R + WKV tile and the CDF's rows per CU all depend on the
stream count, so every draw takes a different mix of kernel paths; each must
round-trip byte-exact."""
import numpy as np
import pytest

from krunch_amd import synthetic
from krunch_amd.inference import InferenceEngine

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def engines():
    w = synthetic.make_weights()
    out = {}
    for w8a8 in (False, True):
        e = InferenceEngine()
        out[w8a8] = e.load(w, w8a8=w8a8)
    return out


@pytest.mark.parametrize("seed", range(6))
def test_random_shapes_roundtrip(engines, seed):
    rng = np.random.default_rng(4242 + seed)
    w8a8 = bool(seed % 2)
    e = engines[w8a8]
    e.window = int(rng.choice([64, 128]))
    B = [1, 17, 129, 300, 347, 420][seed]
    lens = rng.integers(1, 3 * e.window, size=B)
    toks = [synthetic.zipf_tokens(1, int(n), seed_base=7000 + 1000 * seed + i)[0]
            for i, n in enumerate(lens)]
    enc = e.compress_tokens_batched(toks)
    dec = e.decompress_tokens_batched(enc)
    for i, (t, d) in enumerate(zip(toks, dec)):
        np.testing.assert_array_equal(d, t, err_msg=f"seed {seed} B={B} stream {i}")
