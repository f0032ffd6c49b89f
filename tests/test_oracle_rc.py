"""Range-coder oracle: hand-derived known answers, brute-force round trips,
and the C restatement against the Python one."""
import itertools

import numpy as np
import pytest

from oracle import cdf as ocdf
from oracle import crc
from oracle import range_coder as orc

T24 = 1 << 24


def _cdf(*bounds):
    return np.array([bounds], dtype=np.uint32)


# Derivations (total T = 2^24, initial low = 0, high = 2^32 - 1):
#  * cdf [0, T/2, T], sym 0 -> high = 2^31-1 < HALF: E1 emits 0, interval
#    back to full; flush: low < QUARTER -> 0 then one pending complement 1:
#    bits 0 0 1 -> 0x20.
#  * sym 1 -> low = 2^31: E2 emits 1; flush bits 0 1 -> 1 0 1 -> 0xA0.
#  * cdf [0, T/4, 3T/4, T], sym 1 -> [2^30, 3*2^30 - 1]: E3, pending = 1,
#    interval back to full; flush: 0 then two 1s -> 0 1 1 -> 0x60.
#  * then sym 0 -> [0, 2^30 - 1]: E1 emits 0 + pending 1, E1 again emits 0;
#    flush 0 1 -> bits 0 1 0 0 1 -> 0x48.
@pytest.mark.parametrize("cdf_row,syms,expected", [
    ((0, T24 // 2, T24), [0], b"\x20"),
    ((0, T24 // 2, T24), [1], b"\xa0"),
    ((0, T24 // 4, 3 * T24 // 4, T24), [1], b"\x60"),
    ((0, T24 // 4, 3 * T24 // 4, T24), [1, 0], b"\x48"),
])
def test_known_answers(cdf_row, syms, expected):
    cdf = np.repeat(_cdf(*cdf_row), len(syms), axis=0)
    s = np.array(syms, dtype=np.int32)
    assert orc.encode(cdf, s) == expected
    np.testing.assert_array_equal(orc.decode(expected, cdf), s)
    lo, hi = cdf[np.arange(len(s)), s], cdf[np.arange(len(s)), s + 1]
    assert crc.encode_intervals(lo, hi) == expected


def test_brute_force_tiny_alphabet():
    """Every symbol string of length <= 5 over a skewed 3-symbol alphabet
    round-trips and different strings give different bitstreams."""
    cdf_row = (0, 1, T24 // 3, T24)          # symbol 0 has the minimum width 1
    seen = {}
    for n in range(1, 6):
        for syms in itertools.product(range(3), repeat=n):
            cdf = np.repeat(_cdf(*cdf_row), n, axis=0)
            s = np.array(syms, dtype=np.int32)
            bits = orc.encode(cdf, s)
            np.testing.assert_array_equal(orc.decode(bits, cdf), s)
            assert seen.setdefault((n, bits), syms) == syms


@pytest.mark.parametrize("N,V,seed", [(1, 4, 1), (50, 32, 2), (500, 1000, 3), (64, 50277, 4)])
def test_c_restatement_matches_python(N, V, seed):
    rng = np.random.default_rng(seed)
    p = rng.random((N, V)).astype(np.float32) ** 4
    cdf = ocdf.probs_to_cdf(p)
    sym = rng.integers(0, V, size=N).astype(np.int32)
    bits = orc.encode(cdf, sym)
    rows = np.arange(N)
    assert crc.encode_intervals(cdf[rows, sym], cdf[rows, sym + 1]) == bits
    np.testing.assert_array_equal(crc.Decoder(bits).decode_rows(cdf), sym)


def test_min_width_symbols_and_long_pending_runs():
    """Symbols of width 1 (probability 2^-24) every step; straddling
    intervals that build long E3 runs."""
    V = 200
    p = np.full((300, V), 1e-6, dtype=np.float32)
    p[:, 0] = 1.0
    cdf = ocdf.probs_to_cdf(p)
    sym = np.full(300, V - 1, dtype=np.int32)
    bits = orc.encode(cdf, sym)
    np.testing.assert_array_equal(orc.decode(bits, cdf), sym)
    mid = np.repeat(_cdf(0, T24 // 2 - 1, T24 // 2 + 1, T24), 64, axis=0)
    s = np.ones(64, dtype=np.int32)
    bits = orc.encode(mid, s)
    np.testing.assert_array_equal(orc.decode(bits, mid), s)
    assert crc.encode_intervals(mid[:, 1], mid[:, 2]) == bits
