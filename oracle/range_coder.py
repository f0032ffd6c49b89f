"""Oracle: 32-bit range coder with E1/E2/E3 renormalisation (test infrastructure only).

Restates the reference's bit-exact spec `krunch_ac/cpu_reference.py:28-234`
(constants :28-33, MSB-first bit packing :40-84, encode :91-147, pending-bit
emission :150-154, RangeDecoder :161-211, one-shot decode :214-222, binary
search :225-234). Arithmetic uses Python ints, as the spec does.

Pinned by:
  * golden bitstreams written by tests/golden/make_golden.py from the
    reference module itself (tests/test_oracle_golden.py);
  * hand-derived known answers on 2- and 3-symbol alphabets, including an
    E3 (pending-bit) case (tests/test_oracle_rc.py);
  * brute-force round trips on tiny alphabets.
"""
from __future__ import annotations

import numpy as np

PRECISION = 32
FULL = (1 << PRECISION) - 1          # all-ones 32-bit register
HALF = 1 << (PRECISION - 1)
QUARTER = 1 << (PRECISION - 2)
THREE_QUARTERS = HALF + QUARTER


class _Bits:
    """MSB-first bit sink; the final partial byte is zero-padded."""

    def __init__(self):
        self.out = bytearray()
        self.cur = 0
        self.n = 0

    def put(self, bit: int, count: int = 1):
        for _ in range(count):
            self.cur = (self.cur << 1) | bit
            self.n += 1
            if self.n == 8:
                self.out.append(self.cur)
                self.cur = 0
                self.n = 0

    def bytes(self) -> bytes:
        if self.n:
            return bytes(self.out) + bytes([self.cur << (8 - self.n)])
        return bytes(self.out)


class _BitSource:
    """MSB-first bit source; reads zeros past the end of the data."""

    def __init__(self, data: bytes):
        self.data = data
        self.pos = 0          # bit position

    def get(self) -> int:
        byte_i = self.pos >> 3
        b = self.data[byte_i] if byte_i < len(self.data) else 0
        bit = (b >> (7 - (self.pos & 7))) & 1
        self.pos += 1
        return bit


def narrow(low: int, high: int, c_lo: int, c_hi: int, total: int):
    """Interval update for a symbol with cumulative range [c_lo, c_hi) of `total`."""
    span = high - low + 1
    return low + (span * c_lo) // total, low + (span * c_hi) // total - 1


def encode_intervals(c_lo, c_hi, total: int) -> bytes:
    """Encode a sequence of symbol intervals [c_lo[i], c_hi[i]) out of `total`.

    Equivalent to `cpu_reference.encode` given c_lo = cdf[i, sym], c_hi =
    cdf[i, sym+1]; the coder only ever reads those two entries per row.
    """
    low, high, pending = 0, FULL, 0
    sink = _Bits()
    for lo_c, hi_c in zip(c_lo, c_hi):
        low, high = narrow(low, high, int(lo_c), int(hi_c), total)
        while True:
            if high < HALF:                       # E1: both in lower half
                sink.put(0)
                sink.put(1, pending)
                pending = 0
                low, high = 2 * low, 2 * high + 1
            elif low >= HALF:                     # E2: both in upper half
                sink.put(1)
                sink.put(0, pending)
                pending = 0
                low, high = 2 * (low - HALF), 2 * (high - HALF) + 1
            elif low >= QUARTER and high < THREE_QUARTERS:   # E3: straddle
                pending += 1
                low, high = 2 * (low - QUARTER), 2 * (high - QUARTER) + 1
            else:
                break
            low &= FULL
            high &= FULL
    # Flush: one disambiguating bit followed by its pending complements.
    bit = 0 if low < QUARTER else 1
    sink.put(bit)
    sink.put(1 - bit, pending + 1)
    return sink.bytes()


def encode(cdf: np.ndarray, symbols: np.ndarray) -> bytes:
    """`cpu_reference.encode(cdf (N,V+1), symbols (N,))` -> bitstream."""
    assert cdf.ndim == 2 and symbols.shape == (cdf.shape[0],)
    total = int(cdf[0, -1])
    assert total > 0 and total & (total - 1) == 0
    rows = np.arange(cdf.shape[0])
    s = symbols.astype(np.int64)
    return encode_intervals(cdf[rows, s], cdf[rows, s + 1], total)


def search(cdf_row, target: int, V: int) -> int:
    """Largest sym in [0, V) with cdf_row[sym] <= target (cpu_reference.py:225-234)."""
    lo, hi = 0, V
    while lo < hi:
        mid = (lo + hi) // 2
        if int(cdf_row[mid + 1]) <= target:
            lo = mid + 1
        else:
            hi = mid
    return lo


class Decoder:
    """Stateful decoder, the spec of `cpu_reference.RangeDecoder`."""

    def __init__(self, bitstream: bytes):
        self.src = _BitSource(bitstream)
        self.low, self.high, self.value = 0, FULL, 0
        for _ in range(PRECISION):
            self.value = (self.value << 1) | self.src.get()

    def target(self, total: int) -> int:
        span = self.high - self.low + 1
        return ((self.value - self.low + 1) * total - 1) // span

    def consume(self, c_lo: int, c_hi: int, total: int):
        self.low, self.high = narrow(self.low, self.high, c_lo, c_hi, total)
        while True:
            if self.high < HALF:
                shift = 0
            elif self.low >= HALF:
                shift = HALF
            elif self.low >= QUARTER and self.high < THREE_QUARTERS:
                shift = QUARTER
            else:
                break
            self.low = ((self.low - shift) << 1) & FULL
            self.high = (((self.high - shift) << 1) | 1) & FULL
            self.value = (((self.value - shift) << 1) | self.src.get()) & FULL

    def decode_symbol(self, cdf_row) -> int:
        V = len(cdf_row) - 1
        total = int(cdf_row[-1])
        sym = search(cdf_row, self.target(total), V)
        self.consume(int(cdf_row[sym]), int(cdf_row[sym + 1]), total)
        return sym


def decode(bitstream: bytes, cdfs: np.ndarray) -> np.ndarray:
    """`cpu_reference.decode(bitstream, cdfs (N,V+1))` -> symbols (N,) int32."""
    dec = Decoder(bitstream)
    return np.array([dec.decode_symbol(row) for row in cdfs], dtype=np.int32)
