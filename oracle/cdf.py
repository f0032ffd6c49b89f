"""Oracle: probabilities -> integer CDF (test infrastructure only).

`probs_to_cdf` restates the reference spec `krunch_ac/cdf.py:22-74`
(CDF_PRECISION = 24 at :18-19):

  1. renormalise in float32: p = probs / max(rowsum(probs), 1e-30)      (:57-58)
  2. counts = floor(p * (T - V)) + 1   (float32 multiply, MIN_PROB = 1)  (:60)
  3. deficit = T - sum(counts); the argmax bin (first index on ties)
     absorbs the whole deficit                                          (:61-67)
  4. cdf = [0, cumsum(counts)] as uint32                                 (:72-73)

`rowsum_f32` spells out the float32 summation order numpy uses for step 1's
`p.sum(axis=1)` on a C-contiguous row: the row is cut into 8192-element
blocks (numpy's default ufunc buffer size), each block is summed by numpy's
pairwise routine (8 interleaved accumulators over leaves of <= 128
elements, halving splits rounded down to a multiple of 8), and the block
sums are added left to right onto 0. The GPU kernel reproduces exactly this
tree. It is pinned against `numpy.sum` itself (tests/test_oracle_cdf.py).

`probs_to_cdf` is pinned against golden vectors written by the reference's
own `probs_to_cdf` (tests/golden/make_golden.py), against its invariants
(cdf[0]=0, cdf[V]=T, widths >= 1), and against hand-derived special cases.
"""
from __future__ import annotations

import numpy as np

CDF_PRECISION = 24
T = 1 << CDF_PRECISION

NP_BUFSIZE = 8192      # numpy's default ufunc buffer, in elements
PW_LEAF = 128          # numpy pairwise-sum leaf size


def probs_to_cdf(probs: np.ndarray, precision: int = CDF_PRECISION) -> np.ndarray:
    """(N, V) float probabilities -> (N, V+1) uint32 CDF, per cdf.py:22-74."""
    total = 1 << precision
    if probs.ndim == 1:
        probs = probs.reshape(1, -1)
    N, V = probs.shape
    assert V < total
    p = np.ascontiguousarray(probs, dtype=np.float32)
    p = p / np.maximum(p.sum(axis=1, keepdims=True), np.float32(1e-30))
    counts = np.floor(p * np.float32(total - V)).astype(np.int64) + 1
    deficit = total - counts.sum(axis=1)
    counts[np.arange(N), p.argmax(axis=1)] += deficit
    assert (counts.sum(axis=1) == total).all() and (counts > 0).all()
    cdf = np.zeros((N, V + 1), dtype=np.uint32)
    cdf[:, 1:] = np.cumsum(counts, axis=1).astype(np.uint32)
    return cdf


# ---------------------------------------------------------------------------
# numpy's float32 row-sum order, written out (the GPU kernels' summation spec)
# ---------------------------------------------------------------------------

def _pairwise(a: np.ndarray) -> np.float32:
    f = np.float32
    n = len(a)
    if n < 8:
        acc = f(-0.0)
        for x in a:
            acc = f(acc + x)
        return acc
    if n <= PW_LEAF:
        lanes = [f(a[j]) for j in range(8)]
        full = n - n % 8
        for i in range(8, full, 8):
            for j in range(8):
                lanes[j] = f(lanes[j] + a[i + j])
        acc = f(f(f(lanes[0] + lanes[1]) + f(lanes[2] + lanes[3]))
                + f(f(lanes[4] + lanes[5]) + f(lanes[6] + lanes[7])))
        for i in range(full, n):
            acc = f(acc + a[i])
        return acc
    half = n // 2
    half -= half % 8
    return f(_pairwise(a[:half]) + _pairwise(a[half:]))


def rowsum_f32(row: np.ndarray) -> np.float32:
    """Sum of a float32 row in exactly numpy's order for `x.sum(axis=-1)`."""
    row = np.asarray(row, dtype=np.float32)
    acc = np.float32(0.0)
    for start in range(0, len(row), NP_BUFSIZE):
        acc = np.float32(acc + _pairwise(row[start:start + NP_BUFSIZE]))
    return acc


def pairwise_plan(V: int):
    """The summation tree of `rowsum_f32` for a row of length V.

    Returns (leaves, inner, roots): leaves = [(start, len)] in index order;
    inner = [(left, right)] node ids in post-order (leaf ids come first,
    inner node k has id len(leaves)+k); roots = the node id of each
    8192-block. This is the structure the GPU kernel walks.
    """
    leaves, inner = [], []

    def build(start, n):
        if n <= PW_LEAF:
            leaves.append((start, n))
            return ("leaf", len(leaves) - 1)
        half = n // 2
        half -= half % 8
        l = build(start, half)
        r = build(start + half, n - half)
        inner.append((l, r))
        return ("inner", len(inner) - 1)

    roots = [build(s, min(NP_BUFSIZE, V - s)) for s in range(0, V, NP_BUFSIZE)]
    nl = len(leaves)
    ident = lambda node: node[1] if node[0] == "leaf" else nl + node[1]
    return leaves, [(ident(l), ident(r)) for l, r in inner], [ident(r) for r in roots]
