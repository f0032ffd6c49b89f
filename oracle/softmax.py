"""Oracle: the build's deterministic head softmax (test infrastructure only).

The reference turns fp16 logits into probabilities in `det_softmax_cdf.cu:62-185`
(row max, sum of exp(x - max), p = exp * (1/sum)) and then into counts.
`krunch_ac/cdf.py:22-74` is the CDF spec. This build keeps that structure but
fixes every rounding so that CPU and GPU agree bit for bit:

  x_i = float32(logit_i)
  m   = max_i x_i
  e_i = kexp(x_i - m)           # the exp defined below (no libm exp)
  S   = rowsum_f32(e)           # numpy's float32 row-sum order
  q_i = e_i * (1 / S)           # one IEEE division per row
  cdf = probs_to_cdf(q)         # cdf.py:22-74, bit for bit

`kexp` is a Cody-Waite reduction x = n*ln2 + r, |r| <= ln2/2, followed by a
degree-6 minimax polynomial of e^r in Horner form, then scaling by 2^n. The
reduction and every Horner step are fused multiply-adds (one rounding each);
the multiply by log2(e) and the round to integer are single IEEE operations.
numpy has no float32 FMA, so kexp is computed by the C restatement in
`oracle/softmax_kexp.c` (C's fmaf is correctly rounded, as the GPU's
v_fma_f32 is). Inputs below -87 return 0, so the result is never subnormal.

Pinned by: comparison with float64 exp (<= 2 ulp, tests/test_oracle_softmax.py),
exact values at 0 and at multiples of ln 2, monotonicity on a dense grid,
and the CDF invariants.
"""
from __future__ import annotations

import numpy as np

from oracle.cdf import probs_to_cdf, CDF_PRECISION

f32 = np.float32


def kexp(x: np.ndarray) -> np.ndarray:
    """Deterministic float32 exp for x <= 0 (see module docstring)."""
    from oracle.crc import lib
    x = np.asarray(x, dtype=f32)
    xc = np.ascontiguousarray(x.reshape(-1))
    out = np.empty_like(xc)
    lib().orc_kexp(xc.ctypes.data, out.ctypes.data, xc.size)
    return out.reshape(x.shape)


def softmax_probs(logits: np.ndarray) -> np.ndarray:
    """(N, V) fp16/fp32 logits -> (N, V) float32 probabilities q."""
    x = np.asarray(logits).astype(f32)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    e = kexp(x - x.max(axis=1, keepdims=True))
    inv = f32(1.0) / e.sum(axis=1, keepdims=True)
    return (e * inv).astype(f32)


def logits_to_cdf(logits: np.ndarray, precision: int = CDF_PRECISION) -> np.ndarray:
    """(N, V) logits -> (N, V+1) uint32 CDF (softmax_probs then cdf.py)."""
    return probs_to_cdf(softmax_probs(logits), precision)


def sym_intervals(cdf: np.ndarray, symbols: np.ndarray):
    """(cdf[i, sym_i], cdf[i, sym_i + 1]) per row: what the range coder reads."""
    rows = np.arange(cdf.shape[0])
    s = np.asarray(symbols, dtype=np.int64)
    return cdf[rows, s].astype(np.uint32), cdf[rows, s + 1].astype(np.uint32)
