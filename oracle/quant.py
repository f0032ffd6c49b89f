"""w8a8 quantisation and int8 GEMM, the checker for the GPU int8 path.

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline may import this package.

BASELINE config 4 fixes the scheme (symmetric per-output-channel int8
weights with fp32 scales, per-token dynamic int8 activations, int32
accumulation); the reference has no int8 kernel (docs/INT8_WEIGHTS_DESIGN.md
only sketches one), so the definitions below are this build's, restated from
its C ABI (include/krunch_hip.h, kr_quantize_rows / kr_det_matmul_i8):

  amax = max|x| per row
  s   = amax / 127, inv = 127 / amax   (float32 IEEE divides; both 1.0 for
                                        an all-zero row)
  q   = rint(x * inv), the EXACT product (a float32 times a float32 is exact
        in float64) rounded to the nearest integer, ties to even; |q| <= 127
  y   = (float32(sum_k qa*qw) * sa[m]) * sw[n]   (two float32 multiplies)

(The GPU computes q with one FMA, x * inv + 1.5 * 2^23, whose single
rounding is that integer rounding: kr_q8_bits in krunch_amd/csrc/kr_gemm.h.)

Pinned in tests/test_oracle_quant.py by closed forms (hand-computed rows,
ties, zero rows, a row whose product rounded to float32 first would round
the other way), exact rational arithmetic on random rows, the bound
|x - q/inv| <= 1/(2 inv) and exact integer arithmetic.
"""
from __future__ import annotations

import numpy as np


def quantize_rows(x) -> tuple[np.ndarray, np.ndarray]:
    """[M, K] values (fp16 or fp32 representable) -> (int8 [M, K], float32 scales [M])."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(x), axis=1) if x.shape[1] else np.zeros(x.shape[0], np.float32)
    amax = amax.astype(np.float32)
    pos = amax > 0
    safe = np.where(pos, amax, np.float32(1.0)).astype(np.float32)
    s = np.where(pos, safe / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    inv = np.where(pos, np.float32(127.0) / safe, np.float32(1.0)).astype(np.float32)
    prod = x.astype(np.float64) * inv.astype(np.float64)[:, None]      # exact
    q = np.clip(np.rint(prod), -127, 127).astype(np.int8)
    return q, s


def matmul_i8(qa: np.ndarray, sa: np.ndarray, qw: np.ndarray, sw: np.ndarray) -> np.ndarray:
    """qa [M, K] int8, qw [N, K] int8 (rows = output channels) -> float32 [M, N]."""
    # every partial sum is an integer below 127^2 * K < 2^53: exact in float64
    assert qa.shape[1] * 127 * 127 < 2 ** 53
    acc = qa.astype(np.float64) @ qw.astype(np.float64).T
    assert np.abs(acc).max(initial=0) < 2 ** 31
    y = acc.astype(np.float32) * sa.astype(np.float32)[:, None]
    return (y.astype(np.float32) * sw.astype(np.float32)[None, :]).astype(np.float32)


def frag_index_i8(r: int, k: int, K: int) -> int:
    """Byte offset of (r, k) in a fragment-packed int8 [R, K] operand: 16 x 64
    blocks of 1 KB, block (r//16, k//64), lane r%16 + 16*((k%64)//16), byte k%16."""
    blk = (r // 16) * (K // 64) + k // 64
    lane = (r % 16) + 16 * ((k % 64) // 16)
    return blk * 1024 + lane * 16 + (k % 16)


def pack_i8(q: np.ndarray) -> np.ndarray:
    """Row-major int8 [R, K] -> fragment-packed bytes (rows padded to 16 with zeros)."""
    R, K = q.shape
    R16 = (R + 15) // 16 * 16
    pad = np.zeros((R16, K), np.int8)
    pad[:R] = q
    return pad.reshape(R16 // 16, 16, K // 64, 4, 16).transpose(0, 2, 3, 1, 4).reshape(-1)
