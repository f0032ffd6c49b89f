"""w8a8 quantisation and int8 GEMM, the checker for the GPU int8 path.

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline may import this package.

BASELINE config 4 fixes the scheme (symmetric per-output-channel int8
weights with fp32 scales, per-token dynamic int8 activations, int32
accumulation); the reference has no int8 kernel (docs/INT8_WEIGHTS_DESIGN.md
only sketches one), so the definitions below are this build's, restated from
its C ABI (include/krunch_hip.h, kr_quantize_rows / kr_det_matmul_i8):

  s = max|x| / 127 per row (float32 IEEE divide; 1.0 for an all-zero row)
  q = clip(rint(x / s), -127, 127)      (float32 divide, ties to even)
  y = (float32(sum_k qa*qw) * sa[m]) * sw[n]   (two float32 multiplies)

Pinned in tests/test_oracle_quant.py by closed forms (hand-computed rows,
ties, zero rows), the bound |x - q*s| <= s/2 and exact integer arithmetic.
"""
from __future__ import annotations

import numpy as np


def quantize_rows(x) -> tuple[np.ndarray, np.ndarray]:
    """[M, K] values (fp16 or fp32 representable) -> (int8 [M, K], float32 scales [M])."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(x), axis=1) if x.shape[1] else np.zeros(x.shape[0], np.float32)
    s = np.where(amax > 0, amax.astype(np.float32) / np.float32(127.0), np.float32(1.0))
    s = s.astype(np.float32)
    q = np.clip(np.rint(x / s[:, None]), -127, 127).astype(np.int8)
    return q, s


def matmul_i8(qa: np.ndarray, sa: np.ndarray, qw: np.ndarray, sw: np.ndarray) -> np.ndarray:
    """qa [M, K] int8, qw [N, K] int8 (rows = output channels) -> float32 [M, N]."""
    acc = qa.astype(np.int64) @ qw.astype(np.int64).T
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
