"""Drop-in for the reference's `krunch_ac` interface (`krunch_ac/__init__.py:21-32`),
computed on the GPU by the HIP library.

  probs_to_cdf(probs (N,V) float) -> (N, V+1) uint32     spec: cdf.py:22-74
  encode(cdf (N,V+1), symbols (N,)) -> bytes            spec: cpu_reference.py:91-147
  decode(bitstream, cdfs (N,V+1)) -> (N,) int32         spec: cpu_reference.py:214-222

Results are bit-identical to the reference spec functions; `encode_cpu` and
`decode_cpu` are kept as aliases so callers written against the reference
import unchanged (they run on the GPU here).
"""
from __future__ import annotations

import numpy as np
import torch

from krunch_amd import krunch_ac_hip as ops

CDF_PRECISION = 24
T = 1 << CDF_PRECISION
_DEV = "cuda"


def probs_to_cdf(probs: np.ndarray, precision: int = CDF_PRECISION) -> np.ndarray:
    from krunch_amd import _lib
    if probs.ndim == 1:
        probs = probs.reshape(1, -1)
    assert probs.ndim == 2, f"probs must be (N, V), got {probs.shape}"
    N, V = probs.shape
    assert V < (1 << precision), f"vocab size {V} must be < T"
    p = torch.from_numpy(np.ascontiguousarray(probs, dtype=np.float32)).to(_DEV)
    out = torch.empty((N, V + 1), dtype=torch.int32, device=_DEV)
    _lib.call("kr_probs_to_cdf", p.data_ptr(), N, V, V, out.data_ptr(), precision, _lib.stream_ptr())
    return out.cpu().numpy().view(np.uint32)


def encode(cdf: np.ndarray, symbols: np.ndarray) -> bytes:
    assert cdf.ndim == 2 and symbols.shape == (cdf.shape[0],)
    total = int(cdf[0, -1])
    precision = total.bit_length() - 1
    assert total > 0 and (1 << precision) == total, "T must be a power of two"
    N = cdf.shape[0]
    c = torch.from_numpy(np.ascontiguousarray(cdf).view(np.int32)).to(_DEV)
    s = torch.from_numpy(np.ascontiguousarray(symbols, dtype=np.int32)).to(_DEV)
    cap = 8 * N + 64
    buf = torch.zeros(cap, dtype=torch.uint8, device=_DEV)
    st = torch.tensor([0, 0xFFFFFFFF, 0, 0], dtype=torch.int64).to(torch.uint32).to(_DEV)
    ops.encode_step(c, s, buf, st, precision)
    ops.encode_finalize(buf, st)
    nbits = int(st.cpu().to(torch.int64)[3])
    return bytes(buf[:(nbits + 7) // 8].cpu().numpy())


def decode(bitstream: bytes, cdfs: np.ndarray) -> np.ndarray:
    assert cdfs.ndim == 2
    N = cdfs.shape[0]
    total = int(cdfs[0, -1])
    precision = total.bit_length() - 1
    data = np.frombuffer(bitstream, dtype=np.uint8)
    buf = torch.from_numpy(data.copy() if len(data) else np.zeros(1, np.uint8)).to(_DEV)
    if not len(data):
        buf = buf[:0]
    st = torch.zeros(4, dtype=torch.uint32, device=_DEV)
    ops.decode_init(buf, st)
    c = torch.from_numpy(np.ascontiguousarray(cdfs).view(np.int32)).to(_DEV)
    out = torch.empty(N, dtype=torch.int32, device=_DEV)
    for i in range(N):
        ops.decode_step(c[i], buf, st, out[i:i + 1], precision)
    return out.cpu().numpy()


encode_cpu = encode
decode_cpu = decode

__all__ = ["probs_to_cdf", "CDF_PRECISION", "encode", "decode", "encode_cpu", "decode_cpu"]
