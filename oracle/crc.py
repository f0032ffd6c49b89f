"""ctypes binding of oracle/lib/liboracle_rc.so (TEST INFRASTRUCTURE ONLY).

The C range coder (oracle/range_coder.c) restates krunch_ac/cpu_reference.py
and is pinned against oracle/range_coder.py in tests/test_oracle_rc.py. The
same library holds the softmax's exp (oracle/softmax_kexp.c), used by
oracle/softmax.py and pinned in tests/test_oracle_softmax.py, and the
fixed-order float32 GEMM of the row-wise forward (oracle/rowgemm.c), pinned in
tests/test_oracle_rwkv.py against a float64 product and by its row
invariance.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "liboracle_rc.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        L.orc_encode_intervals.argtypes = [P, P, ctypes.c_size_t, ctypes.c_int, P, ctypes.c_size_t]
        L.orc_encode_intervals.restype = ctypes.c_size_t
        L.orc_decoder_size.restype = ctypes.c_size_t
        L.orc_decoder_init.argtypes = [P, P, ctypes.c_uint64]
        L.orc_decoder_target.argtypes = [P, ctypes.c_int]
        L.orc_decoder_target.restype = ctypes.c_uint32
        L.orc_decoder_consume.argtypes = [P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int]
        L.orc_decode_rows.argtypes = [P, P, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_int, P]
        L.orc_kexp.argtypes = [P, P, ctypes.c_size_t]
        L.orc_kexp.restype = None
        I = ctypes.c_int
        L.orc_gemm_rows.argtypes = [P, I, I, P, I, P]
        L.orc_gemm_rows.restype = None
        _LIB = L
    return _LIB


def encode_intervals(lo: np.ndarray, hi: np.ndarray, log2_total: int = 24) -> bytes:
    lo = np.ascontiguousarray(lo, dtype=np.uint32)
    hi = np.ascontiguousarray(hi, dtype=np.uint32)
    cap = 4 * len(lo) + 64
    while True:
        out = np.zeros(cap, dtype=np.uint8)
        n = lib().orc_encode_intervals(lo.ctypes.data, hi.ctypes.data, len(lo), log2_total,
                                       out.ctypes.data, cap)
        if n <= cap:
            return out[:n].tobytes()
        cap = n


class Decoder:
    def __init__(self, data: bytes, log2_total: int = 24):
        self._data = np.frombuffer(data, dtype=np.uint8).copy()
        self._st = ctypes.create_string_buffer(lib().orc_decoder_size())
        self.log2_total = log2_total
        lib().orc_decoder_init(self._st, self._data.ctypes.data, len(self._data))

    def target(self) -> int:
        return lib().orc_decoder_target(self._st, self.log2_total)

    def consume(self, lo: int, hi: int):
        lib().orc_decoder_consume(self._st, lo, hi, self.log2_total)

    def decode_rows(self, cdf: np.ndarray) -> np.ndarray:
        cdf = np.ascontiguousarray(cdf, dtype=np.uint32)
        out = np.empty(cdf.shape[0], dtype=np.int32)
        lib().orc_decode_rows(self._st, cdf.ctypes.data, cdf.shape[0], cdf.shape[1] - 1,
                              self.log2_total, out.ctypes.data)
        return out


def gemm_rows(x: np.ndarray, W: np.ndarray) -> np.ndarray:
    """float32 x [M, K] @ W [K, N], each output summed over k in order
    (oracle/rowgemm.c): a row's result does not depend on M."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    M, K = x.shape
    assert W.shape[0] == K
    N = W.shape[1]
    y = np.empty((M, N), dtype=np.float32)
    if M and N:
        lib().orc_gemm_rows(x.ctypes.data, M, K, W.ctypes.data, N, y.ctypes.data)
    return y
