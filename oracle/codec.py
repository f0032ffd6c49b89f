"""Oracle: one chunk through the whole codec on the CPU (TEST INFRASTRUCTURE ONLY).

Restates the reference's chunk compress / decompress
(`krunch/inference.py:293-361` and `:363-443`, one stream):

  compress:   inputs [BOS] + tok[:-1] -> packed forward over all T tokens
              -> softmax -> integer CDF per row -> range-encode tok[t]
  decompress: per step, stepped forward of the previous token -> CDF ->
              decoder target -> binary search -> consume -> next token

with the oracle's pieces: the fp32 forward in row-wise mode (rwkv4.py; a
row's bits do not depend on how many rows share a product, so packed and
stepped logits agree bit for bit and the round trip is byte-exact), the
deterministic softmax + cdf.py restatement (softmax.py, cdf.py) and the C
range coder (range_coder.c via crc.py). Used by tests/ as the config-1
round trip and by bench.py as its CPU baseline.
"""
from __future__ import annotations

import time

import numpy as np
import torch

from oracle import crc, rwkv4
from oracle import softmax as osm

BOS_TOKEN = 0


def compress(w: dict, toks: np.ndarray, n_layer: int = 12, C: int = 768):
    """tokens [T] -> (bitstream bytes, seconds per stage dict)."""
    toks = np.asarray(toks, dtype=np.int64)
    inp = np.concatenate([[BOS_TOKEN], toks[:-1]])
    t0 = time.perf_counter()
    st = rwkv4.new_state(n_layer, 1, C)
    logits = rwkv4.forward(w, torch.as_tensor(inp[None]), st, rowwise=True)[0].numpy()
    t1 = time.perf_counter()
    cdf = osm.logits_to_cdf(logits)
    lo, hi = osm.sym_intervals(cdf, toks)
    t2 = time.perf_counter()
    bits = crc.encode_intervals(lo, hi)
    t3 = time.perf_counter()
    return bits, {"forward": t1 - t0, "cdf": t2 - t1, "coder": t3 - t2}


def decompress(w: dict, bits: bytes, n_tokens: int, n_layer: int = 12, C: int = 768):
    """bitstream -> (tokens [n_tokens] int64, seconds per stage dict)."""
    st = rwkv4.new_state(n_layer, 1, C)
    dec = crc.Decoder(bits)
    last, out = BOS_TOKEN, np.empty(n_tokens, dtype=np.int64)
    tf = tc = ta = 0.0
    for i in range(n_tokens):
        t0 = time.perf_counter()
        row = rwkv4.forward(w, torch.tensor([[last]]), st, rowwise=True)[0]
        t1 = time.perf_counter()
        c = osm.logits_to_cdf(row.numpy())[0]
        t2 = time.perf_counter()
        target = dec.target()
        sym = int(np.searchsorted(c, target, side="right") - 1)
        dec.consume(int(c[sym]), int(c[sym + 1]))
        t3 = time.perf_counter()
        tf, tc, ta = tf + t1 - t0, tc + t2 - t1, ta + t3 - t2
        out[i] = last = sym
    return out, {"forward": tf, "cdf": tc, "coder": ta}
