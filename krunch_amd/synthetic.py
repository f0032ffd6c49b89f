"""Synthetic inputs for the RWKV-4-169M-shaped codec: weights and token streams.

There are no checkpoints or datasets on the benchmark machines, so every
measurement uses

* random-init weights of the RWKV-4-Pile-169M shape (12 layers, C=768,
  FFN=3072, V=50277) drawn from `torch.Generator().manual_seed(seed)` in a
  fixed order: emb [V,C]; per layer att.key, att.value, att.receptance,
  att.output [C,C], ffn.key [C,F], ffn.receptance [C,C], ffn.value [F,C];
  then per layer time_mix_k, time_mix_v, time_mix_r, ffn time_mix_k,
  ffn time_mix_r ~ U(0,1); then head [C,V]. Matrices ~ N(0, 0.02).
  time_decay = linspace(-5, 3, C) (raw; the decay used is -exp(raw)),
  time_first = ln(0.3), LayerNorm weight 1 / bias 0.
  Matrices are stored [in, out] (y = x @ W), the layout the reference reads
  (`krunch/cpp_path.py:59-86`, keys as in the rwkv package).
* token streams drawn i.i.d. from Zipf(s=1.1) truncated to the vocabulary by
  inverse CDF (rank r -> token r-1), one numpy Generator per chunk seeded
  1000 + chunk index; optionally with repeated 64-token spans.
"""
from __future__ import annotations

import math

import numpy as np
import torch

N_LAYER, N_EMBD, N_FFN, N_VOCAB = 12, 768, 3072, 50277
BOS_TOKEN = 0


def make_weights(n_layer: int = N_LAYER, C: int = N_EMBD, F: int = N_FFN,
                 V: int = N_VOCAB, seed: int = 0, dtype=torch.float16) -> dict:
    g = torch.Generator().manual_seed(seed)
    normal = lambda *shape: (torch.randn(*shape, generator=g) * 0.02)
    w = {"emb.weight": normal(V, C)}
    for i in range(n_layer):
        a, f = f"blocks.{i}.att.", f"blocks.{i}.ffn."
        w[a + "key.weight"] = normal(C, C)
        w[a + "value.weight"] = normal(C, C)
        w[a + "receptance.weight"] = normal(C, C)
        w[a + "output.weight"] = normal(C, C)
        w[f + "key.weight"] = normal(C, F)
        w[f + "receptance.weight"] = normal(C, C)
        w[f + "value.weight"] = normal(F, C)
    for i in range(n_layer):
        a, f, b = f"blocks.{i}.att.", f"blocks.{i}.ffn.", f"blocks.{i}."
        for name in (a + "time_mix_k", a + "time_mix_v", a + "time_mix_r",
                     f + "time_mix_k", f + "time_mix_r"):
            w[name] = torch.rand(C, generator=g)
        w[a + "time_decay"] = torch.linspace(-5.0, 3.0, C)
        w[a + "time_first"] = torch.full((C,), math.log(0.3))
        for ln in ("ln1", "ln2"):
            w[b + ln + ".weight"] = torch.ones(C)
            w[b + ln + ".bias"] = torch.zeros(C)
    w["ln_out.weight"] = torch.ones(C)
    w["ln_out.bias"] = torch.zeros(C)
    w["head.weight"] = normal(C, V)
    keep32 = ("time_decay", "time_first")
    return {k: (v if k.endswith(keep32) else v.to(dtype)).contiguous() for k, v in w.items()}


def zipf_cdf(V: int = N_VOCAB, s: float = 1.1) -> np.ndarray:
    p = np.arange(1, V + 1, dtype=np.float64) ** (-s)
    c = np.cumsum(p)
    return c / c[-1]


def zipf_tokens(n_chunks: int, T: int, V: int = N_VOCAB, s: float = 1.1,
                seed_base: int = 1000, repeat_rate: float = 0.0,
                span: int = 64) -> np.ndarray:
    """[n_chunks, T] int32 token ids. With repeat_rate > 0 each 64-token block
    is, with that probability, a copy of an earlier span of the same chunk."""
    cdf = zipf_cdf(V, s)
    out = np.empty((n_chunks, T), dtype=np.int32)
    for b in range(n_chunks):
        rng = np.random.default_rng(seed_base + b)
        toks = np.minimum(np.searchsorted(cdf, rng.random(T), side="right"), V - 1)
        if repeat_rate > 0:
            for start in range(span, T - span + 1, span):
                if rng.random() < repeat_rate:
                    src = int(rng.integers(0, start - span + 1))
                    toks[start:start + span] = toks[src:src + span]
        out[b] = toks
    return out


def model_inputs(tokens: np.ndarray) -> np.ndarray:
    """[B, T] targets -> [B, T] model inputs [BOS] + tok[:-1] per chunk
    (`krunch/inference.py:305`)."""
    inp = np.empty_like(tokens)
    inp[:, 0] = BOS_TOKEN
    inp[:, 1:] = tokens[:, :-1]
    return inp
