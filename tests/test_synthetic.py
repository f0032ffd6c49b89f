"""Synthetic inputs: deterministic, the documented shapes and distributions."""
import math

import numpy as np
import torch

from krunch_amd import synthetic


def test_weights_shapes_and_init():
    w = synthetic.make_weights(n_layer=2, C=256, F=1024, V=1000)
    assert w["emb.weight"].shape == (1000, 256) and w["head.weight"].shape == (256, 1000)
    assert w["blocks.1.ffn.key.weight"].shape == (256, 1024)
    assert w["blocks.1.ffn.value.weight"].shape == (1024, 256)
    assert w["emb.weight"].dtype == torch.float16
    assert abs(float(w["blocks.0.att.key.weight"].float().std()) - 0.02) < 1e-3
    td = w["blocks.0.att.time_decay"]
    assert td.dtype == torch.float32 and float(td[0]) == -5.0 and float(td[-1]) == 3.0
    assert abs(float(w["blocks.0.att.time_first"][0]) - math.log(0.3)) < 1e-7
    tm = w["blocks.0.att.time_mix_k"].float()
    assert 0 <= float(tm.min()) and float(tm.max()) <= 1
    w2 = synthetic.make_weights(n_layer=2, C=256, F=1024, V=1000)
    assert all(torch.equal(w[k], w2[k]) for k in w)


def test_zipf_tokens():
    t = synthetic.zipf_tokens(3, 20000)
    assert t.shape == (3, 20000) and t.dtype == np.int32
    assert t.min() >= 0 and t.max() < synthetic.N_VOCAB
    assert np.array_equal(t, synthetic.zipf_tokens(3, 20000))
    p = synthetic.zipf_cdf()
    frac0 = (t == 0).mean()
    assert abs(frac0 - p[0]) < 0.01                      # P(rank 1)
    r = synthetic.zipf_tokens(2, 4096, repeat_rate=0.5)
    inp = synthetic.model_inputs(r)
    assert (inp[:, 0] == 0).all() and np.array_equal(inp[:, 1:], r[:, :-1])
