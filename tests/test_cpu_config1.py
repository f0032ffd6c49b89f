"""BASELINE config 1 on the CPU: the 169M-shaped fp32 model (seed 0), one
chunk of T = 1024 Zipf(1.1) tokens, packed forward -> softmax -> integer CDF
-> range-coder encode, then stepped decode; the round trip is byte-exact.
This is the oracle codec (oracle/codec.py) end to end, the CPU baseline
bench.py times."""
import os

import numpy as np
import torch

from krunch_amd import synthetic
from oracle import codec
from oracle import range_coder as orc
from oracle import softmax as osm


def test_config1_cpu_roundtrip_169M_T1024():
    torch.set_num_threads(os.cpu_count() or 1)
    w = synthetic.make_weights(dtype=torch.float32)
    toks = synthetic.zipf_tokens(1, 1024)[0]
    bits, _ = codec.compress(w, toks)
    got, _ = codec.decompress(w, bits, len(toks))
    np.testing.assert_array_equal(got, toks)
    # bits per token of a random-init model on Zipf tokens: near the entropy
    # of the model's (flat-ish) predictions, well below log2(50277) = 15.6
    assert 8 * len(bits) / len(toks) < 17.0


def test_oracle_codec_small_matches_python_coder():
    """The codec's C coder path gives the pure-Python restatement's bytes."""
    w = synthetic.make_weights(n_layer=2, C=256, F=512, V=500, dtype=torch.float32)
    toks = synthetic.zipf_tokens(1, 40, V=500)[0]
    bits, _ = codec.compress(w, toks, n_layer=2, C=256)
    import torch as t
    from oracle import rwkv4
    inp = np.concatenate([[0], toks[:-1]])
    lg = rwkv4.forward(w, t.as_tensor(inp[None]), rwkv4.new_state(2, 1, 256), rowwise=True)[0]
    assert bits == orc.encode(osm.logits_to_cdf(lg.numpy()), toks)
    got, _ = codec.decompress(w, bits, len(toks), n_layer=2, C=256)
    np.testing.assert_array_equal(got, toks)
