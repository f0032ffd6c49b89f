"""A real-checkpoint-format file through the engine.

* A 12-layer RWKV-4-169M-shaped checkpoint in the file layout (torch Linear
  [out, in] matrices, [1, 1, C] time_mix, a non-trivial blocks.0.ln0, LayerNorm
  weights and biases away from 1 / 0, per-channel time_first) saved as a
  weights_only .pth and loaded by load_rwkv4 with its default (the rescaled
  weights the reference's codec reads, krunch/cpp_path.py:26-91, with x never
  halved): the engine's logits are within 1e-2 of the fp32 oracle run on the
  converted weights, and its payload equals the oracle coder fed the oracle
  CDF of those logits. Twelve layers, so the rescale of layers 6-11 is in
  play.
* A small checkpoint compresses and decompresses byte-exact and gives the
  same stream as the in-memory weights.
"""
import math

import numpy as np
import pytest
import torch

from krunch_amd import cpp_path, inference, synthetic
from krunch_amd.weights import convert_rwkv4_state_dict, to_rwkv4_state_dict
from oracle import range_coder as orc
from oracle import rwkv4
from oracle import softmax as osm

pytestmark = pytest.mark.gpu


def _checkpoint(n_layer=12, C=768, F=3072, V=50277, seed=11):
    """RWKV-4 checkpoint tensors (file layout, fp16 like the published ones)."""
    g = torch.Generator().manual_seed(seed)
    n = lambda *s, sd=0.02: torch.randn(*s, generator=g) * sd
    sd = {"emb.weight": n(V, C, sd=0.5), "blocks.0.ln0.weight": 1 + n(C, sd=0.2),
          "blocks.0.ln0.bias": n(C, sd=0.1), "ln_out.weight": 1 + n(C, sd=0.1),
          "ln_out.bias": n(C, sd=0.05), "head.weight": n(V, C)}
    for i in range(n_layer):
        b, a, f = f"blocks.{i}.", f"blocks.{i}.att.", f"blocks.{i}.ffn."
        for ln in ("ln1", "ln2"):
            sd[b + ln + ".weight"], sd[b + ln + ".bias"] = 1 + n(C, sd=0.1), n(C, sd=0.05)
        for m in ("time_mix_k", "time_mix_v", "time_mix_r"):
            sd[a + m] = torch.rand(1, 1, C, generator=g)
        for m in ("time_mix_k", "time_mix_r"):
            sd[f + m] = torch.rand(1, 1, C, generator=g)
        sd[a + "time_decay"] = torch.linspace(-5, 3, C) + n(C, sd=0.3)
        sd[a + "time_first"] = math.log(0.3) + n(C, sd=0.3)
        for m in ("key", "value", "receptance", "output"):
            sd[a + m + ".weight"] = n(C, C)
        sd[f + "key.weight"], sd[f + "value.weight"] = n(F, C), n(C, F)
        sd[f + "receptance.weight"] = n(C, C)
    keep32 = ("time_decay", "time_first")
    return {k: (v if k.endswith(keep32) else v.half()).contiguous() for k, v in sd.items()}


def test_checkpoint_logits_and_payload_vs_oracle(tmp_path):
    sd = _checkpoint()
    torch.save(sd, tmp_path / "rwkv4-169m-shape.pth")
    eng = inference.InferenceEngine()
    eng.window = 32
    eng.load(str(tmp_path / "rwkv4-169m-shape.pth"))
    w = convert_rwkv4_state_dict(sd)           # the default: rescaled, as loaded
    assert not torch.equal(w["blocks.6.att.output.weight"],
                           convert_rwkv4_state_dict(sd, rescale=False)["blocks.6.att.output.weight"])
    toks = synthetic.zipf_tokens(2, 80, seed_base=2600)
    W = eng.weights
    st = cpp_path.fresh_state_batched(W, 2)
    got = cpp_path.forward_packed_batched(W, synthetic.model_inputs(toks), st)
    got = got.float().cpu().numpy().reshape(2, 80, -1)
    ref = rwkv4.forward(w, torch.as_tensor(synthetic.model_inputs(toks)),
                        rwkv4.new_state(12, 2, 768)).numpy()
    d = np.abs(got - ref).max()
    assert d < 1e-2, f"checkpoint logits vs fp32 oracle: max abs {d}"
    enc = eng.compress_tokens_batched(list(toks))
    for b in range(2):
        assert enc[b][8:] == orc.encode(osm.logits_to_cdf(got[b]), toks[b]), f"stream {b}"
    dec = eng.decompress_tokens_batched(enc)
    for t, x in zip(toks, dec):
        np.testing.assert_array_equal(x, t)


def test_pth_checkpoint_roundtrip(tmp_path):
    w = synthetic.make_weights(n_layer=2)
    torch.save(to_rwkv4_state_dict(w), tmp_path / "rwkv4.pth")
    data = b"RWKV-4 checkpoint through the MI355X engine. " * 20
    a = inference.InferenceEngine().load(str(tmp_path / "rwkv4.pth"))
    b = inference.InferenceEngine().load(w)
    blob = a.compress(data)
    assert blob == b.compress(data)
    assert a.decompress(blob) == data
