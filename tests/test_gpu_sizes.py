"""Other RWKV-4 widths than the 169M shape's 768: C = 256, 512 and 1024
(F = 4 C, two layers, V = 1000). For each codec the packed and stepped
forwards give the same bits, the fp16 codec's logits are within 1e-2 of the
fp32 oracle, and the engine round-trips byte-exact, so the LayerNorm-mix,
K/V/R + WKV, panel-product, head and CDF kernels are run at every width
they are built for."""
import numpy as np
import pytest
import torch

from krunch_amd import cpp_path, synthetic
from krunch_amd.inference import InferenceEngine
from oracle import rwkv4

pytestmark = pytest.mark.gpu

V = 1000


def _weights(C):
    return synthetic.make_weights(n_layer=2, C=C, F=4 * C, V=V, seed=C)


@pytest.mark.parametrize("w8a8", [False, True])
@pytest.mark.parametrize("C", [256, 512, 1024])
def test_width_packed_equals_stepped(C, w8a8):
    """B = 3 streams over 40 tokens (small-M kernels on both sides) and 2
    streams over 600 (packed on the tiled kernel): packed == stepped, state
    included; fp16 logits within 1e-2 of the fp32 oracle."""
    w16 = _weights(C)
    W = cpp_path.init_weights(w16, "cuda", w8a8=w8a8)
    try:
        for B, T in ((3, 40), (2, 600)):
            toks = synthetic.zipf_tokens(B, T, V=V, seed_base=40 + C)
            inp = synthetic.model_inputs(toks)
            st = cpp_path.fresh_state_batched(W, B)
            packed = cpp_path.forward_packed_batched(W, inp, st).view(B, T, -1)
            st2 = cpp_path.fresh_state_batched(W, B)
            stepped = torch.stack([cpp_path.forward_stepped_batched(W, inp[:, t], st2)
                                   for t in range(T)], dim=1)
            assert torch.equal(packed, stepped), f"C={C} B={B} T={T}"
            assert torch.equal(st.buf, st2.buf)
            if not w8a8 and T == 40:
                ref = rwkv4.forward(w16, torch.as_tensor(inp), rwkv4.new_state(2, B, C)).numpy()
                err = np.abs(packed.float().cpu().numpy().reshape(B, T, -1)[..., :V] - ref).max()
                assert err < 1e-2, f"C={C}: max abs logit error {err}"
    finally:
        cpp_path.release_weights(w16)


@pytest.mark.parametrize("w8a8", [False, True])
@pytest.mark.parametrize("C", [256, 512, 1024])
def test_width_roundtrip(C, w8a8):
    """Ragged streams through the engine (graph decode), byte-exact."""
    e = InferenceEngine()
    e.window = 64
    e.load(_weights(C), w8a8=w8a8)
    lens = [90, 7, 64 + 33, 1, 150]
    toks = [synthetic.zipf_tokens(1, n, V=V, seed_base=900 + 7 * C + i)[0]
            for i, n in enumerate(lens)]
    enc = e.compress_tokens_batched(toks)
    dec = e.decompress_tokens_batched(enc)
    for t, d in zip(toks, dec):
        np.testing.assert_array_equal(d, t)
