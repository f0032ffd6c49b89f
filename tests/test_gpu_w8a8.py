"""The w8a8 codec end to end on the GPU: logits against
the fp32 oracle (north_star: 5e-2 max-abs) and against the oracle's own int8
restatement; packed == stepped bit for bit (the CDFs of compress and
decompress must agree); a byte-exact round trip and its bits/token beside the
fp16 codec's."""
import numpy as np
import pytest
import torch

from krunch_amd import cpp_path, synthetic
from krunch_amd.inference import InferenceEngine
from oracle import rwkv4

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    w16 = synthetic.make_weights()
    return w16, cpp_path.init_weights(w16, "cuda", w8a8=True)


def test_w8a8_logits_vs_fp32_oracle(model):
    """Against the unquantised fp32 oracle the deviation is the quantisation
    scheme's own: the oracle's int8 restatement (oracle/quant.py) is itself
    0.135 max-abs / 0.020 mean-abs from fp32 on these random-init weights,
    above north_star's 5e-2 max. The int8 noise is also chaotic: rounding the
    oracle's activations to fp16 before quantising (as the GPU stores them)
    moves its logits by 0.119 max / 0.018 mean. So the kernels are pinned
    exactly where exactness is defined (tests/test_gpu_int8.py: quantisation
    and integer GEMM bit for bit; packed == stepped below) and the model here
    is held to the scheme's error: mean < 5e-2, max < 0.2."""
    w16, W = model
    toks = synthetic.zipf_tokens(2, 24)
    inp = synthetic.model_inputs(toks)
    st = cpp_path.fresh_state_batched(W, 2)
    got = cpp_path.forward_packed_batched(W, inp, st).float().cpu().numpy().reshape(2, 24, -1)
    ref = rwkv4.forward(w16, torch.as_tensor(inp), rwkv4.new_state(12, 2, 768)).numpy()
    d = np.abs(got - ref)
    assert d.mean() < 5e-2, f"int8 logits vs fp32 oracle: mean abs {d.mean()}"
    assert d.max() < 0.2, f"int8 logits vs fp32 oracle: max abs {d.max()}"


@pytest.mark.parametrize("B,T", [(3, 40), (2, 600)])
def test_w8a8_packed_equals_stepped(model, B, T):
    _, W = model
    inp = synthetic.model_inputs(synthetic.zipf_tokens(B, T))
    st = cpp_path.fresh_state_batched(W, B)
    packed = cpp_path.forward_packed_batched(W, inp, st).view(B, T, -1)
    st2 = cpp_path.fresh_state_batched(W, B)
    stepped = torch.stack([cpp_path.forward_stepped_batched(W, inp[:, t], st2)
                           for t in range(T)], dim=1)
    assert torch.equal(packed, stepped)
    assert torch.equal(st.buf, st2.buf)


def test_w8a8_round_trip_and_bits(model):
    w16, _ = model
    toks = [synthetic.zipf_tokens(1, n)[0] for n in (300, 77, 1)]
    e8 = InferenceEngine().load(w16, w8a8=True)
    e16 = InferenceEngine().load(w16)
    enc8 = e8.compress_tokens_batched(toks)
    dec8 = e8.decompress_tokens_batched(enc8)
    for a, b in zip(toks, dec8):
        assert np.array_equal(a, b)
    enc16 = e16.compress_tokens_batched(toks)
    bits8 = sum(len(e) - 8 for e in enc8) * 8
    bits16 = sum(len(e) - 8 for e in enc16) * 8
    ntok = sum(len(t) for t in toks)
    # int8 quantisation moves bits/token by well under a percent on this model
    assert abs(bits8 - bits16) / bits16 < 0.02, (bits8 / ntok, bits16 / ntok)
