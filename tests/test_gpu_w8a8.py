"""The w8a8 codec end to end on the GPU.

The oracle's int8 restatement with the GPU's rounding points
(oracle.rwkv4 with w8a8=True, fp16=True: fp16 activations, LayerNorm in the
GPU row kernel's summation order, kexp in the sigmoid and the WKV update)
reproduces the GPU's int8 codec bit for bit through every layer, so:
  * each layer, fed the GPU's input and the same initial state, gives the
    GPU's output and state exactly (teacher forcing over all 12 layers);
  * the model's logits differ only by the head product's summation order
    (fp16 rounding level).
Beside that: the scheme's deviation from the fp32 oracle (an open deviation
from north_star's 5e-2), packed == stepped bit for bit (the CDFs of compress
and decompress must agree), a byte-exact round trip and its bits/token beside
the fp16 codec's."""
import numpy as np
import pytest
import torch

from krunch_amd import _lib, cpp_path, synthetic
from krunch_amd.inference import InferenceEngine
from krunch_amd.model import State
from oracle import rwkv4

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    w16 = synthetic.make_weights()
    return w16, cpp_path.init_weights(w16, "cuda", w8a8=True)


def _decays(W):
    P = W["prepared"]
    return [P.tensors[f"{i}.decay"].cpu() for i in range(P.n_layer)]


def _gpu_and_oracles(model, B=2, T=24):
    w16, W = model
    inp = synthetic.model_inputs(synthetic.zipf_tokens(B, T))
    st = cpp_path.fresh_state_batched(W, B)
    got = cpp_path.forward_packed_batched(W, inp, st).float().cpu().numpy().reshape(B, T, -1)
    ids = torch.as_tensor(inp)
    q16 = rwkv4.forward(w16, ids, rwkv4.new_state(12, B, 768), w8a8=True, fp16=True,
                        decays=_decays(W)).numpy()
    f32 = rwkv4.forward(w16, ids, rwkv4.new_state(12, B, 768)).numpy()
    return got, q16, f32


@pytest.mark.parametrize("B,T", [(2, 24), (3, 64), (4, 1), (256, 1), (360, 1), (1, 600), (2, 2100)])
def test_w8a8_layers_bit_exact_vs_int8_oracle(model, B, T):
    """Teacher forcing: every layer of the GPU's int8 codec (kr_layer_step:
    LN-mix with int8 outputs, int8 K/V/R + WKV, the output and value products
    quantising their fp16 operands on load) fed the GPU's own input rows and a
    fresh state gives exactly the oracle layer's output and state. B = 256
    and 360, T = 1 run the decode step's fused kernels (at 360 rows the fused
    K/V/R + WKV launch takes 3 x 2 tiles); T > 1 the packed ones (M =
    600: the row quantiser and the tiled int8 GEMM; M = 4200: the persistent
    256 x 128 int8 GEMM)."""
    w16, W = model
    P = W["prepared"]
    ids = torch.as_tensor(synthetic.model_inputs(synthetic.zipf_tokens(B, T, seed_base=77)))
    x = P.tensors["emb"][ids.cuda()].contiguous()
    st = State(P.n_layer, B, P.C, "cuda")
    ws_bytes = _lib.lib().kr_forward_workspace_bytes(B * T, P.C, P.F)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    decays = _decays(W)
    for i in range(P.n_layer):
        x_in = x.float().cpu()
        att_xx, aa, bb, pp, ffn_xx = st._layer(i)
        _lib.call("kr_layer_step", P.layer_ptr(i), P.C, P.F, x.data_ptr(), B, T,
                  att_xx.data_ptr(), aa.data_ptr(), bb.data_ptr(), pp.data_ptr(),
                  ffn_xx.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_ptr())
        ost = rwkv4.new_state(1, B, P.C)[0]
        xo = rwkv4.time_mix(x_in, ost, w16, i, False, True, True, decays[i])
        xo = rwkv4.channel_mix(xo, ost, w16, i, False, True, True)
        d = (x.float().cpu() - xo).abs().max().item()
        assert torch.equal(x.float().cpu(), xo), f"layer {i}: output differs by up to {d}"
        for name, got in (("att_xx", att_xx), ("aa", aa), ("bb", bb), ("pp", pp),
                          ("ffn_xx", ffn_xx)):
            assert torch.equal(got.float().cpu(), ost[name].float()), f"layer {i}: {name}"


def test_w8a8_logits_vs_int8_oracle(model):
    """The whole int8 forward against the oracle's int8 restatement: equal
    through the layers (previous test), so the logits differ only by the head
    product's summation order - within 2e-3 (north_star's fp16 tolerance is
    1e-2)."""
    got, q16, _ = _gpu_and_oracles(model)
    d = np.abs(got - q16)
    assert d.max() < 2e-3, f"int8 logits vs int8 oracle: max abs {d.max()}"
    assert d.mean() < 1e-4, f"int8 logits vs int8 oracle: mean abs {d.mean()}"


def test_w8a8_deviation_from_fp32_is_the_schemes(model):
    """OPEN DEVIATION from north_star (int8 logits within 5e-2 of fp32): the
    prescribed scheme (per-output-channel int8 weights, per-token dynamic
    int8 activations) is itself 0.135 max-abs / 0.020 mean-abs from the fp32
    oracle on these random-init weights, in exact arithmetic (the oracle
    without fp16 rounding) as in the GPU's arithmetic. The GPU logits are
    held to that scheme error: max < 0.2, mean < 5e-2 from fp32, and no
    further from fp32 than the int8 oracle plus 1e-2."""
    got, q16, f32 = _gpu_and_oracles(model)
    d = np.abs(got - f32)
    scheme = np.abs(q16 - f32).max()
    msg = (f"int8 vs fp32: GPU max {d.max():.4f} mean {d.mean():.4f}; the scheme itself "
           f"(int8 oracle) max {scheme:.4f} (open deviation: north_star asks 5e-2)")
    assert d.mean() < 5e-2, msg
    assert d.max() < 0.2, msg
    assert d.max() < scheme + 1e-2, msg


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
