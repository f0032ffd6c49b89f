"""The reference-shaped entry points against the oracle and against each
other: the layer ops of krunch_ac_cuda (rwkv4_layer_step_cpp, _t1, _graphed,
the phase profiler), batched_rwkv4.forward_batched, cpp_path's graphed stepped
forward, krunch_ac.encode/decode on the reference's golden bitstreams, and a
`tokenizers` JSON tokenizer through the engine's container."""
import os

import numpy as np
import pytest
import torch

from krunch_amd import batched_rwkv4, cpp_path, synthetic
from krunch_amd import krunch_ac_hip as ops
from oracle import rwkv4

pytestmark = pytest.mark.gpu

DEV = "cuda"
C = 768


@pytest.fixture(scope="module")
def model():
    w16 = synthetic.make_weights()
    return w16, {k: v.float() for k, v in w16.items()}


def _layer_weights(w16, i):
    """The 18 weight arguments of rwkv4_layer_step_cpp for layer i, in the
    reference's order (cpp_path.py:59-78): time_decay as w = -exp(raw)."""
    a, f, b = f"blocks.{i}.att.", f"blocks.{i}.ffn.", f"blocks.{i}."
    g = lambda k: w16[k].to(DEV)
    return (g(b + "ln1.weight"), g(b + "ln1.bias"), g(a + "time_mix_k"), g(a + "time_mix_v"),
            g(a + "time_mix_r"), -torch.exp(g(a + "time_decay").float()), g(a + "time_first"),
            g(a + "key.weight"), g(a + "value.weight"), g(a + "receptance.weight"),
            g(a + "output.weight"), g(b + "ln2.weight"), g(b + "ln2.bias"), g(f + "time_mix_k"),
            g(f + "time_mix_r"), g(f + "key.weight"), g(f + "value.weight"),
            g(f + "receptance.weight"))


def _gpu_state(B):
    z16 = lambda: torch.zeros(B, C, dtype=torch.float16, device=DEV)
    z32 = lambda: torch.zeros(B, C, dtype=torch.float32, device=DEV)
    return [z16(), z32(), z32(), torch.full((B, C), -1e30, device=DEV), z16()]


def _oracle_layer(w32, i, x, st):
    with torch.no_grad():
        y = rwkv4.time_mix(x, st, w32, i, False)
        return rwkv4.channel_mix(y, st, w32, i, False)


def _check_state(gst, ost):
    for g, key in zip(gst, ("att_xx", "aa", "bb", "pp", "ffn_xx")):
        np.testing.assert_allclose(g.float().cpu().numpy(), ost[key].numpy(), atol=2e-2, rtol=2e-3,
                                   err_msg=key)


@pytest.mark.parametrize("layer", [0, 7])
def test_layer_step_cpp_vs_oracle(model, layer):
    """One layer over [B=2, T=24] in two calls (the second starts from the
    carried state): output x and state within the fp16 tolerance of the fp32
    oracle's time_mix + channel_mix (batched_rwkv4.py:85-172)."""
    w16, w32 = model
    g = torch.Generator().manual_seed(layer)
    x = (torch.randn(2, 24, C, generator=g) * 0.3).half()
    gst, ost = _gpu_state(2), rwkv4.new_state(1, 2, C)[0]
    W = _layer_weights(w16, layer)
    for part in (slice(0, 11), slice(11, 24)):
        xp = x[:, part].contiguous()
        got = ops.rwkv4_layer_step_cpp(xp.to(DEV), *gst, *W)
        ref = _oracle_layer(w32, layer, xp.float(), ost)
        err = (got.float().cpu() - ref).abs().max().item()
        assert err < 1e-2, f"layer {layer}: max abs error {err}"
    _check_state(gst, ost)


def test_layer_step_t1_vs_oracle_and_general_op(model):
    """rwkv4_layer_step_cpp_t1 over 6 successive tokens: the oracle within
    tolerance, and the general op on the same [1, 1, C] input bit for bit."""
    w16, w32 = model
    W = _layer_weights(w16, 3)
    g = torch.Generator().manual_seed(11)
    xs = (torch.randn(6, 1, 1, C, generator=g) * 0.3).half()
    s1, s2, ost = _gpu_state(1), _gpu_state(1), rwkv4.new_state(1, 1, C)[0]
    for t in range(6):
        a = ops.rwkv4_layer_step_cpp_t1(xs[t].to(DEV), *s1, *W)
        b = ops.rwkv4_layer_step_cpp(xs[t].to(DEV), *s2, *W)
        assert torch.equal(a, b)
        ref = _oracle_layer(w32, 3, xs[t].float(), ost)
        assert (a.float().cpu() - ref).abs().max().item() < 1e-2
    for u, v in zip(s1, s2):
        assert torch.equal(u, v)
    _check_state(s1, ost)
    with pytest.raises(RuntimeError):
        ops.rwkv4_layer_step_cpp_t1(xs[0].expand(1, 2, C).contiguous().to(DEV), *s1, *W)


def test_layer_step_graphed_replays_once_per_call(model):
    """Three calls of the graphed op give the ungraphed op's outputs and
    state bit for bit (the state advances once per call, first call included)."""
    w16, _ = model
    W = _layer_weights(w16, 5)
    g = torch.Generator().manual_seed(5)
    xs = [(torch.randn(1, 4, C, generator=g) * 0.3).half().to(DEV) for _ in range(3)]
    x_buf = torch.empty(1, 4, C, dtype=torch.float16, device=DEV)
    x_out = torch.empty_like(x_buf)
    s_graph, s_eager = _gpu_state(1), _gpu_state(1)
    ops.clear_layer_graph_cache()
    try:
        for x in xs:
            x_buf.copy_(x)
            got = ops.rwkv4_layer_step_cpp_graphed(5, x_buf, x_out, *s_graph, *W)
            want = ops.rwkv4_layer_step_cpp(x, *s_eager, *W)
            assert got.data_ptr() == x_out.data_ptr()
            assert torch.equal(got, want)
            for u, v in zip(s_graph, s_eager):
                assert torch.equal(u, v)
    finally:
        ops.clear_layer_graph_cache()


def test_phase_profiler(model):
    w16, _ = model
    W = _layer_weights(w16, 0)
    x = torch.randn(2, 16, C, device=DEV).half()
    st = _gpu_state(2)
    before = ops.set_phase_profile(True)
    try:
        ops.reset_phase_times()
        for _ in range(3):
            ops.rwkv4_layer_step_cpp(x, *st, *W)
        t = ops.read_phase_times()
        assert t["call_count"] == 3
        names = [k for k in t if k != "call_count"]
        assert names == ["ln1_mix", "kvr_matmul", "wkv", "ow_matmul_residual", "ln2_mix",
                         "ffn_rk_matmul", "ffn_v_matmul_residual"]
        assert all(t[k] > 0 for k in names), t      # the general path runs all seven
        ops.reset_phase_times()
        assert ops.read_phase_times()["call_count"] == 0
    finally:
        ops.set_phase_profile(before)
    ops.rwkv4_layer_step_cpp(x, *st, *W)
    assert ops.read_phase_times()["call_count"] == (1 if before else 0)


def test_forward_batched_vs_oracle(model):
    """batched_rwkv4.forward_batched (batched_rwkv4.py:175-262) against the
    fp32 oracle forward, in two calls carrying the state; and full_output=False."""
    w16, w32 = model
    B, T = 2, 20
    inp = synthetic.model_inputs(synthetic.zipf_tokens(B, T))
    m = type("M", (), {})()
    m.w, m.version = w16, 4
    ost = rwkv4.new_state(12, B, C)
    state = None
    for part in (slice(0, 9), slice(9, T)):
        ids = torch.as_tensor(inp[:, part])
        logits, state = batched_rwkv4.forward_batched(m, ids.to(DEV), state)
        ref = rwkv4.forward(w32, ids, ost)
        err = (logits.float().cpu() - ref).abs().max().item()
        assert err < 1e-2, err
    for i in (0, 11):
        np.testing.assert_allclose(state[5 * i + 3].cpu().numpy(), ost[i]["pp"].numpy(),
                                   atol=2e-2, rtol=1e-3)
    st2 = batched_rwkv4.init_state_batched(m, B)
    last, _ = batched_rwkv4.forward_batched(m, torch.as_tensor(inp).to(DEV), st2,
                                           full_output=False)
    full, _ = batched_rwkv4.forward_batched(m, torch.as_tensor(inp).to(DEV))
    assert torch.equal(last, full[:, -1])


def test_forward_stepped_graphed_equals_stepped(model):
    w16, _ = model
    W = cpp_path.init_weights(w16, DEV)
    toks = synthetic.zipf_tokens(1, 6)[0]
    sa, sb = cpp_path.fresh_state(W), cpp_path.fresh_state(W)
    cpp_path.clear_graph_cache()
    try:
        last = 0
        for t in toks:
            a = cpp_path.forward_stepped_graphed(W, last, sa)
            b = cpp_path.forward_stepped(W, last, sb)
            assert torch.equal(a, b)
            last = int(t)
        assert torch.equal(sa.buf, sb.buf)
    finally:
        cpp_path.clear_graph_cache()


def test_krunch_ac_encode_decode_on_golden_bitstreams(golden_dir):
    """krunch_ac.probs_to_cdf / encode / decode (krunch_ac/__init__.py:21-32)
    on the inputs of the reference-written golden vectors: CDF SHA, bitstream
    bytes and decoded symbols all equal."""
    import hashlib
    from krunch_amd import krunch_ac
    from tests.golden import make_golden as mg
    g = np.load(os.path.join(golden_dir, "rc_golden.npz"), allow_pickle=False)
    for idx, (N, V, seed) in enumerate(mg.RC_CASES):
        p = mg.rand_probs(N, V, seed)
        sym = g[f"sym{idx}"]
        cdf = krunch_ac.probs_to_cdf(p)
        sha = hashlib.sha256(np.ascontiguousarray(cdf.astype(np.uint32)).tobytes()).hexdigest()
        assert sha == str(g[f"cdf{idx}_sha"]), (N, V)
        bits = krunch_ac.encode(cdf, sym)
        assert bits == g[f"bits{idx}"].tobytes(), (N, V)
        np.testing.assert_array_equal(krunch_ac.decode(bits, cdf), sym)
        assert krunch_ac.encode_cpu is krunch_ac.encode


def test_json_tokenizer_through_container(tmp_path, model):
    """A `tokenizers` BPE JSON built in-process: the engine tokenizes with it,
    writes tokenizer_id 1 (the reference's, inference.py:51), round-trips
    text byte-exact, and refuses a blob whose tokenizer_id differs."""
    from krunch_amd.inference import InferenceEngine, decode_header
    from tests.test_tokenizer import make_bpe_json
    path = make_bpe_json(tmp_path)
    w16, _ = model
    eng = InferenceEngine().load(w16, tokenizer_path=path)
    assert eng.tokenizer_id == 1
    text = ("The quick brown fox jumps over the lazy dog. " * 30 +
            "Unicode: naïve café — 漢字.\n").encode()
    blob = eng.compress(text, chunk_size=1 << 16)
    assert decode_header(blob)["tokenizer_id"] == 1
    assert eng.decompress(blob) == text
    byte_eng = InferenceEngine().load(w16)
    with pytest.raises(ValueError):
        byte_eng.decompress(blob)
