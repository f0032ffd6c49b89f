"""Forward on the 169M-shaped synthetic model: fp16 GPU logits against the
fp32 CPU oracle (1e-2 max-abs), and the invariants that make the codec
round-trip: packed == stepped, windowed == single-shot, batched == alone —
all bit for bit."""
import numpy as np
import pytest
import torch

from krunch_amd import batched_rwkv4, cpp_path, synthetic
from krunch_amd import krunch_ac_hip as ops
from oracle import rwkv4

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    w16 = synthetic.make_weights()
    return w16, cpp_path.init_weights(w16, "cuda")


def test_logits_match_fp32_oracle(model):
    w16, W = model
    toks = synthetic.zipf_tokens(2, 24)
    inp = synthetic.model_inputs(toks)
    st = cpp_path.fresh_state_batched(W, 2)
    got = cpp_path.forward_packed_batched(W, inp, st).float().cpu().numpy().reshape(2, 24, -1)
    ost = rwkv4.new_state(12, 2, 768)
    ref = rwkv4.forward(w16, torch.as_tensor(inp), ost).numpy()
    err = np.abs(got - ref).max()
    assert err < 1e-2, f"max abs logit error {err}"
    # the carried state too
    for i in (0, 11):
        np.testing.assert_allclose(st[3][i].cpu().numpy(), ost[i]["pp"].numpy(), atol=2e-2, rtol=1e-3)


@pytest.mark.parametrize("B,T", [(3, 40), (2, 600)])
def test_packed_equals_stepped_and_windowed(model, B, T):
    """(3, 40): both sides on the small-M kernel; (2, 600): packed on the
    LDS-tiled kernel, stepped on the split-K small-M kernel."""
    _, W = model
    inp = synthetic.model_inputs(synthetic.zipf_tokens(B, T))
    st = cpp_path.fresh_state_batched(W, B)
    packed = cpp_path.forward_packed_batched(W, inp, st).view(B, T, -1)
    st2 = cpp_path.fresh_state_batched(W, B)
    stepped = torch.stack([cpp_path.forward_stepped_batched(W, inp[:, t], st2)
                           for t in range(T)], dim=1)
    assert torch.equal(packed, stepped)
    assert torch.equal(st.buf, st2.buf)
    st3 = cpp_path.fresh_state_batched(W, B)
    a = cpp_path.forward_packed_batched(W, inp[:, :17], st3).view(B, 17, -1)
    b = cpp_path.forward_packed_batched(W, inp[:, 17:], st3).view(B, T - 17, -1)
    assert torch.equal(packed, torch.cat([a, b], dim=1))


def test_batched_equals_alone(model):
    _, W = model
    B, T = 4, 33
    inp = synthetic.model_inputs(synthetic.zipf_tokens(B, T))
    st = cpp_path.fresh_state_batched(W, B)
    both = cpp_path.forward_packed_batched(W, inp, st).view(B, T, -1)
    for b in (0, 3):
        s1 = cpp_path.fresh_state_batched(W, 1)
        alone = cpp_path.forward_packed_batched(W, inp[b:b + 1], s1).view(1, T, -1)
        assert torch.equal(both[b:b + 1], alone)


def test_reference_shaped_entry_points_agree(model):
    """batched_rwkv4.forward_batched and krunch_ac_cuda-style
    rwkv4_layer_step_cpp give the engine's bits."""
    w16, W = model
    B, T = 2, 9
    inp = synthetic.model_inputs(synthetic.zipf_tokens(B, T))
    st = cpp_path.fresh_state_batched(W, B)
    eng = cpp_path.forward_packed_batched(W, inp, st).view(B, T, -1)
    m = type("M", (), {})()
    m.w, m.version = w16, 4
    logits, state = batched_rwkv4.forward_batched(m, torch.as_tensor(inp))
    assert torch.equal(logits, eng)
    # one layer through the reference-shaped op
    dev = "cuda"
    x = w16["emb.weight"].to(dev)[torch.as_tensor(inp, device=dev).long()].contiguous()
    s = cpp_path.fresh_state_batched(W, B)
    a = f"blocks.0.att."
    f = f"blocks.0.ffn."
    g = lambda k: w16[k].to(dev)
    y = ops.rwkv4_layer_step_cpp(
        x, s[0][0], s[1][0], s[2][0], s[3][0], s[4][0], g("blocks.0.ln1.weight"),
        g("blocks.0.ln1.bias"), g(a + "time_mix_k"), g(a + "time_mix_v"), g(a + "time_mix_r"),
        -torch.exp(g(a + "time_decay")), g(a + "time_first"), g(a + "key.weight"),
        g(a + "value.weight"), g(a + "receptance.weight"), g(a + "output.weight"),
        g("blocks.0.ln2.weight"), g("blocks.0.ln2.bias"), g(f + "time_mix_k"), g(f + "time_mix_r"),
        g(f + "key.weight"), g(f + "value.weight"), g(f + "receptance.weight"))
    assert y.shape == x.shape and torch.isfinite(y.float()).all()


def _row_major_only(P):
    """A model descriptor sharing P's tensors with the fragment-packed
    pointers cleared, so every GEMM reads the row-major weights."""
    from krunch_amd import _lib
    import ctypes
    layers = (_lib.KrLayerWeights * P.n_layer)()
    for i in range(P.n_layer):
        ctypes.memmove(ctypes.byref(layers[i]), ctypes.byref(P.layers_c[i]),
                       ctypes.sizeof(_lib.KrLayerWeights))
        for name in ("Kf", "Vf", "Rf", "Of", "fKf", "fVf", "fRf"):
            setattr(layers[i], name, None)
    m = _lib.KrModelWeights(P.n_layer, P.C, P.F, P.V, P.model_c.emb, P.model_c.ln_out_w,
                            P.model_c.ln_out_b, P.model_c.headT,
                            ctypes.cast(layers, ctypes.POINTER(_lib.KrLayerWeights)))
    return m, layers


@pytest.mark.parametrize("B", [1, 37, 256, 360])
def test_fragment_path_equals_row_major_path(model, B):
    """Small-M layers with fragment-packed operands give the row-major
    path's bits (outputs and carried state), over two steps. At 360 rows the
    fused K/V/R + WKV launch takes 3 x 2 tiles."""
    from krunch_amd import _lib
    import ctypes
    _, W = model
    P = W["prepared"]
    m_row, _keep = _row_major_only(P)
    ids = torch.as_tensor(synthetic.zipf_tokens(B, 2), dtype=torch.int32, device="cuda")
    outs = []
    for mdesc in (P.model_c, m_row):
        st = cpp_path.fresh_state_batched(W, B)
        ws, nb = cpp_path.workspace(W, B)
        x = torch.empty((B, P.C), dtype=torch.float16, device="cuda")
        seq = []
        for t in range(2):
            _lib.call("kr_embed", ctypes.byref(mdesc), ids[:, t].contiguous().data_ptr(), B,
                      x.data_ptr(), _lib.stream_ptr())
            _lib.call("kr_forward_layers", ctypes.byref(mdesc), x.data_ptr(), B, 1, st.ptr,
                      ws.data_ptr(), nb, _lib.stream_ptr())
            seq.append(x.clone())
        outs.append((torch.stack(seq), st.buf.clone()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])


def test_pack_fragments_layout():
    """kr_pack_fragments: block (rb, kb) is the 16x32 tile, lane r + 16*g
    holds its 8 columns 8g..8g+7 (checked by reshaping, not by the index)."""
    from krunch_amd import _lib
    N, K = 40, 96
    Wt = torch.randn(N, K, device="cuda").half()
    nbytes = _lib.lib().kr_fragment_bytes(N, K)
    assert nbytes == 48 * K * 2
    out = torch.empty(nbytes // 2, dtype=torch.float16, device="cuda")
    _lib.call("kr_pack_fragments", Wt.data_ptr(), K, N, K, out.data_ptr(), _lib.stream_ptr())
    pad = torch.zeros(48, K, dtype=torch.float16, device="cuda")
    pad[:N] = Wt
    want = pad.view(3, 16, K // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(-1)
    assert torch.equal(out, want)


@pytest.mark.parametrize("M", [16, 48, 256, 400, 512])
def test_small_head_equals_tiled_head(model, M):
    """The decode head (A held in registers, fragment-packed weights streamed
    once; one launch up to 512 rows) gives the large-M head kernel's
    logits (256 x 256 tiles, row-major operands) bit for bit: the head's
    one-chain contract. Includes the 5-column tail block of V = 50277 and a
    padded row stride."""
    from krunch_amd import _lib
    import ctypes
    _, W = model
    P = W["prepared"]
    m_row, _keep = _row_major_only(P)      # no fragment-packed head
    g = torch.Generator(device="cpu").manual_seed(M)
    x = torch.randn((M, P.C), generator=g).half().cuda()
    ld = P.V + 3
    outs = []
    for mdesc in (P.model_c, m_row):
        xn = torch.empty((M, P.C), dtype=torch.float16, device="cuda")
        logits = torch.full((M, ld), float("nan"), dtype=torch.float16, device="cuda")
        _lib.call("kr_head_logits", ctypes.byref(mdesc), x.data_ptr(), M, xn.data_ptr(),
                  logits.data_ptr(), ld, _lib.stream_ptr())
        outs.append(logits)
    assert torch.equal(outs[0][:, :P.V], outs[1][:, :P.V])
    assert torch.isnan(outs[0][:, P.V:]).all()       # padding columns untouched
    ref = torch.nn.functional.layer_norm(x.float(), (P.C,), eps=1e-5) @ \
        P.tensors["headT"].float().t()
    assert (outs[0][:, :P.V].float() - ref).abs().max() < 2e-2


@pytest.mark.parametrize("C,V,M,pad", [(256, 1000, 144, 8), (512, 1000, 256, 3),
                                       (768, 2051, 144, 8), (768, 1000, 48, 3)])
def test_small_head_small_vocab(C, V, M, pad):
    """The decode head where the vocabulary has fewer 16-column blocks than
    the launch has column runs for (63 runs: row groups and runs dealt in
    workgroup order; 129 blocks: 128 runs of one or two blocks), with a
    second row group of 16 rows (M = 144), one group (M = 48), K = 256, 512
    and 768, vector and scalar stores: the large-M head's bits."""
    from krunch_amd import _lib
    import ctypes
    w16 = synthetic.make_weights(n_layer=1, C=C, F=2 * C, V=V, seed=C + V)
    W = cpp_path.init_weights(w16, "cuda")
    try:
        P = W["prepared"]
        m_row, _keep = _row_major_only(P)
        g = torch.Generator(device="cpu").manual_seed(M)
        x = torch.randn((M, C), generator=g).half().cuda()
        ld = V + pad
        outs = []
        for mdesc in (P.model_c, m_row):
            xn = torch.empty((M, C), dtype=torch.float16, device="cuda")
            logits = torch.full((M, ld), float("nan"), dtype=torch.float16, device="cuda")
            _lib.call("kr_head_logits", ctypes.byref(mdesc), x.data_ptr(), M, xn.data_ptr(),
                      logits.data_ptr(), ld, _lib.stream_ptr())
            outs.append(logits)
        assert torch.equal(outs[0][:, :V], outs[1][:, :V])
        assert torch.isnan(outs[0][:, V:]).all()
        ref = torch.nn.functional.layer_norm(x.float(), (C,), eps=1e-5) @ \
            P.tensors["headT"].float().t()
        assert (outs[0][:, :V].float() - ref).abs().max() < 2e-2
    finally:
        cpp_path.release_weights(w16)


@pytest.mark.parametrize("M", [1000, 4096 + 37])
def test_large_m_head_rows_equal_decode_head_rows(model, M):
    """A row's logits are the same bits whichever head kernel computes it and
    however many rows share the call: the large-M head at M rows (ragged last
    row tile, 5-column tail) against the decode head on 256-row slices of the
    same rows (first, middle and last)."""
    from krunch_amd import _lib
    import ctypes
    _, W = model
    P = W["prepared"]
    m_row, _keep = _row_major_only(P)      # no fragment-packed head: the large-M kernel
    g = torch.Generator(device="cpu").manual_seed(M)
    x = torch.randn((M, P.C), generator=g).half().cuda()
    ld = cpp_path.logits_ld(P.V)
    xn = torch.empty((M, P.C), dtype=torch.float16, device="cuda")
    big = torch.full((M, ld), float("nan"), dtype=torch.float16, device="cuda")
    _lib.call("kr_head_logits", ctypes.byref(m_row), x.data_ptr(), M, xn.data_ptr(),
              big.data_ptr(), ld, _lib.stream_ptr())
    for r0 in (0, M // 2 - 128, M - 256):
        xs = x[r0:r0 + 256].contiguous()
        xns = torch.empty((256, P.C), dtype=torch.float16, device="cuda")
        small = torch.full((256, ld), float("nan"), dtype=torch.float16, device="cuda")
        _lib.call("kr_head_logits", P.ptr, xs.data_ptr(), 256, xns.data_ptr(), small.data_ptr(),
                  ld, _lib.stream_ptr())
        assert torch.equal(big[r0:r0 + 256, :P.V], small[:, :P.V]), f"rows {r0}.."
    assert torch.isnan(big[:, P.V:]).all()           # padding columns untouched
    ref = torch.nn.functional.layer_norm(x.float(), (P.C,), eps=1e-5) @ \
        P.tensors["headT"].float().t()
    assert (big[:, :P.V].float() - ref).abs().max() < 2e-2
