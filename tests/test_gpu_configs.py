"""Every BASELINE.json configuration at its real shape, against the oracle.

The compress window of a real config runs kernels no toy-shape test reaches:
the persistent 256x128 GEMM with its vectorised epilogues (M = B*T >= 4096),
the packed WKV over T = 1024, the head and CDF in 8192-row blocks. These tests
check them where exactness is defined:
  * logits of sampled streams within 1e-2 max-abs of the fp32 oracle
    (rows are batch-invariant, so the oracle runs on those streams alone);
  * payloads == the oracle range coder fed the oracle CDF of the GPU logits;
  * stepped logits == packed logits bit for bit at every decode step;
  * byte-exact round trips at the config's B and length.
Streams are synthetic Zipf(1.1) token ids on the 169M-shaped random-init
model."""
import numpy as np
import pytest
import torch

from krunch_amd import cpp_path, synthetic
from krunch_amd import krunch_ac_hip as ops
from krunch_amd.inference import CDF_PRECISION, InferenceEngine
from oracle import range_coder as orc
from oracle import rwkv4
from oracle import softmax as osm

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def w16():
    return synthetic.make_weights()


@pytest.fixture(scope="module")
def eng(w16):
    return InferenceEngine().load(w16)


def _oracle_logits(w16, toks):
    st = rwkv4.new_state(12, toks.shape[0], 768)
    return rwkv4.forward(w16, torch.as_tensor(synthetic.model_inputs(toks)), st).numpy()


def _check_payload(payload, logits16, toks):
    """payload == oracle coder on the oracle CDF of these fp16 logits."""
    assert payload[8:] == orc.encode(osm.logits_to_cdf(logits16), toks)


def test_config2_packed_B64_T1024_vs_oracle(eng, w16):
    """Config 2: one packed window of 64 chunks x 1024 tokens (M = 65,536)."""
    B, T = 64, 1024
    toks = synthetic.zipf_tokens(B, T, seed_base=2000)
    enc = eng.compress_tokens_batched(list(toks))
    W = eng.weights
    st = cpp_path.fresh_state_batched(W, B)
    logits = cpp_path.forward_packed_batched(W, synthetic.model_inputs(toks), st).view(B, T, -1)
    sel = [0, B - 1]
    got = logits[sel].cpu().numpy()
    del logits
    ref = _oracle_logits(w16, toks[sel])
    err = np.abs(got.astype(np.float32) - ref).max()
    assert err < 1e-2, f"config 2 logits vs fp32 oracle: max abs {err}"
    for i, b in enumerate(sel):
        _check_payload(enc[b], got[i], toks[b])
        # bits/token within 0.5% of the fp32 oracle's own chain (its logits,
        # its CDF, its coder) on the same stream
        ref_bits = 8 * len(orc.encode(osm.logits_to_cdf(ref[i]), toks[b]))
        gpu_bits = 8 * (len(enc[b]) - 8)
        assert abs(gpu_bits - ref_bits) / ref_bits < 0.005, (b, gpu_bits / T, ref_bits / T)


def test_config3_stepped_B128_1024_steps(eng):
    """Config 3: 128 streams decoded in lockstep for 1024 steps, byte-exact;
    the stepped logits equal the packed logits bit for bit at every step, and
    at sampled steps the decoded symbol's CDF interval from the full CDF of
    the stepped row equals the interval the compress side encoded."""
    B, T = 128, 1024
    toks = synthetic.zipf_tokens(B, T, seed_base=3000)
    enc = eng.compress_tokens_batched(list(toks))
    dec = eng.decompress_tokens_batched(enc)
    for t, d in zip(toks, dec):
        np.testing.assert_array_equal(d, t)
    W = eng.weights
    inp = torch.as_tensor(synthetic.model_inputs(toks), device=DEV)
    tok_d = torch.as_tensor(toks, device=DEV)
    st = cpp_path.fresh_state_batched(W, B)
    packed = cpp_path.forward_packed_batched(W, inp, st).view(B, T, -1)
    st2 = cpp_path.fresh_state_batched(W, B)
    sampled = {0, 1, 511, 1023}
    for t in range(T):
        stepped = cpp_path.forward_stepped_batched(W, inp[:, t], st2)
        assert torch.equal(stepped, packed[:, t]), f"step {t}"
        if t in sampled:
            cdf = ops.softmax_cdf(stepped)                      # decode side, full rows
            sym = tok_d[:, t].to(torch.int32).contiguous()
            pairs = torch.empty((B, 2), dtype=torch.int32, device=DEV)
            rows = packed[:, t].contiguous()                    # compress side
            from krunch_amd import _lib
            _lib.call("kr_softmax_cdf_pairs", rows.data_ptr(), B, rows.shape[1], rows.shape[1],
                      sym.data_ptr(), pairs.data_ptr(), 24, _lib.stream_ptr())
            lo = cdf.gather(1, sym.long().unsqueeze(1)).squeeze(1)
            hi = cdf.gather(1, sym.long().unsqueeze(1) + 1).squeeze(1)
            assert torch.equal(pairs[:, 0], lo) and torch.equal(pairs[:, 1], hi), f"step {t}"
    assert torch.equal(st.buf, st2.buf)


def test_config4_w8a8_B256_T1024(eng, w16):
    """Config 4: the w8a8 codec on 256 chunks x 1024 tokens (M = 262,144):
    byte-exact round trip; bits/token within 0.5% of the fp16 codec's."""
    B, T = 256, 1024
    toks = synthetic.zipf_tokens(B, T, seed_base=4000)
    e8 = InferenceEngine().load(w16, w8a8=True)
    enc8 = e8.compress_tokens_batched(list(toks))
    dec8 = e8.decompress_tokens_batched(enc8)
    for t, d in zip(toks, dec8):
        np.testing.assert_array_equal(d, t)
    enc16 = eng.compress_tokens_batched(list(toks))
    b8 = sum(len(e) - 8 for e in enc8)
    b16 = sum(len(e) - 8 for e in enc16)
    assert abs(b8 - b16) / b16 < 0.005, (8 * b8 / (B * T), 8 * b16 / (B * T))


def test_config5_three_windows_with_repeats(eng, w16):
    """Config 5 over three 1024-token windows (state carried across windows
    on both sides) of 256 chunks with 5% repeated 64-token spans: byte-exact;
    one stream's payload equals the oracle chain on the logits of a single
    packed call over all 3072 tokens, and those logits are within 1e-2 of the
    fp32 oracle (the carried state stays on track over three windows)."""
    B, T = 256, 3072
    toks = synthetic.zipf_tokens(B, T, repeat_rate=0.05, seed_base=5000)
    enc = eng.compress_tokens_batched(list(toks))
    dec = eng.decompress_tokens_batched(enc)
    for t, d in zip(toks, dec):
        np.testing.assert_array_equal(d, t)
    W = eng.weights
    b = B - 1
    st = cpp_path.fresh_state_batched(W, 1)
    got = cpp_path.forward_packed_batched(W, synthetic.model_inputs(toks[b:b + 1]), st)
    got = got.cpu().numpy()
    _check_payload(enc[b], got, toks[b])
    ref = _oracle_logits(w16, toks[b:b + 1])[0]
    err = np.abs(got.astype(np.float32) - ref).max()
    assert err < 1e-2, f"config 5 logits vs fp32 oracle after 3 windows: max abs {err}"


def _decode_in_calls(eng, enc, calls, report):
    """Lockstep decode of every stream through kr_decode_run, split into
    `calls` calls of equal step counts (the state, coder state and decoded
    symbols carry over; split calls give the bits of one call). Returns
    [B, Tmax] int32 tokens on the host."""
    import struct
    from krunch_amd import _lib
    from krunch_amd.model import State
    P = eng.weights["prepared"]
    B = len(enc)
    n_tok = [struct.unpack(">II", e[:8])[1] for e in enc]
    streams = [e[8:] for e in enc]
    offs = np.cumsum([0] + [len(s) for s in streams])
    inbuf = torch.from_numpy(np.frombuffer(b"".join(streams) + b"\0", dtype=np.uint8).copy()).to(DEV)
    base = torch.from_numpy(offs[:-1].astype(np.int32)).to(DEV)
    limits = torch.tensor([len(s) for s in streams], dtype=torch.int32, device=DEV)
    ac = torch.empty((B, 4), dtype=torch.uint32, device=DEV)
    s = _lib.stream_ptr()
    _lib.call("kr_decode_init_batched", inbuf.data_ptr(), inbuf.numel(), base.data_ptr(),
              limits.data_ptr(), ac.data_ptr(), B, s)
    Tmax = max(n_tok)
    state = State(P.n_layer, B, P.C, DEV)
    syms = torch.zeros(B, dtype=torch.int32, device=DEV)
    tokens = torch.zeros((B, Tmax), dtype=torch.int32, device=DEV)
    count = torch.zeros(B, dtype=torch.int32, device=DEV)
    ntd = torch.tensor(n_tok, dtype=torch.int32, device=DEV)
    x = torch.empty((B, P.C), dtype=torch.float16, device=DEV)
    nbytes = _lib.lib().kr_decode_workspace_bytes(B, 1, P.C, P.F)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    ld = cpp_path.logits_ld(P.V)
    logits = torch.empty((B, ld), dtype=torch.float16, device=DEV)
    step = (Tmax + calls - 1) // calls
    for c in range(calls):
        n = min(step, Tmax - c * step)
        _lib.call("kr_decode_run", P.ptr, B, state.ptr, syms.data_ptr(), x.data_ptr(),
                  ws.data_ptr(), nbytes, logits.data_ptr(), ld, inbuf.data_ptr(), inbuf.numel(),
                  base.data_ptr(), limits.data_ptr(), ac.data_ptr(), tokens.data_ptr(), Tmax,
                  count.data_ptr(), ntd.data_ptr(), CDF_PRECISION, n, 1, 1, s)
        torch.cuda.synchronize()
        report(f"decoded {(c + 1) * step if c + 1 < calls else Tmax} of {Tmax} steps")
    assert torch.equal(count.cpu(), ntd.cpu())
    return tokens.cpu().numpy()


def test_config5_whole(eng, capsys):
    """Config 5 whole: 256 chunks of 262,144 tokens (5% repeated 64-token
    spans), compressed in 256 windows of 1024 tokens with the state carried
    across windows, then decoded in 262,144 lockstep steps of 256 streams:
    byte-exact. The first 3,072 tokens of one stream's payload equal the
    oracle coder fed the oracle CDF of that stream's GPU logits (the bits a
    range coder has emitted after n symbols do not depend on later symbols,
    so the whole stream's prefix equals the n-symbol stream's, short of the
    final flush). Progress lines go straight to the terminal: the test runs
    for about three minutes."""
    def report(msg):
        with capsys.disabled():
            print(f"[config 5 whole] {msg}", flush=True)
    B, T = 256, 262144
    toks = synthetic.zipf_tokens(B, T, repeat_rate=0.05, seed_base=5500)
    report("tokens drawn; compressing")
    enc = eng.compress_tokens_batched(list(toks))
    bpt = 8 * sum(len(e) - 8 for e in enc) / (B * T)
    report(f"compressed: {bpt:.3f} bits/token")
    assert 8.0 < bpt < 17.0, bpt
    b, n = 97, 3072
    st = cpp_path.fresh_state_batched(eng.weights, 1)
    got = cpp_path.forward_packed_batched(eng.weights, synthetic.model_inputs(toks[b:b + 1, :n]), st)
    ref = orc.encode(osm.logits_to_cdf(got.cpu().numpy()), toks[b, :n])
    # the n-symbol stream ends with a flush of pending + 2 bits and a partial
    # byte: 8 bytes cover it unless 55 E3 steps were pending at once
    keep = len(ref) - 8
    assert enc[b][8:8 + keep] == ref[:keep], "stream 97: payload prefix differs from the oracle chain"
    dec = _decode_in_calls(eng, enc, 8, report)
    for i in range(B):
        np.testing.assert_array_equal(dec[i], toks[i], err_msg=f"stream {i}")
