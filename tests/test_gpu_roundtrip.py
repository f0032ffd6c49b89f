"""End to end on the GPU: compress B chunks (packed windows, state carried)
and decompress them in lockstep (fused decode, HIP graph). Byte-exact round
trips; the bitstream equals the oracle coder fed the oracle CDF of the GPU
logits; bits/token within 0.5% of the fp32 oracle's."""
import struct

import numpy as np
import pytest
import torch

from krunch_amd import cpp_path, synthetic
from krunch_amd.inference import InferenceEngine, decode_header, encode_header, HEADER_SIZE
from oracle import range_coder as orc
from oracle import rwkv4
from oracle import softmax as osm

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = InferenceEngine()
    e.window = 64
    return e.load(synthetic.make_weights())


def test_roundtrip_ragged_streams(eng):
    lens = [50, 300, 64 * 3 + 37, 7, 1]
    toks = [synthetic.zipf_tokens(1, n, seed_base=500 + i)[0] for i, n in enumerate(lens)]
    enc = eng.compress_tokens_batched(toks)
    dec = eng.decompress_tokens_batched(enc)
    for t, d in zip(toks, dec):
        np.testing.assert_array_equal(d, t)
    eng.use_graph = False
    dec2 = eng.decompress_tokens_batched(enc)
    eng.use_graph = True
    for t, d in zip(toks, dec2):
        np.testing.assert_array_equal(d, t)


@pytest.mark.parametrize("B", [37, 200, 300])
def test_roundtrip_many_streams(eng, B):
    """Decode steps of 37, 200 and 300 streams: the decode head's last row
    block is partial; at 200 its second row group holds 72 rows; at 300 it
    runs three row groups of 128 rows per column run, the last holding 44."""
    toks = [synthetic.zipf_tokens(1, 12 + (i % 5), seed_base=1300 + i)[0] for i in range(B)]
    enc = eng.compress_tokens_batched(toks)
    dec = eng.decompress_tokens_batched(enc)
    for t, d in zip(toks, dec):
        np.testing.assert_array_equal(d, t)


def test_split_batches_are_byte_identical(eng, monkeypatch):
    """Jobs larger than the stream batch run as several lockstep calls; every
    stream's payload and tokens are the same as in one call (streams are
    independent and every kernel is row-local in its bits)."""
    toks = [synthetic.zipf_tokens(1, 20 + 9 * i, seed_base=1700 + i)[0] for i in range(7)]
    whole = eng.compress_tokens_batched(toks)
    monkeypatch.setenv("KRUNCH_COMPRESS_BATCH", "3")
    monkeypatch.setenv("KRUNCH_DECOMPRESS_BATCH", "2")
    split = eng.compress_tokens_batched(toks)
    assert split == whole
    for t, d in zip(toks, eng.decompress_tokens_batched(whole)):
        np.testing.assert_array_equal(d, t)


def test_calls_split_by_coder_bytes(eng):
    """A small per-call coder-byte cap forces compress and decompress to run
    as several calls (the path that keeps int32 stream offsets and the
    uint32 buffer length of the C ABI in range on very large jobs): payloads
    and tokens are the same as in one call."""
    toks = [synthetic.zipf_tokens(1, 40 + 13 * i, seed_base=2100 + i)[0] for i in range(6)]
    whole = eng.compress_tokens_batched(toks)
    saved = eng.max_call_bytes
    try:
        # 2 streams of the longest (105 tokens: 484 coder bytes) per compress call
        eng.max_call_bytes = 1000
        split = eng.compress_tokens_batched(toks)
        assert split == whole
        eng.max_call_bytes = max(len(e) for e in whole) + 1      # one stream per decode call
        for t, d in zip(toks, eng.decompress_tokens_batched(whole)):
            np.testing.assert_array_equal(d, t)
        eng.max_call_bytes = 10
        with pytest.raises(ValueError):
            eng.compress_tokens_batched(toks[:1])
    finally:
        eng.max_call_bytes = saved


def test_decode_groups_and_graph_agree(eng):
    """Concurrent decode groups (graph branches) and the eager path decode the
    same tokens as one group."""
    toks = [synthetic.zipf_tokens(1, n, seed_base=900 + i)[0] for i, n in enumerate([90, 33, 70, 12, 64, 5, 41])]
    enc = eng.compress_tokens_batched(toks)
    outs = []
    for groups, graph in ((1, True), (3, True), (7, True), (4, False)):
        eng.decode_groups, eng.use_graph = groups, graph
        outs.append(eng.decompress_tokens_batched(enc))
    eng.decode_groups, eng.use_graph = 4, True
    for dec in outs:
        for t, d in zip(toks, dec):
            np.testing.assert_array_equal(d, t)


@pytest.mark.parametrize("layer", [5, 11])
def test_graph_decode_with_an_unpacked_later_layer(eng, layer):
    """A layer with no fragment-packed weights runs on the unfused small-M
    path, which writes the workspace rows and buffer that the graph decode's
    layer-0 LN1-mix fold keeps its carried rows and its argument block in.
    The fold must then stay off: the graph and the eager decode of such a
    model both give back the tokens (every path keeps the same bits)."""
    toks = [synthetic.zipf_tokens(1, n, seed_base=4100 + i)[0] for i, n in enumerate([30, 9, 22, 1])]
    enc = eng.compress_tokens_batched(toks)
    L = eng.weights["prepared"].layers_c[layer]
    saved = (L.Kf, L.fVf)
    L.Kf, L.fVf = None, None
    try:
        for graph in (True, False):
            eng.use_graph = graph
            dec = eng.decompress_tokens_batched(enc)
            for t, d in zip(toks, dec):
                np.testing.assert_array_equal(d, t, err_msg=f"graph={graph}, layer {layer} unpacked")
    finally:
        L.Kf, L.fVf = saved
        eng.use_graph = True


def test_repeated_spans_roundtrip(eng):
    toks = synthetic.zipf_tokens(3, 640, repeat_rate=0.3)
    enc = eng.compress_tokens_batched(list(toks))
    dec = eng.decompress_tokens_batched(enc)
    for t, d in zip(toks, dec):
        np.testing.assert_array_equal(d, t)


def test_bitstream_equals_oracle_chain(eng):
    toks = synthetic.zipf_tokens(2, 150)
    enc = eng.compress_tokens_batched(list(toks))
    W = eng.weights
    st = cpp_path.fresh_state_batched(W, 2)
    logits = cpp_path.forward_packed_batched(W, synthetic.model_inputs(toks), st)
    logits = logits.view(2, 150, -1).cpu().numpy()
    for b in range(2):
        ref = orc.encode(osm.logits_to_cdf(logits[b]), toks[b])
        assert enc[b][8:] == ref


def test_chunk_payloads_equal_oracle_chain(eng):
    """Byte-level chunks (reference inference.py:576-660 compress_chunks_batched):
    each payload is the ">II" (orig_len, n_tokens) mini-header and then the
    oracle coder's bits on the oracle CDF of the GPU logits of the chunk's
    byte-tokenized stream; ragged chunks share one batched call."""
    from krunch_amd.tokenizer import ByteTokenizer
    chunks = [b"The quick brown fox jumps over the lazy dog. " * 3,
              bytes(range(200)), "Grüße, 世界!".encode("utf-8") * 5, b"x"]
    enc = eng.compress_chunks_batched(chunks)
    assert eng.decompress_chunks_batched(enc) == chunks
    tok = ByteTokenizer()
    W = eng.weights
    for c, e in zip(chunks, enc):
        ids = tok.encode_bytes(c)
        assert struct.unpack(">II", e[:8]) == (len(c), len(ids))
        st = cpp_path.fresh_state_batched(W, 1)
        logits = cpp_path.forward_packed_batched(W, synthetic.model_inputs(ids[None, :]), st)
        logits = logits.view(len(ids), -1).cpu().numpy()
        assert e[8:] == orc.encode(osm.logits_to_cdf(logits), ids)


def test_bits_per_token_close_to_fp32_oracle(eng):
    toks = synthetic.zipf_tokens(1, 200)
    enc = eng.compress_tokens_batched(list(toks))
    gpu_bits = 8 * (len(enc[0]) - 8)
    w16 = synthetic.make_weights()
    st = rwkv4.new_state(12, 1, 768)
    ref = rwkv4.forward(w16, torch.as_tensor(synthetic.model_inputs(toks)), st)[0].numpy()
    cdf = osm.logits_to_cdf(ref)
    oracle_bits = 8 * len(orc.encode(cdf, toks[0]))
    assert abs(gpu_bits - oracle_bits) / oracle_bits < 0.005


def test_blob_header_roundtrip():
    h = encode_header(original_len=123456, n_chunks=7, crc32=0xDEADBEEF)
    assert len(h) == HEADER_SIZE == 37
    d = decode_header(h)
    assert (d["original_len"], d["n_chunks"], d["crc32"], d["model_id"]) == (123456, 7, 0xDEADBEEF, 1)


def _decode_direct(eng, enc, splits, use_graph):
    """kr_decode_run over `enc` in len(splits) calls of splits[i] steps each;
    returns every buffer the calls leave behind (tokens, counts, coder and
    model state, next symbols)."""
    from krunch_amd import _lib
    from krunch_amd.inference import CDF_PRECISION
    from krunch_amd.model import State
    P = eng.weights["prepared"]
    dev = P.device
    B = len(enc)
    n_tok = [struct.unpack(">II", e[:8])[1] for e in enc]
    streams = [e[8:] for e in enc]
    offs = np.cumsum([0] + [len(s) for s in streams])
    inbuf = torch.from_numpy(np.frombuffer(b"".join(streams) + b"\0", dtype=np.uint8).copy()).to(dev)
    base = torch.from_numpy(offs[:-1].astype(np.int32)).to(dev)
    limits = torch.tensor([len(s) for s in streams], dtype=torch.int32, device=dev)
    ac = torch.empty((B, 4), dtype=torch.uint32, device=dev)
    s = _lib.stream_ptr()
    _lib.call("kr_decode_init_batched", inbuf.data_ptr(), inbuf.numel(), base.data_ptr(),
              limits.data_ptr(), ac.data_ptr(), B, s)
    Tmax = max(n_tok)
    state = State(P.n_layer, B, P.C, dev)
    syms = torch.zeros(B, dtype=torch.int32, device=dev)
    tokens = torch.zeros((B, Tmax), dtype=torch.int32, device=dev)
    count = torch.zeros(B, dtype=torch.int32, device=dev)
    ntd = torch.tensor(n_tok, dtype=torch.int32, device=dev)
    x = torch.empty((B, P.C), dtype=torch.float16, device=dev)
    nbytes = _lib.lib().kr_decode_workspace_bytes(B, 1, P.C, P.F)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    ld = cpp_path.logits_ld(P.V)
    logits = torch.empty((B, ld), dtype=torch.float16, device=dev)
    for n in splits:
        _lib.call("kr_decode_run", P.ptr, B, state.ptr, syms.data_ptr(), x.data_ptr(),
                  ws.data_ptr(), nbytes, logits.data_ptr(), ld, inbuf.data_ptr(), inbuf.numel(),
                  base.data_ptr(), limits.data_ptr(), ac.data_ptr(), tokens.data_ptr(), Tmax,
                  count.data_ptr(), ntd.data_ptr(), CDF_PRECISION, n, 1, 1 if use_graph else 0, s)
    torch.cuda.synchronize()
    return [t.cpu() for t in (tokens, count, ac, syms, state.buf)]


@pytest.fixture(scope="module")
def eng_w8a8():
    e = InferenceEngine()
    e.window = 64
    return e.load(synthetic.make_weights(), w8a8=True)


@pytest.mark.parametrize("codec", ["fp16", "w8a8"])
def test_graph_decode_leaves_the_eager_state(eng, eng_w8a8, codec):
    """The graph decode runs layer 0's LN1-mix of each decoded symbol inside
    that step's decode kernel and carries layer 0's shifted row one step
    late. Split over calls of any length, it leaves the model state, coder
    state and tokens byte-equal to the eager decode (which runs every layer's
    own LN1-mix), also for streams that finished before the last step. The
    w8a8 codec's layer 0 writes its mixes quantised per row there."""
    eng = eng_w8a8 if codec == "w8a8" else eng
    lens = [40, 17, 33, 5, 1]
    toks = [synthetic.zipf_tokens(1, n, seed_base=3100 + i)[0] for i, n in enumerate(lens)]
    enc = eng.compress_tokens_batched(toks)
    ref = _decode_direct(eng, enc, [45], use_graph=False)
    for b, t in enumerate(toks):
        np.testing.assert_array_equal(ref[0][b, :len(t)].numpy(), t)
    for splits in ([45], [20, 25], [1, 1, 43], [17, 3, 25]):
        got = _decode_direct(eng, enc, splits, use_graph=True)
        for name, a, g in zip(("tokens", "count", "coder", "syms", "model state"), ref, got):
            assert torch.equal(a, g), f"{name} differs after calls of {splits} steps"


@pytest.mark.parametrize("graph,phase", [(True, 5), (False, 6), (True, 3)])
def test_step_timing_changes_nothing_and_reports_each_layer(eng, graph, phase):
    """kr_step_timing: the timed product of every layer stores its waves'
    start and end (and, eagerly launched, takes dispatch events); decoding
    with it on gives the bits of decoding with it off, and it reports one
    positive duration per layer (no event duration for a graph step)."""
    import ctypes
    from krunch_amd import _lib
    toks = [synthetic.zipf_tokens(1, n, seed_base=4700 + i)[0] for i, n in enumerate([25, 8, 19])]
    enc = eng.compress_tokens_batched(toks)
    ref = _decode_direct(eng, enc, [25], use_graph=graph)
    L = _lib.lib()
    _lib.call("kr_step_timing", phase, None)
    try:
        got = _decode_direct(eng, enc, [25], use_graph=graph)
        launch, span = (ctypes.c_double * 64)(), (ctypes.c_double * 64)()
        n = ctypes.c_int(0)
        _lib.call("kr_step_timing_read", launch, span, 64, ctypes.byref(n))
    finally:
        L.kr_step_timing(-1, None)
    for name, a, g in zip(("tokens", "count", "coder", "syms", "model state"), ref, got):
        assert torch.equal(a, g), f"{name} differs with the step timing on"
    assert n.value == 12
    for i in range(12):
        assert 0.0 < span[i] < 1000.0, (i, span[i])
        if graph:
            assert launch[i] == -1.0
        else:
            assert 0.0 < launch[i] < 1000.0, (i, launch[i])
