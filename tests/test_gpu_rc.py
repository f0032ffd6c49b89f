"""GPU range coder: bitstreams byte-identical to the oracle coder on the same
CDFs (the reference's tests/test_ac_kernel_gpu.py:64-215 cases), decode round
trips, batched lockstep decode, and the fused-compress pair encoder."""
import numpy as np
import pytest
import torch

from krunch_amd import _lib
from krunch_amd import krunch_ac_hip as ops
from oracle import cdf as ocdf
from oracle import range_coder as orc
from tests.golden import make_golden as mg

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(N, V, seed):
    p = mg.rand_probs(N, V, seed)
    return ocdf.probs_to_cdf(p), mg.sample_symbols(p, seed)


def _fresh_state(B=1):
    st = torch.zeros((B, 4), dtype=torch.int64)
    st[:, 1] = 0xFFFFFFFF
    return st.to(torch.uint32).to(DEV).reshape(-1).contiguous()


def _gpu_encode(cdf, sym, chunks=1):
    out = torch.zeros(8 * len(sym) + 64, dtype=torch.uint8, device=DEV)
    st = _fresh_state()
    for part in np.array_split(np.arange(len(sym)), chunks):
        c = torch.from_numpy(cdf[part].view(np.int32)).to(DEV)
        s = torch.from_numpy(sym[part].astype(np.int32)).to(DEV)
        ops.encode_step(c, s, out, st)
    ops.encode_finalize(out, st)
    nbits = int(st.cpu().to(torch.int64)[3])
    return bytes(out[:(nbits + 7) // 8].cpu().numpy())


CASES = [(1, 4, 0), (8, 32, 1), (256, 256, 2), (1024, 1024, 3), (256, 50277, 4)]


@pytest.mark.parametrize("N,V,seed", CASES)
def test_encode_byte_identical_to_oracle(N, V, seed):
    cdf, sym = _case(N, V, seed)
    assert _gpu_encode(cdf, sym) == orc.encode(cdf, sym)


def test_multi_call_state_persists():
    cdf, sym = _case(300, 256, 7)
    assert _gpu_encode(cdf, sym, chunks=3) == orc.encode(cdf, sym)


def test_reference_golden_bitstreams(golden_dir):
    g = np.load(golden_dir + "/rc_golden.npz", allow_pickle=False)
    for idx, (N, V, seed) in enumerate(mg.RC_CASES):
        cdf, sym = _case(N, V, seed)
        assert _gpu_encode(cdf, sym) == g[f"bits{idx}"].tobytes()


@pytest.mark.parametrize("N,V,seed", CASES)
def test_decode_roundtrip(N, V, seed):
    cdf, sym = _case(N, V, seed)
    bits = orc.encode(cdf, sym)
    buf = torch.from_numpy(np.frombuffer(bits, np.uint8).copy()).to(DEV)
    st = torch.zeros(4, dtype=torch.uint32, device=DEV)
    ops.decode_init(buf, st)
    c = torch.from_numpy(cdf.view(np.int32)).to(DEV)
    out = torch.empty(N, dtype=torch.int32, device=DEV)
    for i in range(N):
        ops.decode_step(c[i], buf, st, out[i:i + 1])
    np.testing.assert_array_equal(out.cpu().numpy(), sym)


@pytest.mark.parametrize("B,N,V,seed", [(2, 16, 32, 7), (4, 64, 256, 8), (8, 256, 1024, 9),
                                        (3, 300, 50277, 10)])
def test_batched_lockstep_decode(B, N, V, seed):
    cdfs, syms, streams = [], [], []
    for b in range(B):
        c, s = _case(N, V, seed + b)
        cdfs.append(c)
        syms.append(s)
        streams.append(orc.encode(c, s))
    offs = np.cumsum([0] + [len(s) for s in streams])
    buf = torch.from_numpy(np.frombuffer(b"".join(streams), np.uint8).copy()).to(DEV)
    base = torch.from_numpy(offs[:-1].astype(np.int32)).to(DEV)
    lim = torch.tensor([len(s) for s in streams], dtype=torch.int32, device=DEV)
    st = torch.zeros(4 * B, dtype=torch.uint32, device=DEV)
    ops.decode_init_batched(buf, base, st, lim)
    allc = torch.from_numpy(np.stack(cdfs, axis=1).view(np.int32)).to(DEV)   # [N, B, V+1]
    out = torch.empty((N, B), dtype=torch.int32, device=DEV)
    for t in range(N):
        ops.decode_step_batched(allc[t].contiguous(), buf, base, st, out[t], lim)
    np.testing.assert_array_equal(out.cpu().numpy().T, np.stack(syms))


def test_encode_batched_and_pairs_match_oracle():
    B, N, V = 5, 200, 777
    cdfs, syms = zip(*[_case(N, V, 40 + b) for b in range(B)])
    refs = [orc.encode(c, s) for c, s in zip(cdfs, syms)]
    cap = 4 * N + 64
    # one symbol per stream per call
    out = torch.zeros(B * cap, dtype=torch.uint8, device=DEV)
    base = torch.arange(B, dtype=torch.int32, device=DEV) * cap
    st = _fresh_state(B)
    allc = torch.from_numpy(np.stack(cdfs, axis=1).view(np.int32)).to(DEV)
    alls = torch.from_numpy(np.stack(syms, axis=1).astype(np.int32)).to(DEV)
    for t in range(N):
        ops.encode_step_batched(allc[t].contiguous(), alls[t].contiguous(), out, base, st)
    ops.encode_finalize_batched(out, base, st)
    bits = st.view(B, 4)[:, 3].cpu().to(torch.int64).numpy()
    host = out.cpu().numpy()
    for b in range(B):
        assert host[b * cap:b * cap + (bits[b] + 7) // 8].tobytes() == refs[b]
    # all T symbols per stream from intervals, ragged valid counts
    n_valid = np.array([N, 3, 0, N - 1, 57], dtype=np.int32)
    pairs = np.zeros((B, N, 2), dtype=np.uint32)
    for b in range(B):
        lo, hi = ocdf_intervals(cdfs[b], syms[b])
        pairs[b, :, 0], pairs[b, :, 1] = lo, hi
    out2 = torch.zeros(B * cap, dtype=torch.uint8, device=DEV)
    st2 = _fresh_state(B)
    err = torch.zeros(1, dtype=torch.uint32, device=DEV)
    pd = torch.from_numpy(pairs.view(np.int32)).to(DEV)
    nv = torch.from_numpy(n_valid).to(DEV)
    _lib.call("kr_encode_pairs_batched", pd.data_ptr(), N, N, nv.data_ptr(), out2.data_ptr(),
              out2.numel(), base.data_ptr(), st2.data_ptr(), B, 24, err.data_ptr(), _lib.stream_ptr())
    _lib.call("kr_encode_finalize_batched", out2.data_ptr(), out2.numel(), base.data_ptr(),
              st2.data_ptr(), B, err.data_ptr(), _lib.stream_ptr())
    assert int(err.item()) == 0
    bits = st2.view(B, 4)[:, 3].cpu().to(torch.int64).numpy()
    host = out2.cpu().numpy()
    for b in range(B):
        n = int(n_valid[b])
        ref = orc.encode(cdfs[b][:n], syms[b][:n]) if n else orc.encode_intervals([], [], 1 << 24)
        assert host[b * cap:b * cap + (bits[b] + 7) // 8].tobytes() == ref, b


def ocdf_intervals(cdf, sym):
    r = np.arange(len(sym))
    return cdf[r, sym], cdf[r, sym + 1]


def test_output_overflow_is_reported_not_written_past():
    cdf, sym = _case(400, 50277, 3)
    out = torch.zeros(64 + 16, dtype=torch.uint8, device=DEV)
    guard = out[64:]
    st = _fresh_state()
    err = torch.zeros(1, dtype=torch.uint32, device=DEV)
    c = torch.from_numpy(cdf.view(np.int32)).to(DEV)
    s = torch.from_numpy(sym).to(DEV)
    _lib.call("kr_encode_step", c.data_ptr(), c.shape[1], s.data_ptr(), 400, out.data_ptr(), 64,
              st.data_ptr(), 24, err.data_ptr(), _lib.stream_ptr())
    assert int(err.item()) == 1
    assert int(guard.sum().item()) == 0


def _ref_probs(N, V, seed):
    """The reference coder tests' distribution recipe
    (tests/test_ac_reference.py:14-18): uniform randoms, row-normalised."""
    rng = np.random.default_rng(seed)
    p = rng.random((N, V)).astype(np.float32)
    return p / p.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("N,V,seed", [(1, 4, 10), (16, 64, 11), (256, 256, 12),
                                      (1024, 1024, 13), (4096, 50277, 14)])
def test_reference_shapes_roundtrip(N, V, seed):
    """tests/test_ac_reference.py:63-75 on the GPU coder: symbols sampled
    from the rows; CDF, bitstream and decode equal to the oracle's."""
    from krunch_amd import krunch_ac
    p = _ref_probs(N, V, seed)
    rng = np.random.default_rng(seed + 100)
    u = rng.random((N, 1)).astype(np.float32)
    sym = (u < np.cumsum(p, axis=1)).argmax(axis=1).astype(np.int32)
    cdf = krunch_ac.probs_to_cdf(p)
    np.testing.assert_array_equal(cdf, ocdf.probs_to_cdf(p))
    bits = krunch_ac.encode(cdf, sym)
    assert bits == orc.encode(cdf, sym)
    np.testing.assert_array_equal(krunch_ac.decode(bits, cdf), sym)


def test_all_same_symbol_and_rare_symbol():
    """tests/test_ac_reference.py:78-98: a stream of one symbol, and a
    near-minimal-probability symbol (p = 1e-6) at every step."""
    from krunch_amd import krunch_ac
    p = _ref_probs(100, 50, 20)
    sym = np.zeros(100, dtype=np.int32)
    cdf = krunch_ac.probs_to_cdf(p)
    bits = krunch_ac.encode(cdf, sym)
    assert bits == orc.encode(cdf, sym)
    np.testing.assert_array_equal(krunch_ac.decode(bits, cdf), sym)
    V, N = 200, 50
    p = np.full((N, V), 1e-6, dtype=np.float32)
    p[:, 0] = 1.0 - 1e-6 * (V - 1)
    p /= p.sum(axis=1, keepdims=True)
    sym = np.full(N, 199, dtype=np.int32)
    cdf = krunch_ac.probs_to_cdf(p)
    np.testing.assert_array_equal(cdf, ocdf.probs_to_cdf(p))
    # width floor(1e-6 * (2^24 - 200)) + 1 = 17 of 2^24
    assert (np.diff(cdf[:, 199:201].astype(np.int64), axis=1) == 17).all()
    bits = krunch_ac.encode(cdf, sym)
    assert bits == orc.encode(cdf, sym)
    np.testing.assert_array_equal(krunch_ac.decode(bits, cdf), sym)


def test_compression_makes_progress():
    """tests/test_ac_reference.py:111-121: a peaky distribution always
    hitting its likely symbol codes far below the uniform 10 bits/symbol."""
    from krunch_amd import krunch_ac
    N, V = 2048, 1024
    p = np.full((N, V), 1.0, dtype=np.float32)
    p[:, 0] = 1000.0
    p /= p.sum(axis=1, keepdims=True)
    sym = np.zeros(N, dtype=np.int32)
    cdf = krunch_ac.probs_to_cdf(p)
    bits = krunch_ac.encode(cdf, sym)
    assert len(bits) < N // 4, len(bits)
    assert bits == orc.encode(cdf, sym)
    np.testing.assert_array_equal(krunch_ac.decode(bits, cdf), sym)
