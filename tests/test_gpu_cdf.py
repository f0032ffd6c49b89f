"""GPU probabilities/logits -> CDF: bit-exact with the oracle restatement of
krunch_ac/cdf.py (and with the reference's own golden CDFs), softmax bit-exact
with the oracle softmax, fused pairs and fused decode consistent with it."""
import hashlib

import numpy as np
import pytest
import torch

from krunch_amd import _lib
from krunch_amd import krunch_ac
from krunch_amd import krunch_ac_hip as ops
from oracle import cdf as ocdf
from oracle import range_coder as orc
from oracle import softmax as osm
from tests.golden import make_golden as mg

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_probs_to_cdf_golden(golden_dir):
    g = np.load(golden_dir + "/cdf_golden.npz", allow_pickle=False)
    for idx, (kind, N, V, seed) in enumerate(mg.CDF_CASES):
        cdf = krunch_ac.probs_to_cdf(mg.case_probs(kind, N, V, seed))
        sha = hashlib.sha256(np.ascontiguousarray(cdf.astype(np.uint32)).tobytes()).hexdigest()
        assert sha == str(g[f"cdf{idx}_sha"]), (kind, N, V)


@pytest.mark.parametrize("N,V,seed", [(3, 1, 0), (5, 7, 1), (4, 129, 2), (7, 8199, 3),
                                      (6, 50277, 4), (2, 65536, 5)])
def test_probs_to_cdf_matches_oracle(N, V, seed):
    rng = np.random.default_rng(seed)
    p = (rng.random((N, V)) ** 8).astype(np.float32)
    np.testing.assert_array_equal(krunch_ac.probs_to_cdf(p), ocdf.probs_to_cdf(p))


def _logits(N, V, seed, scale=3.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((N, V)) * scale).astype(np.float16)


@pytest.mark.parametrize("N,V,seed,scale", [(4, 50277, 0, 3.0), (8, 50277, 1, 12.0),
                                            (3, 1000, 2, 1.0), (2, 5, 3, 40.0)])
def test_softmax_probs_and_cdf_bit_exact(N, V, seed, scale):
    lg = _logits(N, V, seed, scale)
    d = torch.from_numpy(lg).to(DEV)
    q = ops.softmax_probs(d).cpu().numpy()
    np.testing.assert_array_equal(q, osm.softmax_probs(lg))
    ref = osm.logits_to_cdf(lg)
    np.testing.assert_array_equal(ops.softmax_cdf(d).cpu().numpy().view(np.uint32), ref)
    counts = ops.det_softmax_cdf(d, 1 << 24).cpu().numpy()
    assert (counts[:, 0] == 0).all()
    np.testing.assert_array_equal(counts[:, 1:], np.diff(ref.astype(np.int64), axis=1))


def test_row_result_independent_of_batch():
    lg = _logits(16, 50277, 9)
    d = torch.from_numpy(lg).to(DEV)
    full = ops.softmax_cdf(d).cpu().numpy()
    for r in (0, 7, 15):
        one = ops.softmax_cdf(d[r:r + 1].contiguous()).cpu().numpy()
        np.testing.assert_array_equal(one[0], full[r])


def test_special_logits():
    V = 50277
    lg = np.zeros((3, V), dtype=np.float16)
    lg[1, 123] = 30.0                       # near one-hot
    lg[2, :] = -60000.0
    lg[2, 9] = lg[2, 40000] = 5.0          # two equal maxima: first wins
    d = torch.from_numpy(lg).to(DEV)
    got = ops.softmax_cdf(d).cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got, osm.logits_to_cdf(lg))
    w = np.diff(got.astype(np.int64), axis=1)
    assert w[2, 9] > w[2, 40000]


def test_pairs_match_oracle_intervals():
    N, V = 64, 50277
    lg = _logits(N, V, 11)
    sym = np.random.default_rng(3).integers(0, V, N).astype(np.int32)
    sym[:4] = [0, V - 1, int(np.argmax(lg[2])), int(np.argmax(lg[3]))]
    d = torch.from_numpy(lg).to(DEV)
    s = torch.from_numpy(sym).to(DEV)
    pairs = torch.empty((N, 2), dtype=torch.int32, device=DEV)
    _lib.call("kr_softmax_cdf_pairs", d.data_ptr(), N, V, V, s.data_ptr(), pairs.data_ptr(), 24,
              _lib.stream_ptr())
    lo, hi = osm.sym_intervals(osm.logits_to_cdf(lg), sym)
    got = pairs.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got[:, 0], lo)
    np.testing.assert_array_equal(got[:, 1], hi)


@pytest.mark.parametrize("N,V", [(600, 50277), (700, 1000), (300, 5)])
def test_pairs_persistent_rows_padded_stride(N, V):
    """Many rows, 8-aligned stride: the persistent path that copies the next
    row in while computing the current one. The row padding holds values
    (NaN, +-60000) that must never be read as elements."""
    ld = (V + 7) // 8 * 8 + 8
    lg = _logits(N, V, 13, 4.0)
    full = np.empty((N, ld), dtype=np.float16)
    full[:, :V] = lg
    full[:, V:] = np.float16(60000.0)
    full[::3, V:] = np.float16(np.nan)
    full[1::3, V:] = np.float16(-60000.0)
    sym = np.random.default_rng(4).integers(0, V, N).astype(np.int32)
    d = torch.from_numpy(full).to(DEV)
    s = torch.from_numpy(sym).to(DEV)
    pairs = torch.empty((N, 2), dtype=torch.int32, device=DEV)
    _lib.call("kr_softmax_cdf_pairs", d.data_ptr(), N, V, ld, s.data_ptr(), pairs.data_ptr(), 16,
              _lib.stream_ptr())
    lo, hi = osm.sym_intervals(osm.logits_to_cdf(lg, 16), sym)
    got = pairs.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got[:, 0], lo)
    np.testing.assert_array_equal(got[:, 1], hi)


def test_fused_decode_matches_oracle():
    """B streams; per step each stream has its own logits row. The oracle
    encodes with the oracle CDFs; the fused kernel decodes from the logits."""
    B, N, V = 4, 40, 50277
    rng = np.random.default_rng(5)
    lg = (rng.standard_normal((N, B, V)) * 4).astype(np.float16)
    syms = rng.integers(0, V, (B, N)).astype(np.int32)
    syms[:, ::3] = np.argmax(lg[::3], axis=2).T[:, :syms[:, ::3].shape[1]]
    streams = []
    for b in range(B):
        streams.append(orc.encode(osm.logits_to_cdf(lg[:, b]), syms[b]))
    offs = np.cumsum([0] + [len(s) for s in streams])
    buf = torch.from_numpy(np.frombuffer(b"".join(streams), np.uint8).copy()).to(DEV)
    base = torch.from_numpy(offs[:-1].astype(np.int32)).to(DEV)
    lim = torch.tensor([len(s) for s in streams], dtype=torch.int32, device=DEV)
    st = torch.zeros(4 * B, dtype=torch.uint32, device=DEV)
    _lib.call("kr_decode_init_batched", buf.data_ptr(), buf.numel(), base.data_ptr(),
              lim.data_ptr(), st.data_ptr(), B, _lib.stream_ptr())
    out = torch.empty(B, dtype=torch.int32, device=DEV)
    toks = torch.zeros((B, N), dtype=torch.int32, device=DEV)
    cnt = torch.zeros(B, dtype=torch.int32, device=DEV)
    ntok = torch.tensor([N, N, N - 5, N], dtype=torch.int32, device=DEV)
    lgd = torch.from_numpy(lg).to(DEV)
    for t in range(N):
        _lib.call("kr_softmax_cdf_decode", lgd[t].data_ptr(), B, V, V, buf.data_ptr(), buf.numel(),
                  base.data_ptr(), lim.data_ptr(), st.data_ptr(), out.data_ptr(), toks.data_ptr(),
                  N, cnt.data_ptr(), ntok.data_ptr(), 24, _lib.stream_ptr())
    got = toks.cpu().numpy()
    for b in range(B):
        n = int(ntok[b])
        np.testing.assert_array_equal(got[b, :n], syms[b, :n])
    assert cnt.cpu().tolist() == [N, N, N - 5, N]
