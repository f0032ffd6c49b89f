"""MFMA GEMM: against a float32 torch reference of the same op, every
epilogue, and bit-identity of a row's result across M (different tile
shapes), which the packed/stepped round trip relies on."""
import numpy as np
import pytest
import torch

from krunch_amd import _lib
from krunch_amd import krunch_ac_hip as ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _mk(M, K, N, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = (torch.randn(M, K, generator=g)).to(torch.float16).to(DEV)
    W = (torch.randn(K, N, generator=g) * 0.02).to(torch.float16).to(DEV)
    return x, W


@pytest.mark.parametrize("M,K,N", [(1, 768, 768), (17, 768, 3072), (128, 3072, 768),
                                   (1024, 768, 768), (5000, 768, 768), (300, 768, 50277)])
def test_matmul_vs_fp32_reference(M, K, N):
    x, W = _mk(M, K, N, M + N)
    ref = x.float() @ W.float()
    y32 = ops.det_matmul(x, W, torch.float32)
    torch.testing.assert_close(y32, ref, rtol=1e-3, atol=1e-3)
    y16 = ops.det_matmul(x, W)
    torch.testing.assert_close(y16.float(), ref, rtol=2e-3, atol=2e-3)


def test_rows_bit_identical_across_M():
    K, N = 768, 3072
    x, W = _mk(8192, K, N, 1)
    full = ops.det_matmul(x, W, torch.float32)          # 128x128 tiles
    mid = ops.det_matmul(x[:2048].contiguous(), W, torch.float32)   # 64x64 tiles
    small = ops.det_matmul(x[:200].contiguous(), W, torch.float32)  # 32x32 tiles
    one = ops.det_matmul(x[37:38].contiguous(), W, torch.float32)
    assert torch.equal(full[:2048], mid)
    assert torch.equal(full[:200], small)
    assert torch.equal(full[37:38], one)


def _run(ep, x, Wt, N, res=None, gate=None):
    M, K = x.shape
    out = torch.empty((M, N), dtype=torch.float32 if ep == 0 else torch.float16, device=DEV)
    if res is not None:
        out.copy_(res)
    _lib.call("kr_det_matmul", x.data_ptr(), M, K, Wt.data_ptr(), K, N, out.data_ptr(), N, ep,
              _lib.ptr(out if res is not None else None), _lib.ptr(gate), _lib.stream_ptr())
    return out


@pytest.mark.parametrize("M,K,N", [(333, 768, 768), (4096, 768, 768), (5000, 768, 3072),
                                   (4096, 3072, 768), (8192 + 77, 768, 768)])
def test_epilogues(M, K, N):
    """Epilogues 2-5 (sigmoid, relu^2, residual, gated residual) on the tile
    kernel (M = 333) and on the persistent 256x128 kernel every compress
    window runs (M >= 4096, ragged last row tile at 8269), against torch
    fp32 on the same accumulator."""
    x, W = _mk(M, K, N, 5 + M)
    Wt = W.t().contiguous()
    acc = ops.det_matmul(x, W, torch.float32)
    torch.testing.assert_close(acc, x.float() @ W.float(), rtol=1e-3, atol=1e-3)
    h = acc.half().float()
    res = torch.randn(M, N, device=DEV).half()
    gate = torch.rand(M, N, device=DEV).half()
    torch.testing.assert_close(_run(2, x, Wt, N).float(), torch.sigmoid(h).half().float(),
                               rtol=0, atol=1e-3)
    torch.testing.assert_close(_run(3, x, Wt, N).float(), (torch.relu(h) ** 2).half().float(),
                               rtol=0, atol=1e-3)
    torch.testing.assert_close(_run(4, x, Wt, N, res=res).float(), (res.float() + h).half().float(),
                               rtol=0, atol=2e-3)
    want = (res.float() + (gate.float() * h).half().float()).half().float()
    torch.testing.assert_close(_run(5, x, Wt, N, res=res, gate=gate).float(), want, rtol=0, atol=2e-3)


@pytest.mark.parametrize("M,K,N,ep", [(256, 3072, 768, 5), (37, 768, 3072, 3), (5, 768, 768, 0),
                                      (256, 768, 768, 4), (64, 768, 2304, 2)])
def test_packed_operands_match_row_major(M, K, N, ep):
    """kr_det_matmul_packed on fragment-packed x and W gives kr_det_matmul's
    bits; with out_packed the fp16 result is the packed layout of the same."""
    from krunch_amd import _lib
    x, W = _mk(M, K, N, 11)
    Wt = W.t().contiguous()
    g = torch.Generator(device="cpu").manual_seed(12)
    res = torch.randn((M, N), generator=g).half().cuda()
    gate = torch.rand((M, N), generator=g).half().cuda()
    want = _run(ep, x, Wt, N, res.clone(), gate)

    def pack(X):
        R, KK = X.shape
        buf = torch.empty(_lib.lib().kr_fragment_bytes(R, KK) // 2, dtype=torch.float16,
                          device="cuda")
        _lib.call("kr_pack_fragments", X.data_ptr(), KK, R, KK, buf.data_ptr(), _lib.stream_ptr())
        return buf

    xf, Wf = pack(x), pack(Wt)
    out = torch.empty_like(want)
    r2 = res.clone()
    if ep in (4, 5):
        out = r2
    _lib.call("kr_det_matmul_packed", xf.data_ptr(), M, K, Wf.data_ptr(), N, out.data_ptr(), N, ep,
              r2.data_ptr(), gate.data_ptr(), 0, _lib.stream_ptr())
    assert torch.equal(out, want)
    if ep in (1, 2, 3):
        of = torch.zeros(_lib.lib().kr_fragment_bytes(M, N) // 2, dtype=torch.float16,
                         device="cuda")
        _lib.call("kr_det_matmul_packed", xf.data_ptr(), M, K, Wf.data_ptr(), N, of.data_ptr(), N,
                  ep, None, None, 1, _lib.stream_ptr())
        assert torch.equal(of, pack(want))


def test_packed_multi_equals_separate_launches():
    """kr_det_matmul_packed_multi (the stepped channel-mix R and K products
    in one launch: sigmoid into a row-major gate, relu^2 into a packed
    operand) gives the bits of two kr_det_matmul_packed calls."""
    from krunch_amd import _lib
    M, K = 256, 768
    g = torch.Generator(device="cpu").manual_seed(21)
    x = torch.randn((M, K), generator=g).half().cuda()
    WR = (torch.randn((768, K), generator=g) * 0.03).half().cuda()
    WK = (torch.randn((3072, K), generator=g) * 0.03).half().cuda()

    def pack(X):
        R, KK = X.shape
        buf = torch.empty(_lib.lib().kr_fragment_bytes(R, KK) // 2, dtype=torch.float16,
                          device="cuda")
        _lib.call("kr_pack_fragments", X.data_ptr(), KK, R, KK, buf.data_ptr(), _lib.stream_ptr())
        return buf

    xf, WRf, WKf = pack(x), pack(WR), pack(WK)
    r1 = torch.empty((M, 768), dtype=torch.float16, device="cuda")
    k1 = torch.zeros(_lib.lib().kr_fragment_bytes(M, 3072) // 2, dtype=torch.float16, device="cuda")
    _lib.call("kr_det_matmul_packed", xf.data_ptr(), M, K, WRf.data_ptr(), 768, r1.data_ptr(), 768,
              2, None, None, 0, _lib.stream_ptr())
    _lib.call("kr_det_matmul_packed", xf.data_ptr(), M, K, WKf.data_ptr(), 3072, k1.data_ptr(),
              3072, 3, None, None, 1, _lib.stream_ptr())
    r2 = torch.empty_like(r1)
    k2 = torch.zeros_like(k1)
    jobs = (_lib.KrPackedJob * 2)()
    jobs[0] = _lib.KrPackedJob(xf.data_ptr(), WRf.data_ptr(), 768, r2.data_ptr(), 768, 2, None,
                               None, 0)
    jobs[1] = _lib.KrPackedJob(xf.data_ptr(), WKf.data_ptr(), 3072, k2.data_ptr(), 3072, 3, None,
                               None, 1)
    _lib.call("kr_det_matmul_packed_multi", jobs, 2, M, K, _lib.stream_ptr())
    assert torch.equal(r1, r2) and torch.equal(k1, k2)
