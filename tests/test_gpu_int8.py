"""w8a8 kernels against the numpy oracle: row quantisation bit for bit (both
layouts) and the int8 GEMM exactly (integer sums), every epilogue, on the
small-M (fragment-packed and row-major) and tiled paths."""
import numpy as np
import pytest
import torch

from krunch_amd import _lib
from oracle import quant

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _quant_gpu(x16: torch.Tensor, packed: int):
    M, K = x16.shape
    q = torch.zeros(_lib.lib().kr_quant_bytes(M, K, packed), dtype=torch.int8, device=DEV)
    s = torch.empty(M, dtype=torch.float32, device=DEV)
    _lib.call("kr_quantize_rows", x16.data_ptr(), K, M, K, q.data_ptr(), s.data_ptr(), packed,
              _lib.stream_ptr())
    return q, s


def _pack_w(wq: torch.Tensor):
    N, K = wq.shape
    out = torch.empty(_lib.lib().kr_fragment_bytes(N, K // 2), dtype=torch.uint8, device=DEV)
    _lib.call("kr_pack_fragments", wq.data_ptr(), K // 2, N, K // 2, out.data_ptr(),
              _lib.stream_ptr())
    return out


# K = 256 KI (KI in 1..4, 6, 8, 12) takes the register-resident row kernel,
# any other multiple of 64 the looping one
@pytest.mark.parametrize("M,K", [(1, 768), (37, 768), (300, 3072), (16, 64), (9, 256), (5, 512),
                                 (7, 1024), (3, 1536), (4, 2048), (6, 320)])
def test_quantize_rows_matches_oracle(M, K):
    g = torch.Generator().manual_seed(M + K)
    x = (torch.randn(M, K, generator=g) * torch.rand(M, 1, generator=g) * 8).half()
    if M > 2:
        x[2] = 0                                   # an all-zero row
    qo, so = quant.quantize_rows(x.float().numpy())
    q, s = _quant_gpu(x.to(DEV), 0)
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(q.cpu().numpy().reshape(M, K), qo)
    qp, sp = _quant_gpu(x.to(DEV), 1)
    assert np.array_equal(sp.cpu().numpy(), so)
    assert np.array_equal(qp.cpu().numpy(), quant.pack_i8(qo))


def _ref_epilogue(ep, y, res, gate):
    h = y.astype(np.float16).astype(np.float32)
    if ep == 0:
        return y
    if ep == 1:
        out = h
    elif ep == 2:
        out = 1.0 / (1.0 + np.exp(-h))
    elif ep == 3:
        out = np.maximum(h, 0) ** 2
    elif ep == 4:
        out = res.astype(np.float32) + h
    else:
        out = res.astype(np.float32) + (gate.astype(np.float32) * h).astype(np.float16).astype(np.float32)
    return out.astype(np.float16)


@pytest.mark.parametrize("M,K,N,packed", [(256, 768, 768, 1), (37, 3072, 768, 1), (5, 768, 3072, 1),
                                          (100, 768, 768, 0), (1000, 768, 2304, 0),
                                          (5000, 3072, 768, 0)])
def test_int8_matmul_exact(M, K, N, packed):
    g = torch.Generator().manual_seed(M * 7 + N)
    qa = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sa = torch.rand(M, generator=g) * 0.01 + 1e-4
    sw = torch.rand(N, generator=g) * 0.01 + 1e-4
    want = quant.matmul_i8(qa.numpy(), sa.numpy(), qw.numpy(), sw.numpy())
    if packed:
        xa = torch.from_numpy(quant.pack_i8(qa.numpy())).to(DEV)
        wb = _pack_w(qw.to(DEV))
    else:
        xa, wb = qa.to(DEV), qw.to(DEV)
    out = torch.empty(M, N, dtype=torch.float32, device=DEV)
    sa_d, sw_d = sa.to(DEV), sw.to(DEV)      # kept alive across the launch
    _lib.call("kr_det_matmul_i8", xa.data_ptr(), sa_d.data_ptr(), M, K, wb.data_ptr(),
              sw_d.data_ptr(), N, out.data_ptr(), N, 0, None, None, packed, _lib.stream_ptr())
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("packed", [1, 0])
@pytest.mark.parametrize("ep", [1, 2, 3, 4, 5])
def test_int8_epilogues(ep, packed):
    M, K, N = 64, 768, 768
    g = torch.Generator().manual_seed(ep)
    qa = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sa = torch.rand(M, generator=g) * 1e-3
    sw = torch.rand(N, generator=g) * 1e-3
    res = torch.randn(M, N, generator=g).half()
    gate = torch.rand(M, N, generator=g).half()
    y = quant.matmul_i8(qa.numpy(), sa.numpy(), qw.numpy(), sw.numpy())
    want = _ref_epilogue(ep, y, res.numpy(), gate.numpy())
    xa = torch.from_numpy(quant.pack_i8(qa.numpy())).to(DEV) if packed else qa.to(DEV)
    wb = _pack_w(qw.to(DEV)) if packed else qw.to(DEV)
    out = res.clone().to(DEV)
    sa_d, sw_d, gate_d = sa.to(DEV), sw.to(DEV), gate.to(DEV)   # kept alive across the launch
    _lib.call("kr_det_matmul_i8", xa.data_ptr(), sa_d.data_ptr(), M, K, wb.data_ptr(),
              sw_d.data_ptr(), N, out.data_ptr(), N, ep, out.data_ptr(), gate_d.data_ptr(),
              packed, _lib.stream_ptr())
    got = out.cpu().numpy()
    if ep == 2:   # sigmoid uses the device exp: within 1 fp16 ulp
        np.testing.assert_allclose(got.astype(np.float32), want.astype(np.float32), rtol=1e-3, atol=1e-3)
    else:
        assert np.array_equal(got, want)


@pytest.mark.parametrize("ep", [0, 1, 2, 3, 4, 5])
def test_int8_large_m_epilogues(ep):
    """The large-M int8 path for wide products (256 x 256 tiles, exact int32
    sums) with every epilogue, on ragged row and column tiles (M = 4200,
    N = 2100): the exact integer product, dequantised and passed through the
    epilogue, bit for bit (sigmoid within an fp16 ulp)."""
    M, K, N = 4200, 768, 2100
    g = torch.Generator().manual_seed(100 + ep)
    qa = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sa = torch.rand(M, generator=g) * 1e-3
    sw = torch.rand(N, generator=g) * 1e-3
    res = torch.randn(M, N, generator=g).half()
    gate = torch.rand(M, N, generator=g).half()
    y = quant.matmul_i8(qa.numpy(), sa.numpy(), qw.numpy(), sw.numpy())
    want = y if ep == 0 else _ref_epilogue(ep, y, res.numpy(), gate.numpy())
    xa, wb = qa.to(DEV), qw.to(DEV)
    out = torch.empty(M, N, dtype=torch.float32, device=DEV) if ep == 0 else res.clone().to(DEV)
    sa_d, sw_d, gate_d = sa.to(DEV), sw.to(DEV), gate.to(DEV)   # kept alive across the launch
    res_ptr = out.data_ptr() if ep in (4, 5) else None
    _lib.call("kr_det_matmul_i8", xa.data_ptr(), sa_d.data_ptr(), M, K, wb.data_ptr(),
              sw_d.data_ptr(), N, out.data_ptr(), N, ep, res_ptr, gate_d.data_ptr(), 0,
              _lib.stream_ptr())
    got = out.cpu().numpy()
    if ep == 2:
        np.testing.assert_allclose(got.astype(np.float32), want.astype(np.float32), rtol=1e-3, atol=1e-3)
    else:
        assert np.array_equal(got, want)


def _pack_f16(x16: torch.Tensor):
    """fp16 [M, K] -> fragment-packed (kr_pack_fragments), rows padded to 16."""
    M, K = x16.shape
    out = torch.empty(_lib.lib().kr_fragment_bytes(M, K) // 2, dtype=torch.float16, device=DEV)
    _lib.call("kr_pack_fragments", x16.data_ptr(), K, M, K, out.data_ptr(), _lib.stream_ptr())
    return out


def _activations(M, K, seed):
    """fp16 rows of mixed magnitude, one all-zero row, one row of exact
    halves (ties of x * inv), one with a single nonzero element."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g) * torch.rand(M, 1, generator=g).mul(20).add(1e-3)
    if M > 3:
        x[1] = 0
        x[2] = (torch.arange(K) % 9 - 4).float() * 0.5
        x[3] = 0
        x[3, K // 3] = -7.25
    return x.half()


@pytest.mark.parametrize("M,K,N", [(1, 768, 768), (37, 768, 768), (256, 768, 768),
                                   (256, 3072, 768), (300, 3072, 768), (512, 768, 3072),
                                   (20, 256, 64)])
def test_int8_matmul_quantised_on_load(M, K, N):
    """packed = 2: fp16 fragment-packed activations quantised per row inside
    the product (the decode path's output and value projections) == the
    oracle's quantize_rows followed by the exact int8 product, bit for bit."""
    x = _activations(M, K, M + K + N)
    g = torch.Generator().manual_seed(N)
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.rand(N, generator=g) * 0.01 + 1e-4
    qo, so = quant.quantize_rows(x.float().numpy())
    want = quant.matmul_i8(qo, so, qw.numpy(), sw.numpy())
    xf = _pack_f16(x.to(DEV))
    wb = _pack_w(qw.to(DEV))
    sw_d = sw.to(DEV)
    out = torch.empty(M, N, dtype=torch.float32, device=DEV)
    _lib.call("kr_det_matmul_i8", xf.data_ptr(), None, M, K, wb.data_ptr(), sw_d.data_ptr(), N,
              out.data_ptr(), N, 0, None, None, 2, _lib.stream_ptr())
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("ep", [4, 5])
def test_int8_quantised_on_load_epilogues(ep):
    """The residual and gated epilogues (output projection, value product) on
    the packed = 2 path: equal to packed = 1 on kr_quantize_rows' output."""
    M, K, N = 256, 3072 if ep == 5 else 768, 768
    x = _activations(M, K, ep).to(DEV)
    g = torch.Generator().manual_seed(11 * ep)
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(DEV)
    sw = (torch.rand(N, generator=g) * 1e-3).to(DEV)
    res = torch.randn(M, N, generator=g).half().to(DEV)
    gate = torch.rand(M, N, generator=g).half().to(DEV)
    wb = _pack_w(qw)
    q1, s1 = _quant_gpu(x, 1)
    out1 = res.clone()
    _lib.call("kr_det_matmul_i8", q1.data_ptr(), s1.data_ptr(), M, K, wb.data_ptr(), sw.data_ptr(),
              N, out1.data_ptr(), N, ep, out1.data_ptr(), gate.data_ptr(), 1, _lib.stream_ptr())
    xf = _pack_f16(x)
    out2 = res.clone()
    _lib.call("kr_det_matmul_i8", xf.data_ptr(), None, M, K, wb.data_ptr(), sw.data_ptr(), N,
              out2.data_ptr(), N, ep, out2.data_ptr(), gate.data_ptr(), 2, _lib.stream_ptr())
    assert torch.equal(out1, out2)
    qo, so = quant.quantize_rows(x.float().cpu().numpy())
    y = quant.matmul_i8(qo, so, qw.cpu().numpy(), sw.cpu().numpy())
    want = _ref_epilogue(ep, y, res.cpu().numpy(), gate.cpu().numpy())
    assert np.array_equal(out2.cpu().numpy(), want)


def test_quantised_on_load_rejects_row_major():
    """packed = 2 needs the fragment path: a large M is refused, not run."""
    M, K, N = 600, 768, 768
    x = torch.zeros(M, K, dtype=torch.float16, device=DEV)
    w = torch.zeros(N, K, dtype=torch.int8, device=DEV)
    sw = torch.ones(N, device=DEV)
    out = torch.empty(M, N, dtype=torch.float32, device=DEV)
    rc = _lib.lib().kr_det_matmul_i8(x.data_ptr(), None, M, K, w.data_ptr(), sw.data_ptr(), N,
                                     out.data_ptr(), N, 0, None, None, 2, _lib.stream_ptr())
    assert rc != 0
