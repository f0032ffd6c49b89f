"""Forward oracle: the WKV recurrence against its closed form, T=1 from the
initial state, and the packed == stepped / windowed == single invariants."""
import numpy as np
import torch

from oracle import rwkv4
from tests.golden import make_golden as mg


def _direct_wkv(k, v, w, u):
    """y_t = (sum_{i<t} e^{(t-1-i)w + k_i} v_i + e^{u+k_t} v_t) / (same without v)."""
    B, T, C = k.shape
    k, v, w, u = (a.double() for a in (k, v, w, u))
    y = torch.empty(B, T, C, dtype=torch.float64)
    for t in range(T):
        i = torch.arange(t, dtype=torch.float64)
        wt = torch.exp((t - 1 - i)[None, :, None] * w + k[:, :t])
        cur = torch.exp(u + k[:, t])
        y[:, t] = ((wt * v[:, :t]).sum(1) + cur * v[:, t]) / (wt.sum(1) + cur)
    return y


def test_wkv_closed_form():
    g = torch.Generator().manual_seed(0)
    B, T, C = 3, 40, 16
    k = torch.randn(B, T, C, generator=g) * 2
    v = torch.randn(B, T, C, generator=g)
    w = -torch.exp(torch.linspace(-5, 3, C))
    u = torch.full((C,), float(np.log(0.3)))
    st = rwkv4.new_state(1, B, C)[0]
    y = rwkv4.wkv(k, v, w, u, st)
    np.testing.assert_allclose(y.numpy(), _direct_wkv(k, v, w, u).numpy(), rtol=2e-5, atol=2e-6)


def test_wkv_first_step_is_v():
    g = torch.Generator().manual_seed(1)
    k, v = torch.randn(2, 1, 8, generator=g), torch.randn(2, 1, 8, generator=g)
    st = rwkv4.new_state(1, 2, 8)[0]
    y = rwkv4.wkv(k, v, -torch.ones(8), torch.zeros(8), st)
    torch.testing.assert_close(y, v, rtol=0, atol=1e-7)


def test_packed_equals_stepped_rowwise_and_windowed():
    t = mg.TINY
    w = mg.tiny_weights(**t)
    ids = torch.as_tensor(mg.tiny_ids(**t))
    T = ids.shape[1]
    st_p = rwkv4.new_state(t["n_layer"], t["B"], t["C"])
    packed = rwkv4.forward(w, ids, st_p, rowwise=True)
    st_s = rwkv4.new_state(t["n_layer"], t["B"], t["C"])
    stepped = torch.cat([rwkv4.forward(w, ids[:, i:i + 1], st_s, rowwise=True)
                         for i in range(T)], dim=1)
    assert torch.equal(packed, stepped)
    st_w = rwkv4.new_state(t["n_layer"], t["B"], t["C"])
    windowed = torch.cat([rwkv4.forward(w, ids[:, :3], st_w, rowwise=True),
                          rwkv4.forward(w, ids[:, 3:], st_w, rowwise=True)], dim=1)
    assert torch.equal(packed, windowed)


def test_fp16_rounding_points():
    """forward(fp16=True) rounds activations where the production layer
    stores fp16: its residual stream and logits are fp16-representable, it
    stays within the fp16 tolerance of the fp32 forward, and the int8 codec
    in that mode quantises rows of fp16 values."""
    from krunch_amd import synthetic
    w = synthetic.make_weights(n_layer=2, C=256, F=512, V=1000)
    ids = torch.as_tensor(synthetic.model_inputs(synthetic.zipf_tokens(2, 12, V=1000)))
    st = rwkv4.new_state(2, 2, 256)
    f16 = rwkv4.forward(w, ids, st, fp16=True)
    assert torch.equal(f16, f16.half().float())
    for s in st:
        assert torch.equal(s["att_xx"], s["att_xx"].half().float())
    f32 = rwkv4.forward(w, ids, rwkv4.new_state(2, 2, 256))
    assert (f16 - f32).abs().max() < 1e-2
    q16 = rwkv4.forward(w, ids, rwkv4.new_state(2, 2, 256), w8a8=True, fp16=True)
    assert torch.equal(q16, q16.half().float()) and (q16 - f32).abs().max() < 0.2


def test_rowgemm_order_and_row_invariance():
    """oracle/rowgemm.c: each output is the float32 sum over k in order
    (checked against that sum spelled out in numpy float32, bit for bit),
    close to the float64 product, and a row's bits do not depend on which
    rows share the call (ragged M, N not a multiple of the column block)."""
    from oracle import crc
    rng = np.random.default_rng(3)
    M, K, N = 37, 96, 1000
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((K, N)) * 0.05).astype(np.float32)
    y = crc.gemm_rows(x, W)
    acc = np.zeros((M, N), np.float32)
    for k in range(K):
        acc = (acc + (x[:, k:k + 1] * W[k:k + 1, :]).astype(np.float32)).astype(np.float32)
    np.testing.assert_array_equal(y, acc)
    np.testing.assert_allclose(y, x.astype(np.float64) @ W.astype(np.float64), rtol=1e-5, atol=1e-5)
    for i in (0, 8, 36):
        np.testing.assert_array_equal(crc.gemm_rows(x[i:i + 1], W), y[i:i + 1])
    np.testing.assert_array_equal(crc.gemm_rows(x[5:30], W), y[5:30])


def test_layer_norm_gpu_order_against_torch_and_closed_forms():
    """oracle.rwkv4.layer_norm (the GPU row kernel's summation order) against
    torch's layer_norm (float32, its own order) to float32 rounding, and two
    rows whose result is fixed exactly: a constant row (mean exact, variance
    0, so y = b exactly) and a row of +a / -a in equal numbers (mean 0
    exactly, variance a^2 exactly for a power of two a, so y = +-(a * rstd)
    * w + b with rstd = 1/sqrt(a^2 + 1e-5))."""
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(5)
    for C in (256, 768, 1024):
        x = torch.randn(9, C, generator=g) * torch.rand(9, 1, generator=g).mul(8).add(0.01)
        x[0] = 3.25
        a = 0.5
        x[1] = a * (1 - 2 * (torch.arange(C) % 2)).float()
        w = torch.randn(C, generator=g).half().float()
        b = torch.randn(C, generator=g).half().float()
        y = rwkv4.layer_norm(x, w, b)
        ref = F.layer_norm(x, (C,), w, b, rwkv4.LN_EPS)
        np.testing.assert_allclose(y.numpy(), ref.numpy(), rtol=2e-5, atol=2e-5)
        assert torch.equal(y[0], b)
        f = np.float32
        rstd = f(1.0) / np.sqrt(f(a * a) + f(rwkv4.LN_EPS))
        sign = np.where(np.arange(C) % 2 == 0, f(1), f(-1))
        want = (((sign * f(a)) * rstd).astype(f) * w.numpy()).astype(f) + b.numpy()
        np.testing.assert_array_equal(y[1].numpy(), want.astype(f))


def test_deterministic_sigmoid_and_wkv():
    """The w8a8 codec's kexp-based sigmoid and WKV (fp16 mode of the int8
    oracle) against torch's sigmoid and the WKV closed form, to float32
    rounding; the sigmoid's two branches meet at 0 (0.5 exactly) and are
    symmetric: s(-x) = 1 - s(x) within one rounding."""
    x = torch.linspace(-30, 30, 4001)
    s = rwkv4._sigmoid(x, True)
    np.testing.assert_allclose(s.numpy(), torch.sigmoid(x).numpy(), rtol=3e-7, atol=1e-7)
    assert float(rwkv4._sigmoid(torch.zeros(1), True)[0]) == 0.5
    np.testing.assert_allclose((s + rwkv4._sigmoid(-x, True)).numpy(), 1.0, atol=1.2e-7)
    g = torch.Generator().manual_seed(2)
    B, T, C = 2, 30, 16
    k = torch.randn(B, T, C, generator=g) * 2
    v = torch.randn(B, T, C, generator=g)
    w = -torch.exp(torch.linspace(-5, 3, C))
    u = torch.full((C,), float(np.log(0.3)))
    y = rwkv4.wkv(k, v, w, u, rwkv4.new_state(1, B, C)[0], det=True)
    np.testing.assert_allclose(y.numpy(), _direct_wkv(k, v, w, u).numpy(), rtol=2e-5, atol=2e-6)
