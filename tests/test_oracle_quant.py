"""The w8a8 oracle pinned by hand-computed rows and exact integer checks."""
import numpy as np

from oracle import quant


def test_hand_rows():
    x = np.array([[127.0, -127.0, 0.0, 63.5, 0.5, 1.5, -2.5, 3.0],
                  [0.0] * 8,
                  [2.0, 1.0, -1.0, 0.0, 0.0, 0.0, 0.0, 0.0]], np.float32)
    q, s = quant.quantize_rows(x)
    # row 0: s = 1, ties go to even
    assert s[0] == np.float32(1.0)
    assert q[0].tolist() == [127, -127, 0, 64, 0, 2, -2, 3]
    # zero row: scale 1, all zeros
    assert s[1] == np.float32(1.0) and not q[1].any()
    # row 2: s = 2/127; 1/s = 63.5 -> 64 (even), -63.5 -> -64
    assert s[2] == np.float32(2.0) / np.float32(127.0)
    assert q[2].tolist()[:3] == [127, 64, -64]


def test_exact_product_rounding():
    """q rounds the exact product x * inv: for amax = 3, inv = RN(127/3) =
    42.33333206..., and 1.5 * inv = 63.4999981 -> 63. Rounding the product to
    float32 first would give 63.5 and then 64 (ties to even)."""
    x = np.array([[3.0, 1.5, -1.5, 0.0]], np.float32)
    q, s = quant.quantize_rows(x)
    inv = np.float32(127.0) / np.float32(3.0)
    assert float(inv) == 42.333332061767578
    assert np.float32(np.float32(1.5) * inv) == np.float32(63.5)
    assert q[0].tolist() == [127, 63, -63, 0]
    assert s[0] == np.float32(3.0) / np.float32(127.0)


def test_random_rows_against_rationals():
    """Every q is the nearest integer (ties to even) to x * inv computed in
    exact rational arithmetic, with inv and s the float32 quotients."""
    from fractions import Fraction
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((12, 64)) * rng.uniform(0.001, 50, (12, 1))).astype(np.float16)
    x[3] = 0
    x[5, :8] = np.float16(0.5) * (np.arange(8) - 4)            # exact halves
    q, s = quant.quantize_rows(x)
    for r in range(x.shape[0]):
        amax = max(abs(float(v)) for v in x[r])
        inv = float(np.float32(127.0) / np.float32(amax)) if amax > 0 else 1.0
        for k in range(x.shape[1]):
            p = Fraction(float(x[r, k])) * Fraction(inv)
            fl = p.numerator // p.denominator
            rem = p - fl
            want = fl + (1 if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2) else 0)
            assert q[r, k] == want, (r, k)
        assert s[r] == (np.float32(amax) / np.float32(127.0) if amax > 0 else np.float32(1.0))


def test_error_bound_and_range():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((50, 768)) * rng.uniform(0.01, 10, (50, 1))).astype(np.float16)
    q, s = quant.quantize_rows(x)
    assert np.abs(q).max() <= 127
    assert (np.abs(q).max(axis=1) == 127).all()          # every row uses the full range
    err = np.abs(x.astype(np.float32) - q.astype(np.float32) * s[:, None])
    assert (err <= s[:, None] * 0.5001).all()


def test_matmul_exact_integers():
    rng = np.random.default_rng(1)
    qa = rng.integers(-127, 128, (7, 256)).astype(np.int8)
    qw = rng.integers(-127, 128, (5, 256)).astype(np.int8)
    sa = np.ones(7, np.float32)
    sw = np.ones(5, np.float32)
    y = quant.matmul_i8(qa, sa, qw, sw)
    ref = np.array([[sum(int(a) * int(b) for a, b in zip(qa[i], qw[j])) for j in range(5)]
                    for i in range(7)], np.float32)
    assert np.array_equal(y, ref)


def test_pack_layout():
    q = np.arange(20 * 128, dtype=np.int64).reshape(20, 128).astype(np.int8)
    packed = quant.pack_i8(q)
    assert packed.size == 32 * 128
    for r in (0, 5, 15, 16, 19):
        for k in (0, 1, 15, 16, 63, 64, 127):
            assert packed[quant.frag_index_i8(r, k, 128)] == q[r, k]
