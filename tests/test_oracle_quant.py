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


def test_error_bound_and_range():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((50, 768)) * rng.uniform(0.01, 10, (50, 1))).astype(np.float16)
    q, s = quant.quantize_rows(x)
    assert np.abs(q).max() <= 127
    assert (np.abs(q).max(axis=1) == 127).all()          # every row uses the full range
    err = np.abs(x.astype(np.float32) - q.astype(np.float32) * s[:, None])
    assert (err <= s[:, None] * 0.5000001).all()


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
