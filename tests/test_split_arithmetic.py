"""The arithmetic behind the split-bf16 products (prlstm_amd/csrc/gemm_x6.hip), on the CPU.

Each fp32 value v is split into bf16 pieces v0 = bf16(v) (round to nearest even),
v1 = bf16(v - v0), v2 = v - v0 - v1, and a product a b is computed from the six largest
piece products.  These tests pin the facts the kernel's accuracy rests on, by exact
arithmetic in numpy: the split is exact (v2 is itself a bf16 value), the pieces shrink by
2^-8 each, and the three dropped products stay below 2^-23 |a b|.
"""

import numpy as np


def bf16_rne(x):
    """fp32 -> nearest bf16 (ties to even), returned as fp32 (round on the bit pattern)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return r.astype(np.uint32).view(np.float32)


def split3(v):
    v = np.asarray(v, dtype=np.float32)
    v0 = bf16_rne(v)
    r1 = (v - v0).astype(np.float32)          # exact in fp32
    v1 = bf16_rne(r1)
    v2 = (r1 - v1).astype(np.float32)         # exact in fp32
    return v0, v1, v2


def random_fp32(n, seed, lo=-60, hi=60):
    g = np.random.default_rng(seed)
    mant = g.uniform(1.0, 2.0, n).astype(np.float32)
    exp = g.integers(lo, hi, n)
    sign = g.choice([-1.0, 1.0], n)
    return (sign * mant * np.exp2(exp)).astype(np.float32)


def test_bf16_rounding_matches_a_reference_rule():
    """bf16_rne equals round-to-nearest on the value grid (checked in fp64 on random data)."""
    v = random_fp32(20000, 0)
    r = bf16_rne(v).astype(np.float64)
    vd = v.astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.abs(vd))) - 7)
    assert np.all(np.abs(r - vd) <= ulp / 2 * (1 + 1e-12))
    assert np.all(bf16_rne(r.astype(np.float32)) == r.astype(np.float32))  # on the grid


def test_split_is_exact_and_pieces_shrink():
    v = np.concatenate([random_fp32(50000, 1), np.array([1.0, -1.0, 3.0, 1.0 + 2.0 ** -23, 65504.0,
                                                         2.0 ** -100, 1e-30, 3.3e38], dtype=np.float32)])
    v0, v1, v2 = split3(v)
    assert np.array_equal(bf16_rne(v2), v2), "third piece is a bf16 value"
    s = v0.astype(np.float64) + v1.astype(np.float64) + v2.astype(np.float64)
    assert np.array_equal(s, v.astype(np.float64)), "v0 + v1 + v2 == v exactly"
    av = np.abs(v.astype(np.float64))
    assert np.all(np.abs(v1) <= 2.0 ** -8 * av * (1 + 2.0 ** -7))
    assert np.all(np.abs(v2) <= 2.0 ** -16 * av * (1 + 2.0 ** -6))


def test_dropped_products_below_fp32_rounding():
    a = random_fp32(50000, 2, -20, 20)
    b = random_fp32(50000, 3, -20, 20)
    a0, a1, a2 = (x.astype(np.float64) for x in split3(a))
    b0, b1, b2 = (x.astype(np.float64) for x in split3(b))
    exact = a.astype(np.float64) * b.astype(np.float64)
    kept = a0 * b0 + a0 * b1 + a1 * b0 + a0 * b2 + a1 * b1 + a2 * b0
    dropped = exact - kept
    assert np.allclose(dropped, a1 * b2 + a2 * b1 + a2 * b2, rtol=0, atol=0)
    assert np.all(np.abs(dropped) <= 2.0 ** -23 * np.abs(exact))
    # every piece product is exact in fp32 (8-bit by 8-bit significands)
    for p in (a0 * b0, a0 * b1, a1 * b0, a0 * b2, a1 * b1, a2 * b0):
        assert np.array_equal(p.astype(np.float32).astype(np.float64), p)


def test_one_piece_operand_gives_three_products():
    """A bf16 operand (b1 = b2 = 0) leaves only a0 b, a1 b, a2 b non-zero, whose sum is exact:
    the three-product kernel computes the same terms as the six-product one."""
    a = random_fp32(20000, 4, -20, 20)
    b = bf16_rne(random_fp32(20000, 5, -20, 20))
    b0, b1, b2 = split3(b)
    assert np.all(b1 == 0) and np.all(b2 == 0) and np.array_equal(b0, b)
    a0, a1, a2 = (x.astype(np.float64) for x in split3(a))
    assert np.array_equal((a0 + a1 + a2) * b.astype(np.float64), a.astype(np.float64) * b.astype(np.float64))
