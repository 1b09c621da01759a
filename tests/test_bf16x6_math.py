"""CPU: the arithmetic behind the bf16x6 kernels (the fp32 GEMM and the flash prefill's products),
pinned by what the mathematics fixes rather than by another run of the same formula.

The kernels split an fp32 value x into three bf16 parts, x0 = bf16(x), x1 = bf16(x - x0),
x2 = bf16(x - x0 - x1), each bf16() rounding to nearest even and each residual taken in fp32
(core/bf16x6.hpp, split3x2). They keep the six products x_i y_j with i + j <= 2.

* The split is exact: x0 + x1 + x2 == x for every finite fp32 x of normal range (24 significand
  bits = 3 x 8; each residual is exact in fp32).
* Each part is a bf16 value, so each kept product is exact in fp32 and in float64.
* The dropped terms x1 y2 + x2 y1 + x2 y2 stay within 2^-23 |x y| (|x1| <= 2^-8 |x| and
  |x2| <= 2^-8 |x1|, so each of the two cross terms is at most 2^-24 |x y|): the size of fp32's own
  rounding of a product. Measured on these samples: under 5e-8.
A mistake in the split (a missing residual, rounding by truncation, a dropped kept term) fails
one of these on random inputs."""
import numpy as np

RNG = np.random.default_rng(20261202)


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest-even bf16, returned as fp32 (what v_cvt_pk_bf16_f32 computes for finite x)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32)


def split3(x: np.ndarray):
    x = x.astype(np.float32)
    x0 = bf16_rne(x)
    r1 = (x - x0).astype(np.float32)
    x1 = bf16_rne(r1)
    r2 = (r1 - x1).astype(np.float32)
    x2 = bf16_rne(r2)
    return x0, x1, x2


def samples(n):
    mant = RNG.uniform(1.0, 2.0, n)
    expo = RNG.integers(-60, 60, n)
    sign = RNG.choice([-1.0, 1.0], n)
    x = (sign * mant * np.exp2(expo)).astype(np.float32)
    edge = np.array([1.0, -1.0, 1.0 + 2.0 ** -23, 2.0 - 2.0 ** -23, 3.0, 1.0 / 3.0, 65504.0,
                     np.float32(np.pi), -np.float32(np.e), 2.0 ** -60, 1.00390625, 1.0 + 2 ** -8 + 2 ** -16],
                    np.float32)
    return np.concatenate([x, edge])


def test_split_is_exact_and_parts_are_bf16():
    x = samples(200_000)
    x0, x1, x2 = split3(x)
    for p in (x0, x1, x2):  # each part is a bf16 value: its low 16 bits are zero
        assert not np.any(p.view(np.uint32) & 0xFFFF)
    recon = x0.astype(np.float64) + x1.astype(np.float64) + x2.astype(np.float64)
    assert np.array_equal(recon, x.astype(np.float64))
    ax = np.abs(x.astype(np.float64))
    assert np.all(np.abs(x1) <= 2.0 ** -8 * ax) and np.all(np.abs(x2) <= 2.0 ** -8 * np.abs(x1.astype(np.float64)))


def test_six_term_product_error_below_fp32_rounding():
    x, y = samples(200_000), samples(200_000)[::-1].copy()
    xs, ys = split3(x), split3(y)
    kept = sum(xs[i].astype(np.float64) * ys[j].astype(np.float64)
               for i in range(3) for j in range(3) if i + j <= 2)
    exact = x.astype(np.float64) * y.astype(np.float64)
    rel = np.abs(kept - exact) / np.abs(exact)
    assert float(rel.max()) <= 2.0 ** -23
    assert float(rel.max()) <= 5e-8  # what these samples reach (about 2^-24.3)
    # and each kept product is exact in fp32 (8 x 8 significand bits) wherever it is an fp32
    # normal number; products below 2^-126 (x2 y0 at exponents near -60) are subnormal and round
    normal = lambda p: (np.abs(p) >= 2.0 ** -126) & (np.abs(p) < 2.0 ** 127)
    checked = 0
    for i in range(3):
        for j in range(3 - i):
            p64 = xs[i].astype(np.float64) * ys[j].astype(np.float64)
            ok = normal(p64)
            p32 = (xs[i][ok] * ys[j][ok]).astype(np.float64)
            assert np.array_equal(p32, p64[ok])
            checked += int(ok.sum())
    assert checked > 1_000_000


def test_a_wrong_split_fails():
    """The checks above catch the plausible mistakes: truncating instead of rounding (the split
    stays exact but |x1| can reach 2^-7 |x|), and keeping only the four terms i, j <= 1."""
    x = samples(50_000)
    t0 = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)  # truncation
    t1 = (x - t0).astype(np.float32)
    t1 = (t1.view(np.uint32) & 0xFFFF0000).view(np.float32)
    assert np.any(np.abs(t1) > 2.0 ** -8 * np.abs(x))
    y = samples(50_000)[::-1].copy()
    xs, ys = split3(x), split3(y)
    four = sum(xs[i].astype(np.float64) * ys[j].astype(np.float64) for i in range(2) for j in range(2))
    exact = x.astype(np.float64) * y.astype(np.float64)
    assert float((np.abs(four - exact) / np.abs(exact)).max()) > 2.0 ** -23
