"""The balance loop's division (sjk_dev.h div_by_drecip): RN32(RN64(a * RN64(1/b))) is the correctly rounded
float quotient a / b for every numerator and divisor the seal can meet (reference sj_kvarn.h:980-987, SJ__FDIV).

The device computes exactly these IEEE operations (v_cvt_f64_f32, v_mul_f64, v_cvt_f32_f64, round to nearest
even), so numpy's float64 arithmetic reproduces them bit for bit; the check is against numpy's float32
division, which is IEEE's correctly rounded quotient. Numerators: every fp16 value (the first division,
M / s_col) and random floats over the range of M / s_col (the second, / s_row); divisors: the scale range
[exp(-0.3), exp(10)] (sj_kvarn.h:1001-1008), its ends, powers of two and significands next to 1 and 2.
"""
import numpy as np

LO, HI = np.float32(np.exp(-0.3)), np.float32(np.exp(10.0))


def divisors(rng, n):
    b = np.exp(rng.uniform(-0.3, 10.0, n)).astype(np.float32)
    edge = [LO, HI, 1.0, 2.0, 4.0, 1024.0, 16384.0]
    for e in range(0, 14):
        edge += [np.nextafter(np.float32(2.0 ** e), np.float32(0)), np.nextafter(np.float32(2.0 ** e), np.float32(np.inf))]
    b = np.concatenate([b, np.array(edge, np.float32)])
    return b[(b >= LO) & (b <= HI)]


def by_drecip(a, b):
    yd = 1.0 / b.astype(np.float64)                      # RN64(1 / b)
    return (a.astype(np.float64) * yd).astype(np.float32)


def check(a, b):
    with np.errstate(invalid="ignore", over="ignore"):
        for bb in b:
            want = a / np.float32(bb)
            got = by_drecip(a, np.full(1, bb, np.float32))
            w, g = want.view(np.uint32), got.view(np.uint32)
            nan = np.isnan(want)
            assert np.array_equal(np.isnan(got), nan), bb
            bad = (w != g) & ~nan
            assert not bad.any(), (float(bb), a[bad][:4], want[bad][:4], got[bad][:4])


def test_every_fp16_numerator():
    a = np.arange(1 << 16, dtype=np.uint16).view(np.float16).astype(np.float32)   # +-0, subnormals, +-inf, NaN
    check(a, divisors(np.random.default_rng(7), 3000))


def test_random_float_numerators():
    rng = np.random.default_rng(11)
    # |a| over the quotients M / s_col: [2^-24 / e^10, 65504 / e^-0.3]
    mag = np.exp2(rng.uniform(np.log2(2.0 ** -24 / float(HI)), np.log2(65504.0 / float(LO)), 1 << 17))
    a = (mag * rng.choice([-1.0, 1.0], mag.size)).astype(np.float32)
    check(a, divisors(rng, 1500))


def test_a_planted_mistake_is_caught():
    """The check is sharp: the float-reciprocal product RN32(a * RN32(1/b)) (one rounding too many) fails it."""
    a = np.arange(1 << 16, dtype=np.uint16).view(np.float16).astype(np.float32)
    a = a[np.isfinite(a)]
    b = divisors(np.random.default_rng(3), 50)
    wrong = 0
    for bb in b:
        want = (a / np.float32(bb)).view(np.uint32)
        got = (a * (np.float32(1.0) / np.float32(bb))).astype(np.float32).view(np.uint32)
        wrong += int((want != got).sum())
    assert wrong > 0
