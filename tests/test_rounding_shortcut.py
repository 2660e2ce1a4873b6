"""CPU check of the argument behind the device quantizer's rounding shortcut
(quant_pack in dq8_kernels.hip).  For the group scale s = absmax / 127 (IEEE
quotient) and |v| <= absmax, take a = v * rs with rs any float within 1 ulp
of 1 / s, and u = a + 128 in float32.  Whenever u lies more than 2^-14 from
every half-integer, rint(u) - 128 equals round-half-away(v / s) (the IEEE
quotient, f32::round, tensor.rs:321-339 via weights.rs:117-136), and lies in
[-127, 127] without a clamp.  The values are chosen next to the rounding
boundaries, where the shortcut could go wrong; the device's own results are
compared with the oracle in the GPU tests."""
import numpy as np

F32 = np.float32
MARGIN = F32(2.0 ** -14)


def round_half_away(q):
    return np.where(q >= 0, np.floor(q + 0.5), -np.floor(-q + 0.5))


def cases(rng, n):
    m = (rng.uniform(0.1, 100.0, n) * 2.0 ** rng.integers(-30, 30, n)).astype(F32)
    tiny = rng.random(n) < 0.05  # groups whose scale is FLT_MIN
    m = np.where(tiny, (rng.uniform(0.0, 127.0, n) * np.finfo(F32).tiny).astype(F32), m).astype(F32)
    s = np.maximum(m / F32(127.0), np.finfo(F32).tiny).astype(F32)
    k = rng.integers(-127, 127, n)
    base = ((k + 0.5) * s.astype(np.float64)).astype(F32)
    v = (base.view(np.int32) + rng.integers(-40, 41, n).astype(np.int32)).view(F32)
    v = np.clip(v, -m, m).astype(F32)
    # plus plain values and the extremes +-absmax
    plain = (rng.uniform(-1, 1, n) * m).astype(F32)
    v = np.where(rng.random(n) < 0.2, plain, v)
    v = np.where(rng.random(n) < 0.02, m * np.sign(rng.uniform(-1, 1, n)).astype(F32), v).astype(F32)
    return v, s


def shortcut(v, s, du, margin):
    rs = ((F32(1.0) / s).astype(F32).view(np.int32) + du).view(F32)
    a = (v * rs).astype(F32)
    u = (a + F32(128.0)).astype(F32)
    r = np.rint(u).astype(F32)
    f = (u - r).astype(F32)
    fast = (F32(0.5) - np.abs(f)).astype(F32) > margin
    return fast, r.astype(np.float64) - 128.0


def shortcut_fma(v, s, du, margin):
    # u = v * rs + 128 rounded once (an FMA): the product is exact in the
    # x87 extended format (48 significant bits), and so is the sum whenever
    # |v * rs| >= 2^-10 (64 bits); smaller products leave u within 2^-9 of
    # 128, where a second rounding cannot change rint(u) or the margin test.
    rs = ((F32(1.0) / s).astype(F32).view(np.int32) + du).view(F32)
    u = (v.astype(np.longdouble) * rs.astype(np.longdouble) + np.longdouble(128.0)).astype(F32)
    r = np.rint(u).astype(F32)
    f = (u - r).astype(F32)
    fast = (F32(0.5) - np.abs(f)).astype(F32) > margin
    return fast, r.astype(np.float64) - 128.0


def test_shortcut_agrees_with_the_ieee_quotient_next_to_boundaries():
    rng = np.random.default_rng(1)
    taken = 0
    for _ in range(20):
        v, s = cases(rng, 200_000)
        want = round_half_away((v / s).astype(F32).astype(np.float64))
        assert np.abs(want).max() <= 127
        for du in (-1, 0, 1):  # any reciprocal within 1 ulp
            for form in (shortcut, shortcut_fma):  # u from a multiply and an add, or one FMA
                fast, got = form(v, s, du, MARGIN)
                assert np.array_equal(got[fast], want[fast])
                assert np.abs(got[fast]).max() <= 127
                taken += int(fast.sum())
    assert taken > 0


def test_a_tighter_margin_would_be_wrong():
    # The margin is needed: with 0 in place of 2^-14 the shortcut disagrees
    # with the IEEE quotient on some of these values.
    rng = np.random.default_rng(2)
    bad = 0
    for _ in range(5):
        v, s = cases(rng, 200_000)
        want = round_half_away((v / s).astype(F32).astype(np.float64))
        for du in (-1, 1):
            fast, got = shortcut(v, s, du, F32(0.0))
            bad += int((got[fast] != want[fast]).sum())
    assert bad > 0


def test_multiply_shift_division_is_exact_below_2_31():
    # The quantizer finds a wave's row as floor(n / d) = (n * mul) >> (31 + l),
    # l = ceil(log2 d), mul = ceil(2^(31+l) / d) (Granlund and Montgomery 1994,
    # Thm 4.2).  Checked against integer division for divisors up to 2^24 and
    # numerators next to multiples of d and at the 2^31 - 1 end.
    rng = np.random.default_rng(3)
    ds = np.unique(np.r_[np.arange(1, 300), rng.integers(1, 1 << 24, 2000), 1 << 20, (1 << 20) + 1, (1 << 24) - 1])
    for d in ds.tolist():
        l = (d - 1).bit_length()
        mul = ((1 << (31 + l)) + d - 1) // d
        assert mul < (1 << 32)
        qs = rng.integers(0, ((1 << 31) - 1) // d + 1, 200, dtype=np.int64)
        n = np.unique(np.clip(np.r_[qs * d, qs * d - 1, qs * d + d - 1, (1 << 31) - 1, 0], 0, (1 << 31) - 1))
        got = [(int(v) * mul) >> (31 + l) for v in n.tolist()]
        assert got == [int(v) // d for v in n.tolist()]
