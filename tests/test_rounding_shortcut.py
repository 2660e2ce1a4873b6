"""CPU check of the argument behind the device quantizer's rounding shortcut
(quant_pack in dq8_kernels.hip): for the group scale s = absmax / 127 and
|v| <= absmax, a = v * rs with rs any float within 1 ulp of 1 / s, and
t = a + copysign(0.5, a) in float32, trunc(t) equals round-half-away(v / s)
(the IEEE quotient, f32::round, tensor.rs:321-339 via weights.rs:117-136)
whenever t lies more than 2^-14 from every integer.  The values are chosen
next to the rounding boundaries, where the shortcut could go wrong; the
device's own results are compared with the oracle in the GPU tests."""
import numpy as np

F32 = np.float32


def round_half_away(q):
    return np.where(q >= 0, np.floor(q + 0.5), -np.floor(-q + 0.5))


def cases(rng, n):
    m = (rng.uniform(0.1, 100.0, n) * 2.0 ** rng.integers(-30, 30, n)).astype(F32)
    s = np.maximum(m / F32(127.0), np.finfo(F32).tiny).astype(F32)
    k = rng.integers(-127, 127, n)
    base = ((k + 0.5) * s.astype(np.float64)).astype(F32)
    v = (base.view(np.int32) + rng.integers(-40, 41, n).astype(np.int32)).view(F32)
    v = np.clip(v, -m, m).astype(F32)
    # plus plain values, exact ties and the extremes +-absmax
    plain = (rng.uniform(-1, 1, n) * m).astype(F32)
    v = np.where(rng.random(n) < 0.2, plain, v)
    v = np.where(rng.random(n) < 0.02, m * np.sign(rng.uniform(-1, 1, n)).astype(F32), v).astype(F32)
    return v, s


def test_shortcut_agrees_with_the_ieee_quotient_next_to_boundaries():
    rng = np.random.default_rng(1)
    taken = 0
    for _ in range(20):
        v, s = cases(rng, 200_000)
        want = np.clip(round_half_away((v / s).astype(F32).astype(np.float64)), -127, 127)
        inv = (F32(1.0) / s).astype(F32)
        for du in (-1, 0, 1):  # any reciprocal within 1 ulp
            rs = (inv.view(np.int32) + du).view(F32)
            a = (v * rs).astype(F32)
            t = (a + np.copysign(F32(0.5), a).astype(F32)).astype(F32)
            d = np.abs(t - np.rint(t)).astype(F32)
            fast = d > F32(2.0 ** -14)
            got = np.clip(np.trunc(t.astype(np.float64)), -127, 127)
            assert np.array_equal(got[fast], want[fast])
            taken += int(fast.sum())
    assert taken > 0


def test_a_tighter_margin_would_be_wrong():
    # The margin is needed: with 0 in place of 2^-14 the shortcut disagrees
    # with the IEEE quotient on some of these values.
    rng = np.random.default_rng(2)
    bad = 0
    for _ in range(5):
        v, s = cases(rng, 200_000)
        want = np.clip(round_half_away((v / s).astype(F32).astype(np.float64)), -127, 127)
        inv = (F32(1.0) / s).astype(F32)
        for du in (-1, 1):
            rs = (inv.view(np.int32) + du).view(F32)
            a = (v * rs).astype(F32)
            t = (a + np.copysign(F32(0.5), a).astype(F32)).astype(F32)
            got = np.clip(np.trunc(t.astype(np.float64)), -127, 127)
            bad += int((got != want).sum())
    assert bad > 0
