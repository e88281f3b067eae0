"""The q8_0 append kernel rounds half away from zero as trunc(y + copysign(0.49999997, y))
(then v_cvt_i32_f32, which truncates).  This pins the identity on the host in float32
arithmetic: exhaustively over every float in [0, 128) -- the range |y| = |x| * 127 / amax of
a finite quantized value -- in both signs, and on a random sample up to 2^23."""
import numpy as np

H = np.float32(0.49999997)


def round_half_away(x):
    t = np.trunc(x)
    return np.where(np.abs(x - t) >= np.float32(0.5), t + np.sign(x), t)


def trick(x):
    return np.trunc((x + np.copysign(H, x)).astype(np.float32))


def test_half_is_the_float_below_one_half():
    assert H == np.nextafter(np.float32(0.5), np.float32(0))


def test_identity_exhaustive_below_128():
    top = int(np.float32(128.0).view(np.uint32))
    step = 1 << 24
    for s in range(0, top, step):
        x = np.arange(s, min(s + step, top), dtype=np.uint32).view(np.float32)
        for y in (x, -x):
            assert np.array_equal(trick(y), round_half_away(y)), s


def test_identity_sampled_below_2_to_23():
    r = np.random.default_rng(5)
    u = r.integers(0, int(np.float32(2.0 ** 23).view(np.uint32)), 1 << 22, dtype=np.uint32)
    x = u.view(np.float32)
    for y in (x, -x):
        assert np.array_equal(trick(y), round_half_away(y))
