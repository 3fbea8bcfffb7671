"""Oracle checks of Tensor.maximum_scalar (tensor/tensor.mojo:4232) and
astype_f32_from_int (tensor/cast.mojo:5431-5437)."""
import numpy as np


def test_maximum_scalar_special_cases(oracle):
    x = np.array([-0.0, 0.0, -1.0, 2.0, np.nan, 0.5, -np.inf, np.inf, 0.25], np.float32)
    y = oracle.maximum_scalar_f32(x, 0.0)
    # where(x >= 0, x, 0): -0 >= 0 holds, so -0 stays -0; NaN >= 0 fails -> 0
    assert np.signbit(y[0]) and y[0] == 0
    assert not np.signbit(y[1])
    np.testing.assert_array_equal(y[2:], np.array([0, 2, 0, 0.5, 0, np.inf, 0.25], np.float32))
    # s away from 0: values equal to s return x itself, NaN returns s
    y = oracle.maximum_scalar_f32(np.array([0.25, 0.2, np.nan, -3.0], np.float32), 0.25)
    np.testing.assert_array_equal(y, np.array([0.25, 0.25, 0.25, 0.25], np.float32))
    y = oracle.maximum_scalar_f32(np.array([-0.0, -1.5, -2.5], np.float32), -2.0)
    assert np.signbit(y[0]) and y[1] == np.float32(-1.5) and y[2] == np.float32(-2.0)


def test_maximum_scalar_matches_fmax_off_the_special_cases(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(100_003).astype(np.float32)
    for s in (0.0, 0.5, -1.25, 3.0):
        np.testing.assert_array_equal(oracle.maximum_scalar_f32(x, s),
                                      np.fmax(x, np.float32(s)))


def test_astype_f32_from_int_rounding(oracle):
    p24 = 1 << 24
    x = np.array([p24, p24 + 1, p24 + 2, p24 + 3, -(p24 + 1), (1 << 63) - 1, -(1 << 63),
                  (1 << 40) + (1 << 16), (1 << 40) + (1 << 16) + 1, 7, -7, 0], np.int64)
    want = np.array([p24, p24, p24 + 2, p24 + 4, -p24, 2.0 ** 63, -2.0 ** 63,
                     2.0 ** 40, 2.0 ** 40 + 2 ** 17, 7, -7, 0], np.float64).astype(np.float32)
    np.testing.assert_array_equal(oracle.astype_f32_from_int(x), want)
    rng = np.random.default_rng(5)
    r = rng.integers(-(1 << 63), (1 << 63) - 1, size=50_000, dtype=np.int64)
    small = rng.integers(-(1 << 30), 1 << 30, size=50_000, dtype=np.int64)
    for v in (r, small):
        np.testing.assert_array_equal(oracle.astype_f32_from_int(v), v.astype(np.float32))
