"""Pins of the oracle's fp32 exp/exprel and exp-Euler (CPU only)."""
import numpy as np
import pytest

from oracle import bsmath, neuron

F = np.float32


def _ulp_err(got, ref64):
    ref32 = ref64.astype(F)
    return np.abs(got.astype(np.float64) - ref64) / np.spacing(np.abs(ref32)).astype(np.float64)


def _libm_fmaf():
    import ctypes
    import ctypes.util
    libm = ctypes.CDLL(ctypes.util.find_library('m') or 'libm.so.6')
    libm.fmaf.restype = ctypes.c_float
    libm.fmaf.argtypes = [ctypes.c_float] * 3
    return libm.fmaf


def test_fma32_equals_c_fmaf():
    """The oracle's binary32 fused multiply-add equals C99 fmaf (one rounding) bit for bit, on
    random operands and on near-cancelling ones where a*b + c is tiny."""
    fmaf = _libm_fmaf()
    rs = np.random.RandomState(7)
    a = (rs.randn(4000) * np.exp2(rs.randint(-20, 20, 4000))).astype(F)
    b = (rs.randn(4000) * np.exp2(rs.randint(-20, 20, 4000))).astype(F)
    for c in (rs.randn(4000).astype(F), (-(a * b)).astype(F),
              ((a * b) * F(1 + 2 ** -12)).astype(F)):
        got = bsmath.fma32(a, b, c)
        ref = np.array([fmaf(float(x), float(y), float(z)) for x, y, z in zip(a, b, c)], F)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_fma32_double_rounding_traps():
    """a*b lands exactly on a binary32 tie and c nudges the exact sum off it: one rounding goes
    the way of c, while rounding a*b + c to float64 first and then to float32 would round to
    even (1 + 2^-11) both times."""
    fmaf = _libm_fmaf()
    x = F(1 + 2 ** -12)                       # x*x = 1 + 2^-11 + 2^-24 (a tie in binary32)
    up, down = bsmath.fma32(x, x, F(2 ** -70)), bsmath.fma32(x, x, F(-2 ** -70))
    assert float(up) == 1 + 2 ** -11 + 2 ** -23
    assert float(down) == 1 + 2 ** -11
    assert float(up) == fmaf(float(x), float(x), 2 ** -70)
    assert float(down) == fmaf(float(x), float(x), -2 ** -70)
    naive = F(np.float64(x) * np.float64(x) + 2 ** -70)
    assert float(naive) == 1 + 2 ** -11              # what the trap catches


def test_expf_within_2ulp_of_float64():
    x = np.linspace(-87.0, 88.0, 1_000_001, dtype=F)
    err = _ulp_err(bsmath.expf(x), np.exp(x.astype(np.float64)))
    assert err.max() <= 2.0


def test_expf_special_points():
    assert bsmath.expf(F(0.0)) == F(1.0)
    assert bsmath.expf(F(1.0)) == F(np.e)         # fl32(e), within 1 ulp of exact
    assert bsmath.expf(F(-200.0)) > 0             # clamp, no underflow to garbage
    assert np.isfinite(bsmath.expf(F(200.0)))


def test_exprel_within_3ulp_and_limits():
    z = np.linspace(-30.0, 30.0, 1_000_001, dtype=F)
    z = z[z != 0]
    zd = z.astype(np.float64)
    err = _ulp_err(bsmath.exprel(z), np.expm1(zd) / zd)
    assert err.max() <= 3.0
    assert bsmath.exprel(F(0.0)) == F(1.0)
    # continuity across the series / direct switch at |z| = 1/2
    lo, hi = np.nextafter(F(0.5), F(0)), F(0.5)
    assert abs(float(bsmath.exprel(lo)) - float(bsmath.exprel(hi))) < 4e-7


def test_exprel_tiny_arguments_match_series():
    z = np.array([1e-30, -1e-20, 1e-8, -1e-6, 1e-4], dtype=F)
    assert np.allclose(bsmath.exprel(z), 1.0 + z.astype(np.float64) / 2, rtol=1e-7)


# ---- exp-Euler known answers: brainstate/nn/_exp_euler_test.py ----

def test_kat_exponential_decay():                     # :29-40
    x1 = neuron.exp_euler_step(lambda x: -x, lambda x: -np.ones_like(x), F(1.0), 0.01)
    np.testing.assert_allclose(x1, np.exp(-0.01), rtol=1e-7)


def test_kat_decay_with_time_constant():              # :42-54 (dt = 1 ms, tau = 10 ms)
    x1 = neuron.exp_euler_step(lambda x: -x / F(10.0), lambda x: np.full_like(x, F(-0.1)),
                               F(1.0), 1.0)
    assert np.allclose(x1, np.exp(-0.1))


def test_kat_linear_growth():                          # :56-67
    x1 = neuron.exp_euler_step(lambda x: np.full_like(x, F(2.0)), lambda x: np.zeros_like(x),
                               np.array([1.0], F), 0.1)
    np.testing.assert_allclose(x1, 1.0 + 2.0 * 0.1, rtol=1e-7)


def test_kat_stiff():                                  # :84-97
    x1 = neuron.exp_euler_step(lambda x: F(-100.0) * x, lambda x: np.full_like(x, F(-100.0)),
                               F(1.0), 0.1)
    np.testing.assert_allclose(x1, np.exp(-10.0), rtol=1e-2)
    assert x1 > 0


def test_kat_edge_cases():                             # :301-339
    x1 = neuron.exp_euler_step(lambda x: -x + F(1.0), lambda x: -np.ones_like(x), F(0.0), 0.01)
    assert x1 > 0
    x1 = neuron.exp_euler_step(lambda x: -x, lambda x: -np.ones_like(x), F(1.0), 1e-8)
    np.testing.assert_allclose(x1, 1.0)
    x1 = neuron.exp_euler_step(lambda x: F(-10.0) * x, lambda x: np.full_like(x, F(-10.0)),
                               F(1.0), 1.0)
    np.testing.assert_allclose(x1, np.exp(-10.0), rtol=1e-1)
    assert x1 > 0


def test_exp_euler_exact_for_linear_ode_f64():
    # x' = a - x/tau: exp-Euler is the exact solution for linear drift.
    tau, a, dt = 7.0, 3.0, 0.37
    x0 = np.array([0.5, -2.0, 10.0])
    x1 = neuron.exp_euler_step(lambda x: a - x / tau, lambda x: np.full_like(x, -1 / tau), x0, dt)
    exact = a * tau + (x0 - a * tau) * np.exp(-dt / tau)
    np.testing.assert_allclose(x1, exact, rtol=1e-12)


@pytest.mark.parametrize('dt,tau', [(0.1, 5.0), (0.1, 10.0), (0.05, 5.0)])
def test_decay_factor_is_fp32_of_exact(dt, tau):
    assert neuron.decay_factor(dt, tau) == F(np.exp(-dt / tau))
