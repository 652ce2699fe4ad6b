"""fp32 exp / exprel, restated in numpy float32 arithmetic (test infrastructure only).

The reference's exp-Euler (brainstate/nn/_exp_euler.py:246) calls ``u.math.exprel``
(brainunit) and the HH rates (examples/100_hh_neuron_model.py:49-64) call
``jnp.exp``/``exprel``.  Those library routines are not available here and differ by
an ulp between libms, so the oracle fixes one method and the device kernels use the
same one:

    n = rint(x*log2e);  r = fma(-n, L_lo, fma(-n, L_hi, x));  e^x = 2^n * P7(r)  (Cody & Waite)
    exprel(z) = Taylor_7(z) for |z| < 1/2, else (e^z - 1)/z
    polynomials by Horner's rule with fused multiply-adds

Every step is one correctly rounded float32 operation (+, -, *, /, rint or fma), so this
gives the same bits as the gfx950 code, which is compiled with -ffp-contract=off and
writes each fused multiply-add explicitly.  ``fma32`` emulates the binary32
fusedMultiplyAdd exactly in float64 (see its docstring).

Pinned by: tests/test_oracle_math.py -- fma32 equal to the C library's fmaf on random and
near-tie inputs, max error vs float64 numpy.exp / expm1 (<= 2 ulp over a dense sweep),
exprel(0) = 1, continuity at |z| = 1/2, and the exp-Euler known answers of
brainstate/nn/_exp_euler_test.py:29-97.
"""
import numpy as np

F = np.float32
LOG2E = F(1.4426950408889634)
LN2_HI = F(0.693145751953125)
LN2_LO = F(0.6931471805599453 - 0.693145751953125)
XMAX = F(88.0)
XMIN = F(-87.0)
SERIES = F(0.5)
_EXP_C = [F(1.0 / 5040.0), F(1.0 / 720.0), F(1.0 / 120.0), F(1.0 / 24.0),
          F(1.0 / 6.0), F(0.5), F(1.0), F(1.0)]
_EXPREL_C = [F(1.0 / 40320.0), F(1.0 / 5040.0), F(1.0 / 720.0), F(1.0 / 120.0),
             F(1.0 / 24.0), F(1.0 / 6.0), F(0.5), F(1.0)]


def fma32(a, b, c):
    """fl32(a*b + c) with a single rounding (binary32 fusedMultiplyAdd), elementwise.

    a*b is exact in float64 (24 + 24 <= 53 bits).  s = fl64(a*b + c) and its exact error e
    (TwoSum, Knuth TAOCP vol. 2, 4.2.2) give the exact sum s + e; moving s to its odd
    neighbour when e != 0 and s is even rounds the sum to odd at 53 bits, and rounding that
    to nearest-even at 24 bits is then correctly rounded because 53 >= 24 + 2 (Boldo &
    Melquiond, "Emulation of FMA and correctly rounded sums: proved algorithms using
    rounding to odd", IEEE TC 2008).
    """
    a = np.asarray(a, F)
    b = np.asarray(b, F)
    c = np.asarray(c, F)
    p = a.astype(np.float64) * b.astype(np.float64)
    c64 = c.astype(np.float64)
    s = np.asarray(p + c64)
    bb = s - p
    e = (p - (s - bb)) + (c64 - bb)
    even = (s.view(np.int64) & 1) == 0
    fix = (e != 0) & even & np.isfinite(s)
    s = np.where(fix, np.nextafter(s, np.where(e > 0, np.inf, -np.inf)), s)
    return s.astype(F)


def _pow2i(n):
    n = np.asarray(n, dtype=np.int32)
    return ((n + 127).astype(np.uint32) << np.uint32(23)).view(np.float32)


def expf(x):
    x = np.asarray(x, dtype=F)
    x = np.minimum(np.maximum(x, XMIN), XMAX)
    n = np.rint(x * LOG2E).astype(F)
    r = fma32(-n, LN2_HI, x)
    r = fma32(-n, LN2_LO, r)
    p = np.full_like(r, _EXP_C[0])
    for c in _EXP_C[1:]:
        p = fma32(p, r, c)
    return (p * _pow2i(n.astype(np.int32))).astype(F)


def exprel(z):
    z = np.asarray(z, dtype=F)
    p = np.full_like(z, _EXPREL_C[0])
    for c in _EXPREL_C[1:]:
        p = fma32(p, z, c)
    with np.errstate(divide='ignore', invalid='ignore'):
        big = ((expf(z) - F(1.0)) / z).astype(F)
    return np.where(np.abs(z) < SERIES, p, big).astype(F)
