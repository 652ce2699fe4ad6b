"""fp32 exp / exprel, restated in numpy float32 arithmetic (test infrastructure only).

The reference's exp-Euler (brainstate/nn/_exp_euler.py:246) calls ``u.math.exprel``
(brainunit) and the HH rates (examples/100_hh_neuron_model.py:49-64) call
``jnp.exp``/``exprel``.  Those library routines are not available here and differ by
an ulp between libms, so the oracle fixes one method and the device kernels use the
same one:

    n = rint(x*log2e);  r = (x - n*L_hi) - n*L_lo;  e^x = 2^n * P7(r)     (Cody & Waite)
    exprel(z) = Taylor_7(z) for |z| < 1/2, else (e^z - 1)/z

Every step is one correctly rounded float32 operation, so numpy float32 gives the
same bits as the gfx950 code compiled with -ffp-contract=off.

Pinned by: tests/test_oracle_math.py -- max error vs float64 numpy.exp / expm1
(<= 2 ulp over a dense sweep), exprel(0) = 1, continuity at |z| = 1/2, and the
exp-Euler known answers of brainstate/nn/_exp_euler_test.py:29-97.
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


def _pow2i(n):
    n = np.asarray(n, dtype=np.int32)
    return ((n + 127).astype(np.uint32) << np.uint32(23)).view(np.float32)


def expf(x):
    x = np.asarray(x, dtype=F)
    x = np.minimum(np.maximum(x, XMIN), XMAX)
    n = np.rint(x * LOG2E).astype(F)
    r = (x - n * LN2_HI).astype(F)
    r = (r - n * LN2_LO).astype(F)
    p = np.full_like(r, _EXP_C[0])
    for c in _EXP_C[1:]:
        p = (p * r + c).astype(F)
    return (p * _pow2i(n.astype(np.int32))).astype(F)


def exprel(z):
    z = np.asarray(z, dtype=F)
    p = np.full_like(z, _EXPREL_C[0])
    for c in _EXPREL_C[1:]:
        p = (p * z + c).astype(F)
    with np.errstate(divide='ignore', invalid='ignore'):
        big = ((expf(z) - F(1.0)) / z).astype(F)
    return np.where(np.abs(z) < SERIES, p, big).astype(F)
