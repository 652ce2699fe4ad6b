"""Neuron and synapse state updates in fp32 (test infrastructure only).

exp-Euler, brainstate/nn/_exp_euler.py:226-249:
    J = d f / d x (diagonal, from ``vector_grad``),  phi = exprel(dt*J),
    x' = x + (dt*phi)*f(x)                      (left-to-right, as ``state + dt*phi*drift``)
Each multiply-add of the model updates is one fused multiply-add (``fma32``), as the
device code writes it; XLA likewise contracts multiply-adds when it compiles the
reference for a GPU, so the reference's own bits depend on such fusions.
Pinned by the known answers of brainstate/nn/_exp_euler_test.py:29-97,316-339 and by the
one-step LIF value printed in docs/tutorials/brain_dynamics/04_building_an_snn.ipynb
cell 5 (V_rest=-52, tau=10 ms, V0=-60, I=8, dt=0.1 ms -> -59.84079742 mV).

The models themselves (LIF / LIFRef / Expon / COBA / AlignPostProj) live in the
un-vendored ``brainpy.state``; their step ordering and refractory rule are restated
from the equations and are **parity unpinned** beyond the checks above:
  * Expon synapse: exact solution of dg/dt = -g/tau plus the delta input of the
    step's event mat-vec, ``g' = g*exp(-dt/tau) + in`` (exp-Euler of a linear ODE is
    this exponential; the decay factor is computed once in float64 and rounded).
  * COBA output: ``I = I_ext + g_e*(E_e - V) + g_i*(E_i - V)`` (sum_current_inputs
    order: external input first, then projections in registration order).
  * LIF membrane: ``f = ((V_rest - V) + R*I)*inv_tau``, ``J = (-1 - R*(g_e+g_i))*inv_tau``
    with ``inv_tau = fp32(1/tau)``: under jit the reference's ``/ tau`` by a constant is a
    multiplication, XLA's algebraic simplifier rewriting ``A / Const`` into
    ``A * InvertConstant(Const)``; the same holds for ``/ C`` and the HH rate scales.
  * LIFRef: a neuron is refractory for ``ref_steps`` steps after the spike step
    (the steps with 0 < t - t_spike < tau_ref on the dt grid, or <= tau_ref with
    ``ref_rule='closed'``); V is held there.  Which one brainpy.state uses is not pinned
    (its ``t - t_last <= tau_ref`` in float32 gives 49, 50 or 51 steps at 5 ms / 0.1 ms
    depending on how the absolute times round).
    Spike when V' >= V_th; hard reset V' = V_reset, in the spike step or (deferred_reset,
    brainpy.state's order) at the start of the next.
HH (examples/100_hh_neuron_model.py:49-93, reference-held): rates from the old V, V
and the gates each by exp-Euler from the old state, spike = (V < V_th) & (V' >= V_th).
"""
import numpy as np

from .bsmath import expf, exprel, fma32

F = np.float32
I32 = np.int32


def exp_euler_step(f, jac, x, dt):
    """Generic exp-Euler with a closed-form diagonal Jacobian (fp32 unless x is f64)."""
    x = np.asarray(x)
    dt = x.dtype.type(dt)
    if x.dtype == np.float64:
        z = dt * jac(x)
        phi = np.where(z == 0, 1.0, np.expm1(z) / np.where(z == 0, 1.0, z))
        return x + dt * phi * f(x)
    z = (dt * np.asarray(jac(x), F)).astype(F)
    phi = exprel(z)
    return fma32((dt * phi).astype(F), np.asarray(f(x), F), x)


def decay_factor(dt, tau):
    return F(np.exp(-float(dt) / float(tau)))


def ref_steps(tau_ref, dt, rule='open'):
    """Number of steps after a spike step with 0 < k*dt < tau_ref (``'open'``) or
    0 < k*dt <= tau_ref (``'closed'``, BrainPy's ``t - t_last <= tau_ref`` on the exact grid)."""
    q = float(tau_ref) / float(dt)
    n = int(np.ceil(q - 1e-9)) - 1 if rule == 'open' else int(np.floor(q + 1e-9))
    return max(n, 0)


class LIFParams:
    """``out='cuba'``: current-based synaptic output I += g * scale (brainpy.state CUBA, used
    by examples/400_CUBA_2005_bpu.py:42-58) instead of g * (E - V).  ``spk_reset='soft'``
    (docs/tutorials/brain_dynamics/04_building_an_snn.ipynb cells 5, 11): a spike subtracts
    V_th - V_reset from V' instead of setting V_reset.  ``deferred_reset``: that reset is
    applied at the start of the neuron's next step instead of in its spike step (brainpy.state's
    ``last_V = V - (V_th - V_reset) * last_spk``; examples/203_braintrace_for_snns.py:173-176),
    so a spiking neuron keeps V' >= V_th in between."""

    def __init__(self, V_rest=-60., V_th=-50., V_reset=-60., tau=20., R=1., tau_ref=5.,
                 I_ext=20., E_e=0., E_i=-80., tau_e=5., tau_i=10., dt=0.1, out='coba',
                 scale_e=1., scale_i=1., spk_reset='hard', ref_rule='open',
                 deferred_reset=False):
        self.cuba = out == 'cuba'
        self.soft_reset = spk_reset == 'soft'
        self.deferred_reset = bool(deferred_reset)
        self.scale_e, self.scale_i = F(scale_e), F(scale_i)
        self.V_rest, self.V_th, self.V_reset = F(V_rest), F(V_th), F(V_reset)
        self.tau, self.R, self.I_ext = F(tau), F(R), F(I_ext)
        self.inv_tau = F(F(1.0) / F(tau))
        self.E_e, self.E_i = F(E_e), F(E_i)
        self.dt = F(dt)
        self.de = decay_factor(dt, tau_e)
        self.di = decay_factor(dt, tau_i)
        self.ref_steps = I32(ref_steps(tau_ref, dt, ref_rule))


def lif_membrane(V, ge, gi, p):
    """One exp-Euler step of the COBA (or, p.cuba, CUBA) LIF membrane (no refractoriness, no
    reset).  CUBA: the current does not depend on V, so the Jacobian is -1/tau."""
    V, ge, gi = (np.asarray(x, F) for x in (V, ge, gi))
    if getattr(p, 'cuba', False):
        I = fma32(ge, np.full_like(V, p.scale_e), p.I_ext)
        I = fma32(gi, np.full_like(V, p.scale_i), I)
        J = np.full_like(V, (F(-1.0) * p.inv_tau).astype(F))
    else:
        I = fma32(ge, (p.E_e - V).astype(F), p.I_ext)
        I = fma32(gi, (p.E_i - V).astype(F), I)
        J = (fma32(-p.R, (ge + gi).astype(F), F(-1.0)) * p.inv_tau).astype(F)
    f = (fma32(p.R, I, (p.V_rest - V).astype(F)) * p.inv_tau).astype(F)
    phi = exprel((p.dt * J).astype(F))
    return fma32((p.dt * phi).astype(F), f, V)


def lif_reset(V, p):
    """V after a spike: V_reset, or V - (V_th - V_reset) with a soft reset."""
    V = np.asarray(V, F)
    if getattr(p, 'soft_reset', False):
        return (V - (p.V_th - p.V_reset).astype(F)).astype(F)
    return np.broadcast_to(np.asarray(p.V_reset, F), V.shape).astype(F)


def coba_lif_step(V, ge, gi, ref, in_e, in_i, p, spk_prev=None):
    """Fused Expon + COBA + LIFRef step.  Returns (V, ge, gi, ref, spike).  With
    ``p.deferred_reset`` the neurons of ``spk_prev`` (the previous step's spikes) are reset
    first and this step's spiking neurons keep V'."""
    deferred = getattr(p, 'deferred_reset', False)
    if deferred and spk_prev is not None:
        V = np.where(np.asarray(spk_prev) != 0, lif_reset(V, p), V).astype(F)
    ge = fma32(ge, p.de, in_e)
    gi = fma32(gi, p.di, in_i)
    Vn = lif_membrane(V, ge, gi, p)
    refr = ref > 0
    Vn = np.where(refr, V, Vn).astype(F)
    spk = (~refr) & (Vn >= p.V_th)
    if not deferred:   # hard reset V_reset, or subtractive: V' - (V_th - V_reset)
        Vn = np.where(spk, lif_reset(Vn, p), Vn).astype(F)
    ref = np.where(spk, p.ref_steps, np.where(refr, ref - 1, 0)).astype(I32)
    return Vn, ge, gi, ref, spk


# ---- Hodgkin-Huxley, examples/100_hh_neuron_model.py:25-93 ----

class HHParams:
    def __init__(self, ENa=50., gNa=120., EK=-77., gK=36., EL=-54.387, gL=0.03, C=1.0,
                 V_th=20., I_ext=0., E_e=0., E_i=-80., tau_e=5., tau_i=10., dt=0.05):
        self.ENa, self.gNa, self.EK, self.gK = F(ENa), F(gNa), F(EK), F(gK)
        self.EL, self.gL, self.C, self.V_th = F(EL), F(gL), F(C), F(V_th)
        self.inv_C = F(F(1.0) / F(C))
        self.I_ext, self.E_e, self.E_i = F(I_ext), F(E_e), F(E_i)
        self.dt = F(dt)
        self.de = decay_factor(dt, tau_e)
        self.di = decay_factor(dt, tau_i)


def hh_rates(V):
    """(am, bm, ah, bh, an, bn) at membrane potential V (mV), :49-64."""
    V = np.asarray(V, F)
    k10, k18, k20, k80 = (F(1.0) / F(c) for c in (10.0, 18.0, 20.0, 80.0))  # fp32 reciprocals
    am = (F(1.0) / exprel((-(V + F(40.0))) * k10)).astype(F)
    bm = (F(4.0) * expf((-(V + F(65.0))) * k18)).astype(F)
    ah = (F(0.07) * expf((-(V + F(65.0))) * k20)).astype(F)
    bh = (F(1.0) / (F(1.0) + expf((-(V + F(35.0))) * k10))).astype(F)
    an = (F(0.1) / exprel((-(V + F(55.0))) * k10)).astype(F)
    bn = (F(0.125) * expf((-(V + F(65.0))) * k80)).astype(F)
    return am, bm, ah, bh, an, bn


def hh_init(V):
    """Gates at steady state for V (init_state, :66-70): x_inf = a / (a + b)."""
    am, bm, ah, bh, an, bn = hh_rates(V)
    return (am / (am + bm)).astype(F), (ah / (ah + bh)).astype(F), (an / (an + bn)).astype(F)


def _gate(x, a, b, dt):
    f = fma32(a, (F(1.0) - x).astype(F), (-(b * x)).astype(F))
    J = (-(a + b)).astype(F)
    phi = exprel((dt * J).astype(F))
    return fma32((dt * phi).astype(F), f, x)


def hh_step(V, m, h, n, ge, gi, in_e, in_i, p):
    """Fused Expon + COBA + HH step.  Returns (V, m, h, n, ge, gi, spike)."""
    ge = fma32(ge, p.de, in_e)
    gi = fma32(gi, p.di, in_i)
    am, bm, ah, bh, an, bn = hh_rates(V)
    I = fma32(ge, (p.E_e - V).astype(F), p.I_ext)
    I = fma32(gi, (p.E_i - V).astype(F), I)
    gna = (p.gNa * m * m * m * h).astype(F)
    n2 = (n * n).astype(F)
    gk = (p.gK * n2 * n2).astype(F)
    acc = fma32(-gna, (V - p.ENa).astype(F), I)          # (I - INa - IK - IL), fused
    acc = fma32(-gk, (V - p.EK).astype(F), acc)
    acc = fma32(-p.gL, (V - p.EL).astype(F), acc)
    f = (acc * p.inv_C).astype(F)
    J = (((((-gna) - gk) - p.gL) - (ge + gi)) * p.inv_C).astype(F)
    phi = exprel((p.dt * J).astype(F))
    Vn = fma32((p.dt * phi).astype(F), f, V)
    mn = _gate(m, am, bm, p.dt)
    hn = _gate(h, ah, bh, p.dt)
    nn = _gate(n, an, bn, p.dt)
    spk = (V < p.V_th) & (Vn >= p.V_th)
    return Vn, mn, hn, nn, ge, gi, spk
