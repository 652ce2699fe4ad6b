"""Neuron / synapse models the reference's E/I scripts use, on the fused HIP step kernels.

These stand in for the un-vendored ``brainpy.state`` classes that brainstate redirects to
(brainstate/nn/__init__.py:349-415) and that examples/105_COBA_HH_2007_braincell.py:54-91,
examples/400_CUBA_2005_bpu.py:36-66 and docs/tutorials/brain_dynamics/04_building_an_snn.ipynb
build networks from, plus the reference-held HH neuron of examples/100_hh_neuron_model.py.

Composition, as in brainpy.state: ``AlignPostProj(comm, syn=Expon, out=COBA, post=neuron)``
registers a conductance channel on the post-synaptic neuron; calling the projection with
spikes runs ``comm`` (the event mat-vec) and queues its output as the channel's delta
input; calling the neuron advances every channel's Expon conductance and the membrane in
one fused kernel (``bs_coba_lif_step`` / ``bs_coba_hh_step``): g' = g*exp(-dt/tau) + delta,
COBA current g*(E - V) (or, with ``out=CUBA``, g*scale), exp-Euler membrane, spike.  Up to
two channels per neuron (E and I) map onto the kernel's two; more raise NotImplementedError,
and the channels of one LIF neuron are all COBA or all CUBA.

Units: plain floats in mV, ms, mS (per cm^2 for HH); brainunit is not used.
"""
import numpy as np
import torch

from .. import environ
from .. import ops
from .._state import HiddenState, ShortTermState
from . import init
from ._module import Dynamics, Module

__all__ = ['Expon', 'COBA', 'CUBA', 'AlignPostProj', 'LIF', 'LIFRef', 'HH']


class _Desc:
    """``Cls.desc(...)``: a deferred constructor (brainpy.state ParamDescriber)."""

    def __init__(self, cls, args, kwargs):
        self.cls, self.args, self.kwargs = cls, args, kwargs

    def __call__(self):
        return self.cls(*self.args, **self.kwargs)


class _Describable:
    @classmethod
    def desc(cls, *args, **kwargs):
        return _Desc(cls, args, kwargs)


def _dev():
    from .. import _native
    _native.require_gpu()
    return torch.device('cuda', torch.cuda.current_device())


class Expon(Module, _Describable):
    """Exponential conductance dg/dt = -g/tau, g += delta input each step."""
    __module__ = 'brainstate_amd.nn'
    _init_first = True

    def __init__(self, in_size, tau=8.0, g_initializer=0.0, name=None):
        super().__init__(name=name)
        self.in_size = init.to_size(in_size)
        self.tau = float(tau)
        self.g_initializer = g_initializer
        self.delta = None

    def init_state(self, batch_size=None, **kwargs):
        n = int(np.prod(self.in_size))
        shape = (n,) if batch_size is None else (int(batch_size), n)
        g = init.param(self.g_initializer, (n,), batch_size)
        self.g = HiddenState(torch.zeros(shape, device=_dev()) + (
            float(g) if init._is_scalar(g) else torch.as_tensor(np.asarray(g, np.float32),
                                                                device=_dev()).reshape(shape)))
        self.delta = None

    def add_delta_input(self, key, value):
        self.delta = value if self.delta is None else self.delta + value


class COBA(Module, _Describable):
    """Conductance-based output: I = g * (E - V)."""
    __module__ = 'brainstate_amd.nn'

    def __init__(self, E, name=None):
        super().__init__(name=name)
        self.E = float(E)


class CUBA(Module, _Describable):
    """Current-based output: I = g * scale (brainpy.state CUBA; examples/400_CUBA_2005_bpu.py
    uses scale = 1 V, i.e. 1.0 with g in mS and currents in mA)."""
    __module__ = 'brainstate_amd.nn'

    def __init__(self, scale=1.0, name=None):
        super().__init__(name=name)
        self.scale = float(scale)


class AlignPostProj(Module):
    """Projection with post-aligned synapse (brainpy.state AlignPostProj)."""
    __module__ = 'brainstate_amd.nn'

    def __init__(self, *modules, comm, syn, out, post, name=None):
        super().__init__(name=name)
        if modules:
            raise NotImplementedError('prefetch modules before comm are not supported')
        self.comm = comm
        self.syn = syn() if isinstance(syn, _Desc) else syn
        self.out = out() if isinstance(out, _Desc) else out
        if not isinstance(self.syn, Expon) or not isinstance(self.out, (COBA, CUBA)):
            raise NotImplementedError('the fused kernels implement Expon synapses with COBA '
                                      'or CUBA output')
        self.post = post
        post._add_channel(self)

    def update(self, spk):
        current = self.comm(spk)
        self.syn.add_delta_input(self.name or id(self), current)
        return current


class _COBANeuron(Dynamics):
    def __init__(self, in_size, name=None):
        super().__init__(in_size, name=name)
        self._channels = []

    def _add_channel(self, proj):
        if len(self._channels) >= 2:
            raise NotImplementedError('the fused step kernels take at most two conductance '
                                      'channels (E and I)')
        if self._channels and isinstance(proj.out, CUBA) != self._cuba():
            raise NotImplementedError('the channels of one neuron must all be COBA or all CUBA')
        self._channels.append(proj)

    def _cuba(self):
        return bool(self._channels) and isinstance(self._channels[0].out, CUBA)

    def _channel_args(self, need_g=True):
        """(g, inputs, E, tau) of the two channels; a missing channel has a zero conductance
        (allocated only when ``need_g``), no input, E = 0 and tau = 1."""
        g, ins, E, tau = [], [], [], []
        for ch in self._channels:
            g.append(ch.syn.g.value)
            ins.append(ch.syn.delta)
            E.append(ch.out.scale if isinstance(ch.out, CUBA) else ch.out.E)
            tau.append(ch.syn.tau)
        while len(E) < 2:
            g.append(torch.zeros_like(self.V.value) if need_g else None)
            ins.append(None)
            E.append(0.0)
            tau.append(1.0)
        return g, ins, E, tau

    def _finish_channels(self, g):
        for ch, gv in zip(self._channels, g):
            ch.syn.g.value = gv
            ch.syn.delta = None

    def get_spike(self):
        return self.spike.value


def _state_shape(n, batch_size):
    """[n], or [batch_size, n] under init_all_states(batch_size=...) (states gain a leading
    batch axis; the step kernels run over all batch_size * n neurons at once)."""
    return (n,) if batch_size is None else (int(batch_size), n)


def _initial_V(V_initializer, n, batch_size, shape):
    V = init.param(V_initializer, (n,), batch_size)
    if init._is_scalar(V):
        V = np.full(shape, float(V), np.float32)
    V = V.detach().cpu().numpy() if torch.is_tensor(V) else np.asarray(V)
    return torch.as_tensor(np.ascontiguousarray(V, np.float32).reshape(shape), device=_dev())


def _ext_input(x, V):
    """(scalar input, per-neuron input or None): a one-element input is a scalar; an array
    must broadcast to the population's state shape (V's) and becomes each neuron's input."""
    if torch.is_tensor(x) or isinstance(x, np.ndarray):
        if np.prod(tuple(x.shape)) == 1:
            return float(x.reshape(()).item() if torch.is_tensor(x) else x.reshape(())), None
        t = torch.as_tensor(x, dtype=torch.float32, device=V.device)
        try:
            t = torch.broadcast_to(t, V.shape)
        except RuntimeError:
            raise ValueError(f'external input of shape {tuple(t.shape)} does not broadcast to '
                             f'the population\'s shape {tuple(V.shape)}') from None
        return 0.0, t.contiguous()
    return float(x), None


def _scalar_or_array(v, dtype=np.float32):
    """A neuron parameter: a float, or (more than one element) a numpy array of ``dtype``
    (fp32, as the step computes; float64 for a refractory period, whose step count is taken
    from the value given, as for a scalar)."""
    if torch.is_tensor(v):
        v = v.detach().cpu().numpy()
    a = np.asarray(v, np.float64)
    return float(a.reshape(())) if a.size == 1 else a.astype(dtype)


class _ParamCache:
    """The device arrays of a population's per-neuron parameters, built on first use and
    kept until a parameter is assigned another value (object), dt changes or the state's
    shape or device does (an array changed in place is not seen)."""

    def __init__(self):
        self.key = None
        self.value = None

    @staticmethod
    def _same(a, b):
        if isinstance(a, np.ndarray) or isinstance(b, np.ndarray):
            return a is b   # the cache holds the arrays, so an id is not reused meanwhile
        return type(a) is type(b) and a == b

    def get(self, key, build):
        if self.key is None or len(self.key) != len(key) or \
                not all(self._same(a, b) for a, b in zip(self.key, key)):
            self.value = build()
            self.key = key
        return self.value


class LIFRef(_COBANeuron, _Describable):
    """Leaky integrate-and-fire with refractory period; ``spk_reset='hard'`` sets V_reset after
    a spike, ``'soft'`` subtracts V_th - V_reset.  ``ref_rule`` fixes how many steps tau_ref
    holds a neuron after its spike step: ``'open'`` those with k*dt < tau_ref, ``'closed'``
    those with k*dt <= tau_ref (one more when tau_ref is a multiple of dt).

    ``reset_timing``: ``'next'`` (default) applies the reset at the start of the neuron's next
    update, as brainpy.state's neurons do (``last_V = V - (V_th - V_reset) * last_spk`` before
    the update; the reference-held neuron of examples/203_braintrace_for_snns.py:173-176 does
    the same): after a spike step ``V`` keeps the value that crossed ``V_th``, so ``V >=
    V_th`` exactly where ``get_spike()`` is set.  ``'same'`` resets within the spike step
    (BrainPy 2.x's LifRef): ``V`` reads ``V_reset`` right after it.  Spike trains and every
    other state are identical either way."""
    __module__ = 'brainstate_amd.nn'

    def __init__(self, in_size, R=1., tau=5., tau_ref=5., V_th=1., V_reset=0., V_rest=0.,
                 V_initializer=0., spk_reset='hard', ref_rule='open', reset_timing='next',
                 name=None):
        super().__init__(in_size, name=name)
        if spk_reset not in ('hard', 'soft'):
            raise ValueError(f"spk_reset must be 'hard' or 'soft', got {spk_reset!r}")
        if ref_rule not in ('open', 'closed'):
            raise ValueError(f"ref_rule must be 'open' or 'closed', got {ref_rule!r}")
        if reset_timing not in ('next', 'same'):
            raise ValueError(f"reset_timing must be 'next' or 'same', got {reset_timing!r}")
        self.spk_reset = spk_reset
        self.ref_rule = ref_rule
        self.reset_timing = reset_timing
        # scalars, or arrays of the population's shape (one value per neuron; eager steps only)
        self.R, self.tau = (_scalar_or_array(v) for v in (R, tau))
        self.tau_ref = _scalar_or_array(tau_ref, np.float64)
        self.V_th, self.V_reset, self.V_rest = (_scalar_or_array(v)
                                                for v in (V_th, V_reset, V_rest))
        self.V_initializer = V_initializer
        self._arrays = _ParamCache()

    def has_param_arrays(self):
        return any(isinstance(v, np.ndarray) for v in
                   (self.R, self.tau, self.tau_ref, self.V_th, self.V_reset, self.V_rest))

    def _param_arrays(self, V):
        """Per-neuron parameters for the step kernel (None when every one is a scalar),
        uploaded once and kept until a parameter is reassigned."""
        if not self.has_param_arrays():
            return None
        dt = float(environ.get_dt())
        key = (self.R, self.tau, self.tau_ref, self.V_th, self.V_reset, self.V_rest,
               self.ref_rule, dt, tuple(V.shape), V.device)
        return self._arrays.get(key, lambda: self._build_arrays(V, dt))

    def _build_arrays(self, V, dt):
        arr = lambda v: v if isinstance(v, np.ndarray) else None   # noqa: E731
        inv_tau = None
        if isinstance(self.tau, np.ndarray):
            inv_tau = (np.float32(1.0) / self.tau).astype(np.float32)   # fp32 reciprocal
        ref_steps = None
        if isinstance(self.tau_ref, np.ndarray):
            # ops.refractory_steps element-wise: the float64 value given over dt
            q = self.tau_ref.astype(np.float64) / dt
            n = np.ceil(q - 1e-9) - 1 if self.ref_rule == 'open' else np.floor(q + 1e-9)
            ref_steps = np.maximum(n, 0).astype(np.int32)
        return ops.lif_arrays(V, V_rest=arr(self.V_rest), V_th=arr(self.V_th),
                              V_reset=arr(self.V_reset), inv_tau=inv_tau, R=arr(self.R),
                              ref_steps=ref_steps)

    def init_state(self, batch_size=None, **kwargs):
        shape = _state_shape(self.num, batch_size)
        self.V = HiddenState(_initial_V(self.V_initializer, self.num, batch_size, shape))
        self.ref = HiddenState(torch.zeros(shape, dtype=torch.int32, device=_dev()))
        self.spike = ShortTermState(torch.zeros(shape, dtype=torch.bool, device=_dev()))

    def params(self, I_ext=0.0):
        """The scalar parameters (an array-valued one takes a placeholder here; the step
        reads it per neuron)."""
        _, _, E, tau = self._channel_args(need_g=False)   # E holds the CUBA scales for CUBA channels
        sc = lambda v, d: d if isinstance(v, np.ndarray) else v   # noqa: E731
        V_rest, V_th, V_reset = sc(self.V_rest, 0.0), sc(self.V_th, 0.0), sc(self.V_reset, 0.0)
        tau_m, R, tau_ref = sc(self.tau, 1.0), sc(self.R, 1.0), sc(self.tau_ref, 0.0)
        deferred = self.reset_timing == 'next'
        if self._cuba():
            return ops.lif_params(V_rest=V_rest, V_th=V_th, V_reset=V_reset,
                                  tau=tau_m, R=R, tau_ref=tau_ref, I_ext=I_ext,
                                  tau_e=tau[0], tau_i=tau[1], dt=environ.get_dt(),
                                  out='cuba', scale_e=E[0], scale_i=E[1],
                                  spk_reset=self.spk_reset, ref_rule=self.ref_rule,
                                  deferred_reset=deferred)
        return ops.lif_params(V_rest=V_rest, V_th=V_th, V_reset=V_reset,
                              tau=tau_m, R=R, tau_ref=tau_ref, I_ext=I_ext,
                              E_e=E[0], E_i=E[1], tau_e=tau[0], tau_i=tau[1],
                              dt=environ.get_dt(), spk_reset=self.spk_reset,
                              ref_rule=self.ref_rule, deferred_reset=deferred)

    def update(self, x=0.):
        g, ins, E, tau = self._channel_args()
        I, arr = _ext_input(x, self.V.value)
        p = self.params(I)
        spk = ops.coba_lif_step(self.V.value, g[0], g[1], self.ref.value, ins[0], ins[1], p,
                                I_ext=arr, arrays=self._param_arrays(self.V.value),
                                spk_prev=self.spike.value if p.deferred_reset else None)
        self._finish_channels(g)
        self.spike.value = spk.view(torch.bool).reshape(self.V.value.shape)
        return self.spike.value


class LIF(LIFRef):
    """LIF without a refractory period (LIFRef with tau_ref = 0)."""
    __module__ = 'brainstate_amd.nn'

    def __init__(self, in_size, R=1., tau=5., V_th=1., V_reset=0., V_rest=0., V_initializer=0.,
                 spk_reset='hard', reset_timing='next', name=None):
        super().__init__(in_size, R=R, tau=tau, tau_ref=0., V_th=V_th, V_reset=V_reset,
                         V_rest=V_rest, V_initializer=V_initializer, spk_reset=spk_reset,
                         reset_timing=reset_timing, name=name)


class HH(_COBANeuron, _Describable):
    """Hodgkin-Huxley neuron of examples/100_hh_neuron_model.py:25-93 (exp-Euler on V, m, h, n)."""
    __module__ = 'brainstate_amd.nn'

    def __init__(self, in_size, ENa=50., gNa=120., EK=-77., gK=36., EL=-54.387, gL=0.03,
                 V_th=20., C=1.0, V_initializer=-65., name=None):
        super().__init__(in_size, name=name)
        # scalars, or arrays of the population's shape (one value per neuron; eager steps only)
        self.ENa, self.gNa, self.EK, self.gK = (_scalar_or_array(v) for v in (ENa, gNa, EK, gK))
        self.EL, self.gL, self.V_th, self.C = (_scalar_or_array(v) for v in (EL, gL, V_th, C))
        self.V_initializer = V_initializer
        self._arrays = _ParamCache()

    def init_state(self, batch_size=None, **kwargs):
        shape = _state_shape(self.num, batch_size)
        dev = _dev()
        self.V = HiddenState(_initial_V(self.V_initializer, self.num, batch_size, shape))
        m, h, nn_ = (torch.empty(shape, device=dev) for _ in range(3))
        ops.hh_init(self.V.value, m, h, nn_)
        self.m, self.h, self.n = HiddenState(m), HiddenState(h), HiddenState(nn_)
        self.spike = ShortTermState(torch.zeros(shape, dtype=torch.bool, device=dev))

    def has_param_arrays(self):
        return any(isinstance(v, np.ndarray) for v in
                   (self.ENa, self.gNa, self.EK, self.gK, self.EL, self.gL, self.V_th, self.C))

    def _param_arrays(self, V):
        """Per-neuron parameters for the step kernel (None when every one is a scalar),
        uploaded once and kept until a parameter is reassigned."""
        if not self.has_param_arrays():
            return None
        key = (self.ENa, self.gNa, self.EK, self.gK, self.EL, self.gL, self.V_th, self.C,
               tuple(V.shape), V.device)
        return self._arrays.get(key, lambda: self._build_arrays(V))

    def _build_arrays(self, V):
        arr = lambda v: v if isinstance(v, np.ndarray) else None   # noqa: E731
        inv_C = (np.float32(1.0) / self.C).astype(np.float32) if isinstance(self.C, np.ndarray) \
            else None
        return ops.hh_arrays(V, ENa=arr(self.ENa), gNa=arr(self.gNa), EK=arr(self.EK),
                             gK=arr(self.gK), EL=arr(self.EL), gL=arr(self.gL), inv_C=inv_C,
                             V_th=arr(self.V_th))

    def params(self, I_ext=0.0):
        """The scalar parameters (an array-valued one takes a placeholder here)."""
        if self._cuba():
            raise NotImplementedError('the HH kernels implement COBA channels only')
        _, _, E, tau = self._channel_args(need_g=False)
        sc = lambda v, d: d if isinstance(v, np.ndarray) else v   # noqa: E731
        return ops.hh_params(ENa=sc(self.ENa, 0.), gNa=sc(self.gNa, 0.), EK=sc(self.EK, 0.),
                             gK=sc(self.gK, 0.), EL=sc(self.EL, 0.), gL=sc(self.gL, 0.),
                             C=sc(self.C, 1.), V_th=sc(self.V_th, 0.), I_ext=I_ext, E_e=E[0],
                             E_i=E[1], tau_e=tau[0], tau_i=tau[1], dt=environ.get_dt())

    def update(self, x=0.):
        g, ins, E, tau = self._channel_args()
        I, arr = _ext_input(x, self.V.value)
        p = self.params(I)
        spk = ops.coba_hh_step(self.V.value, self.m.value, self.h.value, self.n.value, g[0],
                               g[1], ins[0], ins[1], p, I_ext=arr,
                               arrays=self._param_arrays(self.V.value))
        self._finish_channels(g)
        self.spike.value = spk.view(torch.bool).reshape(self.V.value.shape)
        return self.spike.value
