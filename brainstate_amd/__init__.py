"""brainstate_amd: MI355X (gfx950) engine for brainstate's spiking-network step.

The public surface mirrors brainstate's for this path: ``State`` classes, ``environ``,
``nn`` (event connectivity, neurons, synapses), ``transform.for_loop``.  All compute runs in
the HIP library ``_lib/libbsamd.so`` through the C ABI of include/brainstate_amd.h.
"""
from . import environ, nn, transform
from ._state import DelayState, FakeState, HiddenState, ParamState, ShortTermState, State

__version__ = '0.1.0'

__all__ = ['State', 'ShortTermState', 'HiddenState', 'ParamState', 'FakeState', 'DelayState',
           'environ', 'transform', 'nn']
