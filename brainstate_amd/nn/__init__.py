"""brainstate.nn surface for the spiking-network step (event connectivity, neurons, synapses)."""
from . import init
from ._delay import (Delay, DelayAccess, InterpolationRegistry, OutputDelayAt, Prefetch,
                     PrefetchDelay, PrefetchDelayAt, StateWithDelay, not_receive_update_output,
                     receive_update_output)
from ._event import EventFixedNumConn, EventFixedProb, EventLinear, FixedNumConn
from ._exp_euler import exp_euler_step
from ._fuse import fuse
from ._module import Dynamics, Module, init_all_states
from ._neurons import COBA, CUBA, HH, LIF, AlignPostProj, Expon, LIFRef

__all__ = ['init', 'Module', 'Dynamics', 'init_all_states', 'FixedNumConn', 'EventFixedNumConn',
           'EventFixedProb', 'EventLinear', 'Expon', 'COBA', 'CUBA', 'AlignPostProj', 'LIF',
           'LIFRef', 'HH', 'fuse', 'Delay', 'DelayAccess', 'StateWithDelay', 'InterpolationRegistry',
           'Prefetch', 'PrefetchDelay', 'PrefetchDelayAt', 'OutputDelayAt',
           'receive_update_output', 'not_receive_update_output', 'exp_euler_step']
