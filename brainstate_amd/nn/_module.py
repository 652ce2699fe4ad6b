"""Module / Dynamics bases mirroring brainstate/nn/_module.py and brainstate/nn/_dynamics.py.

``Module.__call__`` runs ``update`` (brainstate/nn/_module.py:242-243).  ``Dynamics`` adds
before-update hooks run ahead of ``update`` and after-update hooks run after it
(brainstate/nn/_dynamics.py:477-500): the first is how a post-synaptic neuron advances the
synapses projecting onto it, the second how delays record a state after every step
(``prefetch_delay`` / ``output_delay``, :222-298).
"""
import contextlib
import threading
from collections import OrderedDict

import numpy as np

from .. import _trace

_calls = threading.local()


@contextlib.contextmanager
def record_calls():
    """Record the outermost module calls made inside the block, as (module, args, kwargs)
    in call order (calls a module makes of other modules are not listed)."""
    log = []
    prev = getattr(_calls, 'log', None), getattr(_calls, 'depth', 0)
    _calls.log, _calls.depth = log, 0
    try:
        yield log
    finally:
        _calls.log, _calls.depth = prev


def _size(x):
    if isinstance(x, (int, np.integer)):
        return (int(x),)
    return tuple(int(v) for v in x)


class Module:
    __module__ = 'brainstate_amd.nn'

    def __init__(self, name=None):
        self.name = name

    def __call__(self, *args, **kwargs):
        tr = _trace._active.trace
        if tr is not None:   # a for_loop recording pass: logged, not run
            return tr.call(self, args, kwargs)
        log = getattr(_calls, 'log', None)
        if log is None:
            return self._run(*args, **kwargs)
        if _calls.depth == 0:
            log.append((self, args, kwargs))
        _calls.depth += 1
        try:
            return self._run(*args, **kwargs)
        finally:
            _calls.depth -= 1

    def _run(self, *args, **kwargs):
        return self.update(*args, **kwargs)

    def update(self, *args, **kwargs):
        raise NotImplementedError(f'{type(self).__name__}.update')

    def init_state(self, *args, **kwargs):
        pass

    def children(self):
        for v in list(vars(self).values()):
            if isinstance(v, Module):
                yield v
            elif isinstance(v, (list, tuple)):
                for x in v:
                    if isinstance(x, Module):
                        yield x
            elif isinstance(v, dict):
                for x in v.values():
                    if isinstance(x, Module):
                        yield x

    def nodes(self):
        """All modules reachable from this one (self first), each once."""
        seen, order, stack = set(), [], [self]
        while stack:
            m = stack.pop(0)
            if id(m) in seen:
                continue
            seen.add(id(m))
            order.append(m)
            stack.extend(m.children())
        return order


class Dynamics(Module):
    __module__ = 'brainstate_amd.nn'

    def __init__(self, in_size, name=None):
        super().__init__(name=name)
        self.in_size = _size(in_size)
        self.out_size = self.in_size
        self._before_updates = OrderedDict()
        self._after_updates = OrderedDict()

    @property
    def varshape(self):
        return self.in_size

    @property
    def num(self):
        return int(np.prod(self.in_size))

    @property
    def before_updates(self):
        return self._before_updates

    @property
    def after_updates(self):
        return self._after_updates

    def add_before_update(self, key, fn):
        if key in self._before_updates:
            raise KeyError(f'{key} has been registered in before_updates of {self}')
        self._before_updates[key] = fn

    def add_after_update(self, key, fn):
        if key in self._after_updates:
            raise KeyError(f'{key} has been registered in after_updates of {self}')
        self._after_updates[key] = fn

    def get_before_update(self, key):
        if key not in self._before_updates:
            raise KeyError(f'{key} is not registered in before_updates of {self}')
        return self._before_updates[key]

    def get_after_update(self, key):
        if key not in self._after_updates:
            raise KeyError(f'{key} is not registered in after_updates of {self}')
        return self._after_updates[key]

    def has_before_update(self, key):
        return key in self._before_updates

    def has_after_update(self, key):
        return key in self._after_updates

    def prefetch(self, item):
        """Reference to a state that may not exist yet (brainstate/nn/_dynamics.py:192-220)."""
        from ._delay import Prefetch
        return Prefetch(self, item)

    def prefetch_delay(self, state, *time_and_index, init=None, interpolation=None, **kwargs):
        """The state ``time`` ago, recorded after every update (:222-262)."""
        from ._delay import PrefetchDelayAt
        return PrefetchDelayAt(self, state, *time_and_index, delay_init=init,
                               interpolation=interpolation, **kwargs)

    def output_delay(self, *time_and_index, init=None, interpolation=None, **kwargs):
        """The update's output ``time`` ago (:264-298)."""
        from ._delay import OutputDelayAt
        return OutputDelayAt(self, *time_and_index, interpolation=interpolation,
                             delay_init=init, **kwargs)

    def children(self):
        yield from super().children()
        for fn in list(self._before_updates.values()) + list(self._after_updates.values()):
            if isinstance(fn, Module):
                yield fn

    def _run(self, *args, **kwargs):
        for fn in self._before_updates.values():
            if hasattr(fn, '_receive_update_input'):
                fn(*args, **kwargs)
            else:
                fn()
        ret = self.update(*args, **kwargs)
        for fn in self._after_updates.values():
            if hasattr(fn, '_not_receive_update_output'):
                fn()
            else:
                fn(ret)
        return ret


def init_all_states(target, *args, **kwargs):
    """Call ``init_state`` on every module of the tree (brainstate/nn/_collective_ops.py:299-346).

    Synapses first, delays last (they size their history from the states they record, as
    brainstate's call_order(3) on Delay.init_state arranges), everything else in between.
    """
    nodes = target.nodes()
    first = [m for m in nodes if getattr(m, '_init_first', False)]
    last = [m for m in nodes if getattr(m, '_init_last', False)]
    rest = [m for m in nodes if m not in first and m not in last]
    for m in first + rest + last:
        m.init_state(*args, **kwargs)
    return target
