"""Module / Dynamics bases mirroring brainstate/nn/_module.py and brainstate/nn/_dynamics.py.

``Module.__call__`` runs ``update`` (brainstate/nn/_module.py:242-243).  ``Dynamics`` adds
before-update hooks run ahead of ``update`` (brainstate/nn/_dynamics.py:477-500), which is
how a post-synaptic neuron advances the synapses projecting onto it.
"""
from collections import OrderedDict

import numpy as np


def _size(x):
    if isinstance(x, (int, np.integer)):
        return (int(x),)
    return tuple(int(v) for v in x)


class Module:
    __module__ = 'brainstate_amd.nn'

    def __init__(self, name=None):
        self.name = name

    def __call__(self, *args, **kwargs):
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

    @property
    def varshape(self):
        return self.in_size

    @property
    def num(self):
        return int(np.prod(self.in_size))

    def add_before_update(self, key, fn):
        if key in self._before_updates:
            raise KeyError(f'before-update "{key}" already registered')
        self._before_updates[key] = fn

    def has_before_update(self, key):
        return key in self._before_updates

    def children(self):
        yield from super().children()
        for fn in self._before_updates.values():
            if isinstance(fn, Module):
                yield fn

    def __call__(self, *args, **kwargs):
        for fn in self._before_updates.values():
            fn()
        return self.update(*args, **kwargs)


def init_all_states(target, *args, **kwargs):
    """Call ``init_state`` on every module of the tree (brainstate/nn/_collective_ops.py:299-346).

    Synapses first, then everything else, so that neurons find their conductance channels
    initialised.
    """
    nodes = target.nodes()
    first = [m for m in nodes if getattr(m, '_init_first', False)]
    rest = [m for m in nodes if not getattr(m, '_init_first', False)]
    for m in first + rest:
        m.init_state(*args, **kwargs)
    return target
