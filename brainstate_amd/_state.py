"""State containers mirroring brainstate/_state.py (State :264, ShortTermState :1166,
HiddenState :1258, ParamState :1872, FakeState :1897, DelayState).

Values are torch device tensors (or Python scalars for homogeneous parameters).  There is
no tracing: the simulation loop is compiled by the whole-loop runner instead of XLA, so a
State here is a named, mutable handle on device memory.
"""
import torch

from . import _trace


class State:
    __module__ = 'brainstate_amd'

    def __init__(self, value, name=None):
        self._value = value
        self._name = name

    @property
    def value(self):
        tr = _trace._active.trace
        if tr is not None:   # a for_loop recording pass (brainstate_amd/_trace.py)
            return tr.read(self, self._value)
        return self._value

    @value.setter
    def value(self, v):
        tr = _trace._active.trace
        if tr is not None:
            tr.write(self)
        if isinstance(v, State):
            raise ValueError('Cannot assign a State object to State.value; assign its value.')
        old = self._value
        if torch.is_tensor(old) and torch.is_tensor(v) and old.shape != v.shape:
            raise ValueError(f'State shape mismatch: {tuple(old.shape)} vs {tuple(v.shape)}')
        self._value = v

    @property
    def name(self):
        return self._name

    def restore_value(self, v):
        tr = _trace._active.trace
        if tr is not None:
            tr.write(self)
        self._value = v

    def __repr__(self):
        v = self._value
        desc = f'{type(v).__name__}{tuple(v.shape)}' if torch.is_tensor(v) else repr(v)
        return f'{type(self).__name__}({desc})'


class ShortTermState(State):
    pass


class HiddenState(ShortTermState):
    pass


class ParamState(State):
    pass


class DelayState(ShortTermState):
    """History buffer of a Delay (brainstate/_state.py DelayState)."""
    pass


class FakeState:
    """Holds a value without registering it as a state (brainstate/_state.py:1897)."""

    def __init__(self, value, name=None):
        self.value = value
        self.name = name
