"""Global settings and context stack, mirroring brainstate/environ.py.

Keys used by the spiking step: ``dt`` (ms, plain float here: brainunit is not available),
``t``, and ``precision`` (32 -> float32 / int32, brainstate/environ.py:143,1281-1295,1366).
"""
import contextlib
import threading

import numpy as np

_settings = {'precision': 32}
_local = threading.local()


def _stack():
    if not hasattr(_local, 'stack'):
        _local.stack = []
    return _local.stack


def set(**kwargs):  # noqa: A001 - mirrors brainstate.environ.set
    if 'precision' in kwargs and kwargs['precision'] not in (32,):
        raise NotImplementedError('the HIP engine computes in float32 / int32 (precision 32)')
    _settings.update(kwargs)


def pop(key, default=None):
    """Remove a global setting and return its value (brainstate/environ.py pop)."""
    if key not in _settings:
        if default is not None:
            return default
        raise KeyError(f'"{key}" is not a global setting')
    return _settings.pop(key)


def get(key, default=None, desc=None):
    for frame in reversed(_stack()):
        if key in frame:
            return frame[key]
    if key in _settings:
        return _settings[key]
    if default is not None:
        return default
    raise KeyError(f'"{key}" is not found in the context or the global settings '
                   f'({desc or "set it with brainstate_amd.environ.set"})')


def all():  # noqa: A001
    out = dict(_settings)
    for frame in _stack():
        out.update(frame)
    return out


@contextlib.contextmanager
def context(**kwargs):
    """Temporary settings, innermost wins (brainstate/environ.py:253-424)."""
    _stack().append(dict(kwargs))
    try:
        yield all()
    finally:
        _stack().pop()


def get_dt():
    """brainstate/environ.py:904-948 (dt in ms)."""
    return float(get('dt', desc='the time step dt'))


def dftype():
    return np.float32


def ditype():
    return np.int32
