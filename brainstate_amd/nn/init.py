"""Parameter initialisation, mirroring brainstate/nn/init.py:144-226 (``param``)."""
import numpy as np
import torch

from .._state import State


def to_size(x):
    if x is None:
        return None
    if isinstance(x, (int, np.integer)):
        return (int(x),)
    return tuple(int(v) for v in x)


def _is_scalar(x):
    if isinstance(x, (bool, int, float, np.integer, np.floating)):
        return True
    if isinstance(x, np.ndarray) or torch.is_tensor(x):
        return x.ndim == 0
    return False


def _broadcastable(a, b):
    for x, y in zip(reversed(tuple(a)), reversed(tuple(b))):
        if x != 1 and y != 1 and x != y:
            return False
    return True


def param(parameter, sizes, batch_size=None, allow_none=True, allow_scalar=True):
    """None / scalar pass through (a scalar weight stays homogeneous, :188-189); a callable
    is called with the shape (batch first); an array must broadcast to ``sizes`` (:208-210)
    and is repeated along a leading batch axis when ``batch_size`` is given (:214-224)."""
    if parameter is None:
        if allow_none:
            return None
        raise ValueError('Expect a parameter with type of float, ArrayType, Initializer, or '
                         'Callable function, but we got None. ')
    if allow_scalar and _is_scalar(parameter):
        return parameter
    sizes = to_size(sizes)
    if callable(parameter) and not isinstance(parameter, State):
        if batch_size is not None:
            sizes = (batch_size,) + sizes
        return parameter(sizes)
    if isinstance(parameter, State):
        value = parameter.value
    elif isinstance(parameter, (np.ndarray, torch.Tensor)):
        value = parameter
    else:
        raise ValueError(f'Unknown parameter type: {type(parameter)}')
    if not _broadcastable(value.shape, sizes):
        raise ValueError(f'The shape of the parameter {tuple(value.shape)} does not match with '
                         f'the given size {sizes}')
    if batch_size is not None:   # :214-224: repeat along a new leading batch axis
        if value.ndim <= len(sizes):
            lib = torch if torch.is_tensor(value) else np
            value = lib.broadcast_to(value, tuple(sizes)) if tuple(value.shape) != tuple(sizes) \
                else value
            value = value[None].repeat(batch_size, *([1] * len(sizes))) if torch.is_tensor(value) \
                else np.repeat(value[None], batch_size, axis=0)
        elif value.shape[0] != batch_size:
            raise ValueError(f'The batch size of the parameter {value.shape[0]} does not match '
                             f'with the given batch size {batch_size}')
    return type(parameter)(value) if isinstance(parameter, State) else value


class Constant:
    """Initializer filling a constant (braintools.init.Constant)."""

    def __init__(self, value=0.0):
        self.value = value

    def __call__(self, shape):
        return np.full(shape, self.value, dtype=np.float32)


class Normal:
    """Normal(mean, scale) initializer drawn from a numpy generator (seeded)."""

    def __init__(self, mean=0.0, scale=1.0, seed=None):
        self.mean, self.scale = mean, scale
        self.rng = np.random.RandomState(seed)

    def __call__(self, shape):
        return self.rng.normal(self.mean, self.scale, shape).astype(np.float32)


class Uniform:
    def __init__(self, low=0.0, high=1.0, seed=None):
        self.low, self.high = low, high
        self.rng = np.random.RandomState(seed)

    def __call__(self, shape):
        return self.rng.uniform(self.low, self.high, shape).astype(np.float32)
