"""Recording pass of a ``for_loop`` step function: what the step does, found without running
it on the device.

The reference traces the step function once and compiles the trace into one scan
(brainstate/transform/_loop_collect_return.py:254,268).  ``for_loop`` here hands an E/I
network step to the persistent runner, and it may do so only when the runner computes what
the step computes at every step.  A recording pass calls the step function with

* module calls recorded and not run: the outermost calls are logged as (module, args,
  kwargs) and return a placeholder (``DryOut``) that aborts the pass when used;
* State writes aborting the pass (a step that assigns a State outside its modules does
  something the runner would not);
* reads of short-term States (neuron V, spikes, conductances, ...) returning the stored
  tensor marked, so that the only operations allowed on it are those that keep it a spike
  vector: slicing along the last axis, ``!= 0`` / ``> 0``, dtype conversions, copies and
  metadata.  Any other operation on a marked tensor aborts the pass, so a step cannot feed
  the stale state into anything the runner would have to recompute;
* the loop's per-step arguments replaced by placeholders (``StepArg``) in a first pass, so
  that a step whose module calls do not depend on them is found with one call, as the
  reference's single trace; a step that uses them (``20. if t < 5. else 0.``) is then
  recorded again step by step with the concrete values, still launching no kernel of the
  network (``Trace.dependent``);
* every allowed operation on a marked tensor producing an empty tensor of the right shape and
  dtype instead of computing (no device work while recording).
"""
import contextlib
import threading

import torch
from torch.overrides import TorchFunctionMode
from torch.utils._pytree import tree_flatten


class NotFusable(BaseException):
    """The step does something the runner does not: record no further.  A BaseException, so
    that a step function's own ``except Exception`` cannot swallow it."""


class Dependent(BaseException):
    """The step uses a per-step argument: record it again step by step."""


def _abort(exc):
    tr = _active.trace
    if tr is not None:
        tr.failed = exc
    raise exc


def _raise_dep(self, *a, **k):
    _abort(Dependent())


def _raise_nf(self, *a, **k):
    _abort(NotFusable())


_DUNDERS = ('__bool__', '__float__', '__int__', '__index__', '__complex__', '__len__',
            '__iter__', '__getitem__', '__setitem__', '__contains__', '__array__', '__format__',
            '__str__', '__lt__', '__le__', '__gt__', '__ge__', '__ne__', '__neg__',
            '__pos__', '__abs__', '__invert__', '__round__', '__floor__', '__ceil__',
            '__trunc__', '__call__', '__enter__', '__exit__')
_BINARY = ('add', 'sub', 'mul', 'truediv', 'floordiv', 'mod', 'pow', 'matmul', 'and', 'or',
           'xor', 'lshift', 'rshift', 'divmod')


def _placeholder(name, raiser, doc):
    ns = {'__slots__': ('index',), '__doc__': doc, '__hash__': object.__hash__,
          '__eq__': raiser,
          '__torch_function__': classmethod(lambda cls, *a, **k: raiser(None)),
          '__getattr__': raiser}
    for d in _DUNDERS:
        ns[d] = raiser
    for b in _BINARY:
        for pre in ('__', '__r', '__i'):
            ns[f'{pre}{b}__'] = raiser
    return type(name, (), ns)


StepArg = _placeholder('StepArg', _raise_dep,
                       'Stand-in for the i-th per-step argument of the loop in the first '
                       'recording pass: any use of its value aborts that pass.')
DryOut = _placeholder('DryOut', _raise_nf,
                      'What a module call returns while recording: any use of it aborts the '
                      'pass (the output of a call the runner makes is never seen by the step).')


def _new(cls, index):
    obj = object.__new__(cls)
    object.__setattr__(obj, 'index', index)
    return obj


class _Active(threading.local):
    trace = None


_active = _Active()


def active():
    """The recording in progress on this thread, or None."""
    return _active.trace


# operations allowed on a marked tensor: each maps a 0/1 (or bool) vector with ones exactly at
# the spikes to another such vector (or only reads metadata)
_META = {'shape', 'dtype', 'device', 'ndim', 'is_cuda', 'layout', 'requires_grad'}
_META_FN = {'size', 'dim', 'numel', '__len__', 'nelement', 'is_contiguous', 'element_size',
            'get_device', 'stride'}
_CAST_FN = {'bool', 'float', 'double', 'half', 'int', 'long', 'short', 'byte', 'to', 'clone',
            'contiguous', 'detach', 'type_as'}
_CMP_ZERO = {'ne', '__ne__', 'gt', '__gt__', 'not_equal', 'greater'}


class Mark:
    """A marked tensor: read from ``state`` (a short-term State) outside any module, and a
    spike-vector equivalent of it over the columns [lo, hi) of its last axis (``exact``:
    nothing but slicing and copies applied, so a spike State's values are the spikes)."""
    __slots__ = ('state', 'lo', 'hi', 'n', 'exact', 'tensor')

    def __init__(self, state, lo, hi, n, exact, tensor):
        self.state, self.lo, self.hi, self.n, self.exact = state, lo, hi, n, exact
        self.tensor = tensor   # keeps the tensor alive, so its id is not reused


def _slice_range(key, shape):
    """(lo, hi) of a basic slice along the last axis that keeps every other axis whole, else
    None."""
    if not shape:
        return None
    n = shape[-1]
    if isinstance(key, slice):
        key = (key,) if len(shape) == 1 else (Ellipsis, key)
    if not isinstance(key, tuple) or not key:
        return None
    last, lead = key[-1], key[:-1]
    if not isinstance(last, slice):
        return None
    if len(lead) == 1 and lead[0] is Ellipsis:
        pass
    elif len(lead) == len(shape) - 1 and all(isinstance(s, slice) and s == slice(None)
                                             for s in lead):
        pass
    else:
        return None
    for v in (last.start, last.stop, last.step):
        if v is not None and not isinstance(v, int):
            return None
    lo, hi, step = last.indices(n)
    if step != 1 or hi < lo:
        return None
    return lo, hi


class _Mode(TorchFunctionMode):
    def __init__(self, trace):
        super().__init__()
        self.trace = trace

    def __torch_function__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        tr = self.trace
        flat = tree_flatten((args, kwargs))[0]
        marked = None
        for a in flat:
            if isinstance(a, StepArg):
                _abort(Dependent())
            if isinstance(a, DryOut):
                _abort(NotFusable())
            if torch.is_tensor(a) and id(a) in tr.marks:
                if marked is not None:
                    _abort(NotFusable())
                marked = tr.marks[id(a)]
        if marked is None:
            return func(*args, **kwargs)
        name = getattr(func, '__name__', '')
        if name == '__get__':
            if getattr(getattr(func, '__self__', None), '__name__', None) in _META:
                return func(*args, **kwargs)
            _abort(NotFusable())
        if name in _META_FN:
            return func(*args, **kwargs)
        src = args[0] if args else None
        if not (torch.is_tensor(src) and id(src) in tr.marks):
            _abort(NotFusable())
        if name == '__getitem__' and len(args) == 2 and not kwargs:
            r = _slice_range(args[1], tuple(src.shape))
            if r is None:
                _abort(NotFusable())
            out = func(*args)   # a view: no device work
            return tr.mark(out, marked.state, marked.lo + r[0], marked.lo + r[1], marked.n,
                           marked.exact)
        if name in _CMP_ZERO:
            other = args[1] if len(args) > 1 else kwargs.get('other')
            if len(args) > 2 or isinstance(other, bool) or not isinstance(other, (int, float)) \
                    or other != 0:
                _abort(NotFusable())
            out = torch.empty(src.shape, dtype=torch.bool, device=src.device)
            return tr.mark(out, marked.state, marked.lo, marked.hi, marked.n, False)
        if name in _CAST_FN:
            try:
                meta = func(torch.empty(src.shape, dtype=src.dtype, device='meta'),
                            *args[1:], **kwargs)
            except Exception:
                _abort(NotFusable())
            if not torch.is_tensor(meta):
                _abort(NotFusable())
            dev = kwargs.get('device', None)
            for a in args[1:]:
                if isinstance(a, (str, torch.device)) or (torch.is_tensor(a) and
                                                          a.device != src.device):
                    dev = a if not torch.is_tensor(a) else a.device
            if dev is not None and torch.device(dev) != src.device and \
                    not (torch.device(dev).type == src.device.type and
                         torch.device(dev).index is None):
                _abort(NotFusable())
            out = torch.empty(src.shape, dtype=meta.dtype, device=src.device)
            exact = marked.exact and name in ('clone', 'contiguous', 'detach') or \
                (marked.exact and meta.dtype == src.dtype)
            return tr.mark(out, marked.state, marked.lo, marked.hi, marked.n, exact)
        _abort(NotFusable())


class Trace:
    """One recording: ``run(f, args)`` calls ``f`` once in recording mode and returns
    (calls, output); ``marks`` maps id(tensor) -> Mark."""

    def __init__(self):
        self.marks = {}
        self.failed = None
        self.calls = None

    def mark(self, t, state, lo, hi, n, exact):
        self.marks[id(t)] = Mark(state, lo, hi, n, exact, t)
        return t

    # hooks called by State and Module while this trace is active
    def read(self, state, value):
        from ._state import ShortTermState, State, ParamState
        if torch.is_tensor(value) and isinstance(state, State) and \
                not isinstance(state, ParamState) and \
                (isinstance(state, ShortTermState) or type(state) is State):
            if id(value) not in self.marks:
                n = int(value.shape[-1]) if value.dim() else 1
                self.mark(value, state, 0, n, n, True)
        return value

    def write(self, state):
        _abort(NotFusable())

    def call(self, module, args, kwargs):
        self.calls.append((module, args, kwargs))
        return _new(DryOut, len(self.calls) - 1)

    def run(self, f, args):
        self.calls = []
        self.failed = None
        prev = _active.trace
        _active.trace = self
        try:
            with _Mode(self):
                out = f(*args)
        finally:
            _active.trace = prev
        if self.failed is not None:   # raised inside f and swallowed there
            raise self.failed
        return self.calls, out


def step_args(n):
    return [_new(StepArg, j) for j in range(n)]


@contextlib.contextmanager
def rng_guard():
    """Snapshot the host and device random states; ``restore()`` puts them back."""
    import random

    import numpy as np
    saved = [random.getstate(), np.random.get_state(), torch.get_rng_state()]
    cuda = torch.cuda.is_available() and torch.cuda.is_initialized()
    if cuda:
        saved.append(torch.cuda.get_rng_state_all())

    class G:
        def changed(self):
            now = [random.getstate(), np.random.get_state(), torch.get_rng_state()]
            if cuda:
                now.append(torch.cuda.get_rng_state_all())
            if now[0] != saved[0] or not torch.equal(now[2], saved[2]):
                return True
            a, b = now[1], saved[1]
            if a[0] != b[0] or not np.array_equal(a[1], b[1]) or tuple(a[2:]) != tuple(b[2:]):
                return True
            return cuda and any(not torch.equal(x, y) for x, y in zip(now[3], saved[3]))

        def restore(self):
            random.setstate(saved[0])
            np.random.set_state(saved[1])
            torch.set_rng_state(saved[2])
            if cuda:
                torch.cuda.set_rng_state_all(saved[3])
    yield G()
