"""Loop drivers mirroring brainstate.transform.for_loop / jit.

The reference traces the step function once and runs it as an XLA While loop
(brainstate/transform/_loop_collect_return.py:487-572).  Here each step launches the HIP
kernels directly (no tracing); a network that fits the persistent runner runs whole loops
in one launch via ``brainstate_amd.nn.fuse``.
"""
import torch


def _stack(outs):
    if not outs:
        return outs
    first = outs[0]
    if torch.is_tensor(first):
        return torch.stack(outs)
    if isinstance(first, (tuple, list)):
        return type(first)(_stack([o[i] for o in outs]) for i in range(len(first)))
    if isinstance(first, dict):
        return {k: _stack([o[k] for o in outs]) for k in first}
    if first is None:
        return None
    return outs


def for_loop(f, *xs, length=None, reverse=False, unroll=1, pbar=None):
    """Call ``f(*x_t)`` for t along the leading axis of ``xs`` and stack the outputs
    (brainstate/transform/_loop_collect_return.py:487-572)."""
    if length is None:
        if not xs:
            raise ValueError('for_loop needs xs or length')
        length = len(xs[0])
    order = range(length - 1, -1, -1) if reverse else range(length)
    outs = [f(*[x[i] for x in xs]) for i in order]
    if reverse:
        outs = outs[::-1]
    return _stack(outs)


def jit(fn=None, **kwargs):
    """Kernels are compiled ahead of time; ``jit`` returns the function unchanged."""
    if fn is None:
        return lambda f: f
    return fn
