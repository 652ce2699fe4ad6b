"""Host tests of for_loop's recording pass (brainstate_amd/_trace.py): module calls recorded
and not run, State writes and other uses of the recorded state aborting it, per-step
arguments detected, and the run-length merge of per-step inputs.  No GPU needed: the
modules here are plain Module subclasses over CPU tensors."""
import numpy as np
import pytest
import torch

from brainstate_amd import _trace, transform
from brainstate_amd._state import HiddenState, ParamState, ShortTermState
from brainstate_amd.nn._module import Module


class _Boom(Module):
    def update(self, *a, **k):
        raise AssertionError('a module ran while recording')


class _Pop:
    def __init__(self, n=10):
        self.spike = ShortTermState(torch.zeros(n, dtype=torch.bool))
        self.V = HiddenState(torch.zeros(n))
        self.w = ParamState(torch.ones(n))
        self.E, self.I, self.N = _Boom(), _Boom(), _Boom()


def _rec(f, *args):
    tr = _trace.Trace()
    calls, out = tr.run(f, list(args))
    return tr, calls, out


def test_calls_recorded_and_spike_slices_marked():
    p = _Pop(10)

    def step(t):
        spk = p.spike.value != 0.
        p.E(spk[:8])
        p.I(spk[8:])
        return p.N(20.)
    tr, calls, out = _rec(step, *_trace.step_args(1))
    assert [c[0] for c in calls] == [p.E, p.I, p.N]
    (_, (a,), _), (_, (b,), _), (_, args, kw) = calls
    ma, mb = tr.marks[id(a)], tr.marks[id(b)]
    assert ma.state is p.spike and (ma.lo, ma.hi) == (0, 8) and a.shape == (8,)
    assert mb.state is p.spike and (mb.lo, mb.hi) == (8, 10) and a.dtype == torch.bool
    assert args == (20.,) and kw == {}
    assert isinstance(out, _trace.DryOut) and out.index == 2


def test_batched_slices_and_conversions():
    p = _Pop(6)
    p.spike = ShortTermState(torch.zeros(3, 6, dtype=torch.bool))

    def step():
        spk = p.spike.value.to(torch.float32)
        p.E(spk[..., :4])
        p.I(spk[:, 4:])
        p.N(0.)
        return p.spike.value
    tr, calls, out = _rec(step)
    ma = tr.marks[id(calls[0][1][0])]
    mb = tr.marks[id(calls[1][1][0])]
    assert (ma.lo, ma.hi, mb.lo, mb.hi) == (0, 4, 4, 6)
    assert calls[0][1][0].dtype == torch.float32
    assert tr.marks[id(out)].state is p.spike


@pytest.mark.parametrize('bad', ['write', 'reduce', 'arith', 'index', 'use_out', 'restore'])
def test_other_uses_abort(bad):
    p = _Pop(10)

    def step():
        spk = p.spike.value
        if bad == 'write':
            p.V.value = torch.ones(10)
        elif bad == 'reduce':
            spk.sum()
        elif bad == 'arith':
            p.N(p.V.value * 2.)
        elif bad == 'index':
            p.E(spk[[0, 2]])
        elif bad == 'restore':
            p.V.restore_value(torch.ones(10))
        out = p.N(1.)
        if bad == 'use_out':
            out.float()
        return out
    with pytest.raises(_trace.NotFusable):
        _rec(step)


def test_step_arguments_detected():
    p = _Pop(4)
    for use in (lambda t: float(t), lambda t: t < 5., lambda t: t * 2, lambda t: f'{t}',
                lambda t: torch.as_tensor(t), lambda t: np.asarray(t), lambda t: t.item()):
        def step(t, use=use):
            use(t)
            p.N(0.)
        with pytest.raises(_trace.Dependent):
            _rec(step, *_trace.step_args(1))
    # passed on untouched (into a context or a module call) it is not a use
    from brainstate_amd import environ

    def step(t, x):
        with environ.context(t=t):
            p.N(x)
    tr, calls, _ = _rec(step, *_trace.step_args(2))
    assert isinstance(calls[0][1][0], _trace.StepArg) and calls[0][1][0].index == 1


def test_swallowed_abort_still_reported():
    p = _Pop(4)

    def step(t):
        try:
            float(t)
        except Exception:    # a BaseException is not caught here
            pass
        try:
            p.V.value = torch.ones(4)
        except BaseException:
            pass
        p.N(0.)
    with pytest.raises(_trace.Dependent):
        _rec(step, *_trace.step_args(1))

    def step2():
        try:
            p.V.value = torch.ones(4)
        except BaseException:
            pass
        p.N(0.)
    with pytest.raises(_trace.NotFusable):
        _rec(step2)


def test_plain_tensor_work_runs_and_modules_do_not():
    p = _Pop(4)
    seen = []

    def step():
        x = torch.arange(4.) * 2     # unrelated tensors compute normally
        seen.append(float(x.sum()))
        p.N(x)
    tr, calls, _ = _rec(step)
    assert seen == [12.0] and torch.equal(calls[0][1][0], torch.arange(4.) * 2)
    # outside a recording the hooks are inert
    assert _trace.active() is None
    p.V.value = torch.ones(4)
    assert torch.equal(p.V.value, torch.ones(4))


def test_rng_guard_detects_and_restores():
    with _trace.rng_guard() as g:
        assert not g.changed()
        a = torch.rand(3)
        np.random.rand()
        assert g.changed()
        g.restore()
        assert not g.changed()
        assert torch.equal(torch.rand(3), a)


def test_input_runs_merged():
    segs = transform._merge([1., 1., 2., 2., 2., 1.])
    assert segs == [(0, 2, 1.), (2, 3, 2.), (5, 1, 1.)]
    a, b = torch.ones(3), torch.zeros(3)
    segs = transform._merge([a, a.clone(), b, 5.])
    assert [(s[0], s[1]) for s in segs] == [(0, 2), (2, 1), (3, 1)]
    assert transform._merge([1., None]) is None
    # one number per step, straight from xs: runs found without calling the step
    xs = [torch.tensor([20., 20., 20., 0., 0.])]
    assert transform._schedule(xs, 0, 5, None) == [(0, 3, 20.), (3, 2, 0.)]
    assert transform._schedule([np.array([1, 1, 3])], 0, 3, None) == [(0, 2, 1.), (2, 1, 3.)]
    assert transform._schedule([torch.tensor([True, False, True])], 0, 3, None) is None
