"""Host-side behaviour of the brainstate-compatible layer (CPU only, no device work)."""
import numpy as np
import pytest
import torch

import brainstate_amd as bs
from brainstate_amd.nn import init


def test_efferent_pre_is_rejected():            # brainstate/nn/_event_fixedprob.py:123-140
    with pytest.raises(NotImplementedError, match="efferent_target='pre'"):
        bs.nn.EventFixedProb(10, 20, 0.1, 1.0, efferent_target='pre')


def test_bad_arguments_assert():                 # :125, :141, :145, :147
    with pytest.raises(AssertionError):
        bs.nn.EventFixedProb(10, 20, 0.1, 1.0, efferent_target='both')
    with pytest.raises(AssertionError):
        bs.nn.EventFixedProb(10, 20, 1.5, 1.0)
    with pytest.raises(AssertionError):
        bs.nn.EventFixedProb(10, 20, 0.1, 1.0, afferent_ratio=2.0)
    with pytest.raises(AssertionError):
        bs.nn.EventFixedProb(10, 20, '3', 1.0)


def test_zero_connections_use_fake_state():      # :198-200
    m = bs.nn.EventFixedProb(10, 20, 0.0, 1.5)
    assert m.conn_num == 0
    assert isinstance(m.weight, bs.FakeState) and m.weight.value == 1.5


def test_alias():
    assert bs.nn.EventFixedProb is bs.nn.EventFixedNumConn


def test_param_rules():                          # brainstate/nn/init.py:144-226
    assert init.param(0.6, (3, 4)) == 0.6        # scalar stays scalar (homogeneous)
    assert init.param(None, (3,)) is None
    with pytest.raises(ValueError):
        init.param(None, (3,), allow_none=False)
    a = init.param(lambda s: np.ones(s), (3, 4))
    assert a.shape == (3, 4)
    assert init.param(np.ones((1, 4)), (3, 4)).shape == (1, 4)   # broadcastable kept
    with pytest.raises(ValueError):
        init.param(np.ones((2, 4)), (3, 4))
    with pytest.raises(ValueError):
        init.param('x', (3,))


def test_environ_context_and_dt():
    with pytest.raises(KeyError):
        bs.environ.get('no_such_key')
    bs.environ.set(dt=0.1)
    assert bs.environ.get_dt() == 0.1
    with bs.environ.context(dt=0.05, t=3.0):
        assert bs.environ.get_dt() == 0.05 and bs.environ.get('t') == 3.0
        with bs.environ.context(dt=0.01):
            assert bs.environ.get_dt() == 0.01
        assert bs.environ.get_dt() == 0.05
    assert bs.environ.get_dt() == 0.1
    assert bs.environ.dftype() == np.float32 and bs.environ.ditype() == np.int32
    with pytest.raises(NotImplementedError):
        bs.environ.set(precision=64)


def test_state_value_semantics():
    s = bs.State(torch.zeros(3))
    s.value = torch.ones(3)
    assert torch.equal(s.value, torch.ones(3))
    with pytest.raises(ValueError):
        s.value = torch.ones(4)
    with pytest.raises(ValueError):
        s.value = bs.State(1)
    assert isinstance(bs.HiddenState(1), bs.ShortTermState)


def test_for_loop_stacks_like_scan():            # brainstate/transform/_loop_collect_return.py
    acc = bs.State(torch.zeros(()))

    def f(x):
        acc.value = acc.value + x
        return acc.value.clone()

    ys = bs.transform.for_loop(f, torch.arange(5.0))
    assert ys.tolist() == [0, 1, 3, 6, 10]
    ys = bs.transform.for_loop(lambda i: (torch.tensor(i), {'a': torch.tensor(2 * i)}),
                               [0, 1, 2])
    assert ys[0].tolist() == [0, 1, 2] and ys[1]['a'].tolist() == [0, 2, 4]
    assert bs.transform.jit(f) is f


def test_progress_bar_arguments():               # brainstate/transform/_progress_bar_test.py:83-131
    PB = bs.transform.ProgressBar
    with pytest.raises(ValueError):
        PB(freq=0)
    with pytest.raises(ValueError):
        PB(freq=2, count=5)
    assert PB(desc='Running').desc == 'Running'
    assert PB(desc=('step {i}', lambda d: {'i': d['i']})).desc[0] == 'step {i}'
    with pytest.raises(TypeError):
        PB(desc=('step {i}', 'not-callable'))
    with pytest.raises(TypeError):
        PB(desc=(123, lambda d: d))
    with pytest.raises(TypeError):
        PB(desc=123)
    with pytest.raises(ValueError):
        PB(desc=('only-one',))


def test_progress_bar_in_for_loop(capsys):       # _progress_bar_test.py:134-200
    PB, loop = bs.transform.ProgressBar, bs.transform.for_loop
    # steps per update as the reference resolves them: count -> n // count, default 5 %
    # (every step up to 20), explicit freq; updates stop at n, the close draws the rest
    assert PB(count=2).init(4).freq == 2
    assert PB().init(10).freq == 1 and PB().init(40).freq == 2
    assert PB(freq=3).init(10).freq == 3
    for n, pbar in ((4, PB(count=2)), (10, PB()), (40, PB()), (10, PB(freq=3)),
                    (5, PB(freq=2, desc='run')),
                    (5, PB(freq=2, desc=('iter {i}', lambda d: {'i': d['i']})))):
        ys = loop(lambda x: x * 2, torch.arange(float(n)), pbar=pbar)
        assert ys.tolist() == [2.0 * i for i in range(n)]
    with pytest.raises(ValueError):
        loop(lambda x: x * 2, torch.arange(4.0), pbar=PB(count=100))
    with pytest.raises(ValueError):
        loop(lambda x: x * 2, torch.arange(4.0), pbar=PB(freq=100))
    # an int is ProgressBar(freq=int)
    assert loop(lambda x: x + 1, torch.arange(6.0), pbar=2).tolist() == [1, 2, 3, 4, 5, 6]
    bar = PB(freq=3).init(10)
    for i in range(10):
        bar.step(i)
    assert bar.shown == 9
    bar.close()
    assert bar.shown == 10


def test_checkpointed_scan_known_answer_sequence():
    # brainstate/transform/_loop_collect_return_test.py:66-79: ys = [0, 0, 2, 6, 12]
    c = bs.State(torch.zeros(()))

    def f(i):
        out = c.value.clone()
        c.value = c.value + 2 * i
        return out

    assert bs.transform.for_loop(f, torch.arange(5.0)).tolist() == [0, 0, 2, 6, 12]


def test_module_tree_and_init_order():
    class Leaf(bs.nn.Module):
        def __init__(self, log, first=False):
            super().__init__()
            self.log = log
            self._init_first = first

        def init_state(self):
            self.log.append(self)

    log = []

    class Net(bs.nn.Module):
        def __init__(self):
            super().__init__()
            self.a = Leaf(log)
            self.b = [Leaf(log, first=True)]

    net = Net()
    bs.nn.init_all_states(net)
    assert log[0] is net.b[0] and log[1] is net.a


def test_exp_euler_operand_check_rejects_host_tensors():
    """exp_euler_step's kernel launch is preceded by a host check: a host tensor (or a size
    or layout mismatch) raises instead of reaching the kernel as a host pointer."""
    import torch
    from brainstate_amd.nn import _exp_euler
    x = torch.zeros(4)
    with pytest.raises(ValueError, match='on a GPU'):
        _exp_euler._check_operands((x, x, x, x), 4)


def test_external_input_forms():                 # N(x): scalar, one element, or one per neuron
    from brainstate_amd.nn._neurons import _ext_input
    V = torch.zeros(2, 5)
    assert _ext_input(20., V) == (20.0, None)
    assert _ext_input(np.array([3.5]), V) == (3.5, None)
    assert _ext_input(torch.tensor([[1.5]]), V) == (1.5, None)
    I, arr = _ext_input(torch.arange(5.), V)          # broadcast over the batch rows
    assert I == 0.0 and arr.shape == (2, 5) and arr.is_contiguous()
    assert arr[1].tolist() == [0., 1., 2., 3., 4.]
    I, arr = _ext_input(np.array([[1.], [2.]], np.float32), V)   # one input per replica
    assert arr[:, 3].tolist() == [1., 2.]
    with pytest.raises(ValueError, match='does not broadcast'):
        _ext_input(torch.ones(3), V)


def test_for_loop_eager_outputs_are_snapshots():
    """Each step's outputs are copied when the step returns them: a tensor the next step
    updates in place keeps each step's value, as scan's stacked ys do; outputs whose shape
    changes fall back to stacking what came, None leaves stay None, reverse order and empty
    loops stack as before."""
    import brainstate_amd as bs
    import torch
    old = bs.transform.fuse_loops
    bs.transform.fuse_loops = False
    try:
        v = torch.zeros(3)

        def f(x):
            v.add_(x)            # in place: every step returns the same tensor object
            return v, None, {'twice': 2 * v}

        ys, none, d = bs.transform.for_loop(f, torch.arange(1.0, 5.0))
        assert none is None
        assert ys[:, 0].tolist() == [1, 3, 6, 10] and d['twice'][:, 0].tolist() == [2, 6, 12, 20]
        ys = bs.transform.for_loop(lambda x: x * torch.ones(2), torch.arange(3.0), reverse=True)
        assert ys.tolist() == [[0, 0], [1, 1], [2, 2]]
        with pytest.raises(RuntimeError):   # shapes that differ cannot be stacked
            bs.transform.for_loop(lambda x: torch.ones(int(x) + 1), torch.arange(3.0))
        ys = bs.transform.for_loop(lambda x: torch.ones(2, dtype=torch.int64) * int(x)
                                   if x < 1 else torch.ones(2) * x, torch.arange(3.0))
        assert ys.dtype == torch.float32 and ys.tolist() == [[0, 0], [1, 1], [2, 2]]
        assert bs.transform.for_loop(lambda x: x, torch.zeros(0)) == []
        ys = bs.transform.for_loop(lambda x: float(x), torch.arange(3.0))
        assert ys == [0.0, 1.0, 2.0]
    finally:
        bs.transform.fuse_loops = old
