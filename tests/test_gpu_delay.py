"""GPU tests of the ring-buffer Delay (bs_delay_* kernels through brainstate_amd.nn.Delay):
the reference's own delay tests (brainstate/nn/_delay_test.py) restated, bit-equality with the
oracle restatement for every read mode, and a module-built E/I net with delayed spikes."""
import os
import sys

import numpy as np
import pytest

from oracle import delay as odelay
from oracle import network

pytestmark = pytest.mark.gpu

F = np.float32
GOLD = os.path.join(os.path.dirname(__file__), 'golden')
sys.path.insert(0, GOLD)
sys.path.insert(0, os.path.dirname(__file__))
import make_golden  # noqa: E402


@pytest.fixture(scope='module')
def bs():
    import torch
    if not torch.cuda.is_available():
        pytest.fail('GPU tests need a ROCm GPU')
    import brainstate_amd
    brainstate_amd.environ.set(dt=0.1)
    return brainstate_amd


def say(*a):
    print('[case]', *a, flush=True)


def _ones(n, v):
    import torch
    return torch.ones(n, device='cuda') * v


def np_(x):
    return x.cpu().numpy()


def test_rotation_delay_reference(bs):
    """_delay_test.py:62-85."""
    say('rotation delay')
    d = bs.nn.Delay(np.ones((1,), F))
    d.register_entry('a', 0.)
    d.register_entry('b', 1.)
    d.register_entry('c2', 1.9)
    d.register_entry('c', 2.)
    d.init_state()
    for i in range(100):
        d.update(_ones(1, i))
        assert np.allclose(np_(d.at('a')), i)
        assert np.allclose(np_(d.at('b')), max(i - 10, 0))
        assert np.allclose(np_(d.at('c')), max(i - 20, 0))
    with pytest.raises(KeyError):
        d.register_entry('c', 10.)


@pytest.mark.parametrize('method,cases', [
    ('round', [(0.01, 0.0), (1.04, 10.0), (1.06, 11.0)]),            # :126-152
    ('linear_interp', [(0.01, 0.1), (1.04, 10.4), (1.06, 10.6)]),    # :154-182
])
@pytest.mark.parametrize('shape', [(1,), (1, 1), (1, 1, 1)])
def test_time_interp_reference(bs, method, cases, shape):
    import torch
    say('time interp', method, shape)
    d = bs.nn.Delay(np.ones(shape, F), time=2., interp_method=method)
    d.init_state()
    for i in range(100):
        t = float(F(i) * F(0.1))
        with bs.environ.context(t=t):
            d.update(torch.ones(shape, device='cuda') * i)
            for td, n in cases:
                got = np_(d.retrieve_at_time(float(F(t - F(td)))))
                assert got.shape == shape
                assert np.allclose(got, max(i - n, 0.0), atol=1e-4), (i, td)


def test_jit_error_check_reference(bs):
    """_delay_test.py:110-124."""
    say('jit error check')
    d = bs.nn.Delay(np.ones((1,), F), time=2., interp_method='round')
    d.init_state()
    with bs.environ.context(t=0, jit_error_check=True):
        d.retrieve_at_time(-2.0)
        with pytest.raises(ValueError):
            d.retrieve_at_time(-2.1)
        d.retrieve_at_time(-2.01)
        with pytest.raises(ValueError):
            d.retrieve_at_time(-2.09)
        with pytest.raises(ValueError):
            d.retrieve_at_time(0.1)


def test_write_ptr_and_update_every_reference(bs):
    """_delay_test.py:275-289, 444-461, 748-800."""
    say('write ptr / update_every')
    d = bs.nn.Delay(np.zeros((1,), F), time=1.0)
    d.init_state()
    for i in range(d.max_length * 2 + 5):
        d.update(_ones(1, i))
        assert d.write_ptr.value == (i + 1) % d.max_length
    d = bs.nn.Delay(np.zeros((5,), F), time=1.0)
    d.init_state(batch_size=4)
    assert d.write_ptr.value.shape == ()
    for i in range(20):
        d.update(np.ones((4, 5), F) * i)
    assert d.write_ptr.value == 20 % d.max_length
    d = bs.nn.Delay(np.zeros((2,), F), time=1.0, update_every=0.5)
    assert d.update_every_step == 5
    d.init_state()
    for i in range(20):
        d.update(_ones(2, i))
    assert int(d.write_ptr.value) == 20 % 15
    d = bs.nn.Delay(np.zeros((1,), F), time=1.0, update_every=0.5, interpolation='round')
    d.init_state()
    for i in range(11):
        d.update(_ones(1, float(i)))
    assert set(np_(d.history.value).ravel().tolist()) == {0.0, 5.0, 10.0}
    with bs.environ.context(t=1.0):
        assert np.allclose(np_(d.retrieve_at_time(1.0)), 10.0)
        assert np.allclose(np_(d.retrieve_at_time(0.5)), 5.0)
    with pytest.raises(ValueError):
        bs.nn.Delay(np.zeros((2,), F), time=1.0, update_every=0.05)
    d.reset_state()
    assert int(d.write_ptr.value) == 0


def test_construction_errors_and_init_reference(bs):
    """_delay_test.py:410-442, 586-653, 676-746."""
    say('construction')
    with pytest.warns(DeprecationWarning):
        bs.nn.Delay(np.zeros((1,), F), time=1.0, delay_method='concat')
    assert bs.nn.Delay(np.zeros((1,), F), time=1.0, interp_method='linear_interp').interp_method \
        == 'linear'
    assert bs.nn.Delay(np.zeros((1,), F), time=1.0, interp_method='round').interp_method == 'nearest'
    with pytest.raises(ValueError):
        bs.nn.Delay(np.zeros((1,), F), time=1.0, interpolation='bogus')
    with pytest.raises(TypeError):
        bs.nn.Delay(np.zeros((1,), F), time=1.0, interpolation=123)
    with pytest.raises(TypeError):
        bs.nn.Delay(np.zeros((2,), F), time=1.0, init='not-valid')
    with pytest.raises(ValueError):
        bs.nn.InterpolationRegistry.get('does_not_exist')
    for name in ['nearest', 'round', 'linear', 'linear_interp', 'cubic', 'hermite',
                 'polynomial2', 'polynomial3']:
        assert name in bs.nn.InterpolationRegistry.list_methods()
    for init, want in ((np.array(5.0, F), 5.0), (3.0, 3.0),
                       (lambda shape, dtype: np.ones(shape, dtype) * 7.0, 7.0)):
        d = bs.nn.Delay(np.zeros((2,), F), time=1.0, init=init)
        d.init_state()
        assert np.allclose(np_(d.history.value[0]), want)
    d = bs.nn.Delay(np.zeros((2,), F), time=2.0, entries={'a': 1.0, 'b': (0.5,)})
    d.register_entry('latest', None)
    d.init_state()
    for i in range(10):
        d.update(_ones(2, i))
    assert np_(d.at('a')).shape == (2,) and np_(d.at('b')).shape == (2,)
    assert np.allclose(np_(d.at('latest')), 9)
    with pytest.raises(KeyError):
        d.at('missing')
    with pytest.raises(AssertionError):
        d.at(123)
    acc = d.access('acc', 1.0)
    assert isinstance(acc, bs.nn.DelayAccess)
    assert np.array_equal(np_(acc()), np_(d.at('acc')))
    with pytest.raises(AssertionError):
        bs.nn.DelayAccess(object(), 1.0, entry='bad')


def test_notebook_worked_values(bs):
    """02_synaptic_delays.ipynb cells 11, 17, 27."""
    say('notebook values')
    d = bs.nn.Delay(np.zeros((1,), F), time=10.0)
    d.init_state()
    for i in range(20):
        d.update(np.array([i * 10.0], F))
    assert [float(np_(d.retrieve_at_step(k))[0]) for k in (0, 5, 10)] == [190.0, 140.0, 90.0]
    d = bs.nn.Delay(np.zeros(3, F), time=10.0)
    a2, a5 = d.access('e2', 2.0), d.access('e5', 5.0)
    d.init_state()
    for i in range(200):
        d.update(np.array([i, 2.0 * i, 3.0 * i], F))
    assert np_(a2()).tolist() == [179, 358, 537] and np_(a5()).tolist() == [149, 298, 447]
    d = bs.nn.Delay(np.zeros(3, F), time=10.0)
    d.register_entry('het', np.array([2.0, 5.0, 8.0]), np.array([0, 1, 2]))
    d.init_state()
    for i in range(200):
        d.update(np.array([i, 10.0 * i, 100.0 * i], F))
    assert np_(d.at('het')).tolist() == [179, 1490, 11900]


@pytest.mark.parametrize('method', ['linear', 'nearest', 'cubic', 'hermite', 'polynomial2',
                                    'polynomial3'])
def test_reads_bit_equal_oracle(bs, method):
    """Random float32 history: step reads, fancy-indexed vector reads and continuous-time
    reads equal the oracle restatement bit for bit."""
    import torch
    say('reads vs oracle', method)
    rs = np.random.RandomState(5)
    shape = (3, 7)
    d = bs.nn.Delay(np.zeros(shape, F), time=2.0, interpolation=method)
    o = odelay.Delay(shape, time=2.0, interpolation=method)
    steps = rs.randint(0, 21, (4, 3))
    col = rs.randint(-7, 7, (4, 3))
    d.register_entry('v', steps.astype(F) * F(0.1) - F(0.01), 1, col)
    o.register_entry('v', steps.astype(F) * F(0.1) - F(0.01), 1, col)
    d.init_state()
    o.init_state()
    for i in range(57):
        x = rs.randn(*shape).astype(F)
        d.update(torch.from_numpy(x).cuda())
        o.update(x)
    assert d.write_ptr.value == o.write_ptr
    for k in (0, 1, 7, 20, 25):
        assert np.array_equal(np_(d.retrieve_at_step(k)), o.retrieve_at_step(k)), k
    assert np.array_equal(np_(d.at('v')), o.at('v'))
    assert np.array_equal(np_(d.retrieve_at_step(np.array([[0, 3], [5, 9]]), 2)),
                          o.retrieve_at_step(np.array([[0, 3], [5, 9]]), 2))
    now = 5.6
    for td in rs.uniform(now - 1.9, now, 30):
        with bs.environ.context(t=now):
            got = np_(d.retrieve_at_time(float(td)))
        assert np.array_equal(got, o.retrieve_at_time(F(td), F(now))), td


def test_state_with_delay_and_prefetch(bs):
    """_delay_test.py:832-888 and the prefetch_delay chain of _dynamics.py:222-262, 655-745."""
    import torch
    say('state with delay')

    class Mod(bs.nn.Dynamics):
        def __init__(self):
            super().__init__(3)
            self.V = bs.State(torch.zeros(3, device='cuda'))
            self.plain = torch.zeros(3)

        def update(self, x):
            self.V.value = self.V.value * 0.9 + x
            return self.V.value

    m = Mod()
    swd = bs.nn.StateWithDelay(m, 'V')
    swd.register_entry('e', 0.5)
    swd.init_state()
    for i in range(3):
        m.V.value = torch.ones(3, device='cuda') * i
        swd.update()
    assert int(swd.write_ptr.value) != 0 and np_(swd.at('e')).shape == (3,)
    swd.reset_state()
    assert int(swd.write_ptr.value) == 0
    assert swd.state is m.V
    with pytest.raises(TypeError):
        _ = bs.nn.StateWithDelay(m, 'plain').state

    m2 = Mod()
    v5 = m2.prefetch_delay('V', 0.5)         # 5 steps
    out2 = m2.output_delay(0.2)              # 2 steps of the update's output
    bs.nn.init_all_states(m2)
    vals = []
    for i in range(12):
        m2(torch.ones(3, device='cuda') * i)
        vals.append(np_(m2.V.value).copy())
        want5 = vals[i - 5] if i >= 5 else np.zeros(3, F)
        want2 = vals[i - 2] if i >= 2 else np.zeros(3, F)
        assert np.array_equal(np_(v5()), want5), i
        assert np.array_equal(np_(out2()), want2), i
    assert np.array_equal(np_(m2.prefetch('V')()), vals[-1])


class _DelayedEINet:
    """The config-[1] E/I net whose projections read N.prefetch_delay('spike', delay)."""

    def __init__(self, bs, delay):
        from test_gpu_api import _EINet
        self.base = _EINet(bs)
        self.sd = self.base.N.prefetch_delay('spike', delay)
        self.sd.state_delay.init_state()

    def update(self, t):
        b = self.base
        with b.bs.environ.context(t=t):
            spk = self.sd()
            b.E(spk[:b.n_exc])
            b.I(spk[b.n_exc:])
            b.N(20.)
            return b.N.get_spike()


@pytest.mark.parametrize('delay,D', [(0.5, 5), (0.12, 2)])
def test_delayed_module_net_eager_and_fused(bs, delay, D):
    """prefetch_delay('spike', delay) -> ceil(delay/dt) steps: eager steps through the module
    API and the fused runner with fuse(delay=...) both give the oracle's delayed raster."""
    import torch
    say('delayed module net', delay, D)
    T = 200
    pe, pi, V0, p = make_golden.config1_net()
    ref = network.run_coba_lif(V0, pe, pi, p, 3200, T, delay_steps=D)
    assert ref['counts'].sum() > 500
    with bs.environ.context(dt=0.1):
        net = _DelayedEINet(bs, delay)
        assert net.sd.delay_info[0] == D
        spikes = bs.transform.for_loop(net.update, torch.arange(T) * 0.1)
        assert np.array_equal(spikes.cpu().numpy(), ref['raster'])
        net2 = _DelayedEINet(bs, delay)
        r = bs.nn.fuse(net2.base.N, net2.base.E, net2.base.I, n_exc=3200, inp=20., delay=delay)
        assert r.delay_steps == D
        raster = torch.zeros(T, 4000, dtype=torch.uint8, device='cuda')
        r.run(T, raster=raster)
        r.check()
    assert np.array_equal(raster.cpu().numpy().astype(bool), ref['raster'])
