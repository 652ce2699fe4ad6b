"""Pins for oracle.delay (the reference Delay restated) and the delayed network oracles.

The expected values are the reference's own (brainstate/nn/_delay_test.py, and the worked
outputs of docs/tutorials/brain_dynamics/02_synaptic_delays.ipynb); the interpolators are
pinned by the polynomials each reproduces exactly; the delayed network by two independent
formulations (spike history read at step D in numpy, a ring of D+1 input slots in C) and by
where the first synaptic input lands.
"""
import numpy as np
import pytest

from oracle import cbuild, delay, network, neuron

F = np.float32


def test_delay_steps_rule():
    assert delay.delay_steps(None, 0.1) == 0
    assert delay.delay_steps(1.0, 0.1) == 10
    assert delay.delay_steps(1.9, 0.1) == 19
    assert delay.delay_steps(2.0, 0.1) == 20
    # float64 ratio 11.000000000000002 rounds to float32 11.0 before the ceil
    assert delay.delay_steps(1.1, 0.1) == 11
    np.testing.assert_array_equal(delay.delay_steps(np.array([2.0, 5.0, 8.0]), 0.1), [20, 50, 80])


def test_rotation_delay_reference():
    """_delay_test.py:62-85."""
    d = delay.Delay((1,))
    d.register_entry('a', 0.)
    d.register_entry('b', 1.)
    d.register_entry('c2', 1.9)
    d.register_entry('c', 2.)
    d.init_state()
    assert d.max_length == 21
    for i in range(100):
        d.update(np.ones(1) * i)
        assert np.allclose(d.at('a'), i)
        assert np.allclose(d.at('b'), max(i - 10, 0))
        assert np.allclose(d.at('c'), max(i - 20, 0))


def test_duplicate_entry_raises():
    """_delay_test.py:34-43."""
    d = delay.Delay((10, 20))
    d.register_entry('a', 1.)
    d.register_entry('c', None)
    with pytest.raises(KeyError):
        d.register_entry('c', 10.)


def test_max_time_monotonic():
    """_delay_test.py:45-60."""
    d = delay.Delay((1,))
    d.register_entry('big', 5.0)
    d.register_entry('small', 1.0)
    assert d.max_time == 5.0
    d = delay.Delay((1,))
    d.register_entry('small', 1.0)
    d.register_entry('big', 7.0)
    assert d.max_time == 7.0


@pytest.mark.parametrize('method,cases', [
    ('round', [(0.01, 0.0), (1.04, 10.0), (1.06, 11.0)]),            # :126-152
    ('linear_interp', [(0.01, 0.1), (1.04, 10.4), (1.06, 10.6)]),    # :154-182
])
def test_time_interp_reference(method, cases):
    d = delay.Delay((1,), time=2., interpolation=method)
    d.init_state()
    for i in range(100):
        t = F(i) * F(0.1)
        d.update(np.ones(1) * i)
        for td, n in cases:
            got = d.retrieve_at_time(F(t - F(td)), t)
            assert np.allclose(got, max(i - n, 0.0), atol=1e-4), (i, td)


def test_write_ptr_reference():
    """_delay_test.py:275-289, 444-461, 508-521."""
    d = delay.Delay((1,), time=1.0)
    d.init_state()
    assert d.write_ptr == 0
    for i in range(d.max_length * 2 + 5):
        d.update(np.ones(1) * i)
        assert d.write_ptr == (i + 1) % d.max_length
    d = delay.Delay((5,), time=1.0)
    d.init_state(batch_size=4)
    for i in range(20):
        d.update(np.ones((4, 5)) * i)
    assert d.write_ptr == 20 % d.max_length and d.history.shape == (11, 4, 5)


def test_update_every_reference():
    """_delay_test.py:748-800."""
    d = delay.Delay((2,), time=1.0, update_every=0.5)
    assert d.every == 5 and d.max_length == 3
    d.init_state()
    for i in range(20):
        d.update(np.ones(2) * i)
    assert d.write_ptr == 20 % 15
    d = delay.Delay((1,), time=1.0, update_every=0.5)
    d.init_state()
    for i in range(11):
        d.update(np.ones(1) * float(i))
    assert set(d.history.ravel().tolist()) == {0.0, 5.0, 10.0}
    d = delay.Delay((1,), time=1.0, update_every=0.5, interpolation='round')
    d.init_state()
    for i in range(11):
        d.update(np.ones(1) * float(i))
    assert np.allclose(d.retrieve_at_time(1.0, 1.0), 10.0)
    assert np.allclose(d.retrieve_at_time(0.5, 1.0), 5.0)


def test_init_and_latest_reference():
    """_delay_test.py:618-636, 676-683."""
    for init in (F(5.0), 3.0, lambda shape, dtype: np.ones(shape, dtype) * 7.0):
        d = delay.Delay((2,), time=1.0, init=init)
        d.init_state()
        want = 7.0 if callable(init) else float(init)
        assert np.allclose(d.history[0], want)
    d = delay.Delay((2,), time=2.0)
    d.register_entry('latest', None)
    d.init_state()
    for i in range(10):
        d.update(np.ones(2) * i)
    assert np.allclose(d.at('latest'), 9)


def test_notebook_worked_values():
    """02_synaptic_delays.ipynb cells 11, 17 and 27 (printed expected values)."""
    d = delay.Delay((1,), time=10.0)
    d.init_state()
    assert d.max_length == 101
    for i in range(20):
        d.update(np.array([i * 10.0]))
    assert [float(d.retrieve_at_step(k)[0]) for k in (0, 5, 10)] == [190.0, 140.0, 90.0]
    d = delay.Delay((3,), time=10.0)
    d.register_entry('e2', 2.0)
    d.register_entry('e5', 5.0)
    d.init_state()
    for i in range(200):
        d.update(np.array([i, 2.0 * i, 3.0 * i]))
    np.testing.assert_array_equal(d.at('e2'), [179, 358, 537])
    np.testing.assert_array_equal(d.at('e5'), [149, 298, 447])
    d = delay.Delay((3,), time=10.0)
    d.register_entry('het', np.array([2.0, 5.0, 8.0]), np.array([0, 1, 2]))
    d.init_state()
    for i in range(200):
        d.update(np.array([i, 10.0 * i, 100.0 * i]))
    np.testing.assert_array_equal(d.at('het'), [179, 1490, 11900])


def test_vector_delay_shapes_reference():
    """_delay_test.py:211-272: fancy indexing with broadcast step / index arrays."""
    rs = np.random.RandomState(0)
    d = delay.Delay((2,))
    d.register_entry('a', rs.uniform(0., 10., (2, 2)), rs.randint(0, 2, (2, 2)))
    d.init_state()
    assert d.at('a').shape == (2, 2)
    d = delay.Delay((2, 2))
    d.register_entry('a', rs.uniform(0., 10., (2, 2)), 1, rs.randint(0, 2, (2, 2)))
    d.init_state()
    assert d.at('a').shape == (2, 2)


@pytest.mark.parametrize('method,degree', [('linear', 1), ('cubic', 1), ('hermite', 1),
                                           ('polynomial2', 2), ('polynomial3', 3)])
def test_interpolators_reproduce_polynomials(method, degree):
    """Each method is exact on polynomials up to its degree (Catmull-Rom and the
    finite-difference Hermite reproduce lines, the Lagrange forms their own degree)."""
    rs = np.random.RandomState(1)
    coef = rs.uniform(-1, 1, degree + 1)
    d = delay.Delay((1,), time=3.0, interpolation=method)
    d.init_state()
    for i in range(40):
        d.update(np.array([np.polyval(coef, i / 10.0)], F))
    now = F(3.9)   # the step-39 write is the newest slot
    for fts in rs.uniform(3.0, 20.0, 25):   # every tap stays behind the write pointer
        step = 39 - fts
        got = d.retrieve_at_time(F(now - F(fts) * F(0.1)), now)[0]
        want = np.polyval(coef, step / 10.0)
        assert abs(float(got) - want) < 2e-5 * max(1.0, abs(want)), (method, fts)


def test_hermite_taps_match_finite_difference_form():
    """The 4-tap weights equal the reference's h00 v0 + h10 m0 + h01 v1 + h11 m1 with
    m0 = (v1 - v_-1)/2, m1 = (v2 - v0)/2 (_delay.py:246-266)."""
    rs = np.random.RandomState(2)
    for t in rs.uniform(0, 1, 20):
        v = rs.randn(4)
        offs, w = delay.tap_weights('hermite', t)
        h00, h10 = 2 * t**3 - 3 * t**2 + 1, t**3 - 2 * t**2 + t
        h01, h11 = -2 * t**3 + 3 * t**2, t**3 - t**2
        ref = h00 * v[1] + h10 * 0.5 * (v[2] - v[0]) + h01 * v[2] + h11 * 0.5 * (v[3] - v[1])
        assert offs == (-1, 0, 1, 2)
        assert abs(float(np.dot(np.asarray(w, np.float64), v)) - ref) < 1e-5


# ---- delayed networks ----

def _net(seed=3):
    n, n_exc = 4000, 3200
    pe = network.Projection(0, n_exc, n, 80, 0.6, seed)
    pi = network.Projection(n_exc, n, n, 80, 6.7, seed + 1)
    V0 = np.random.RandomState(seed + 2).uniform(-60, -50, n).astype(F)
    return n, n_exc, pe, pi, V0, neuron.LIFParams(I_ext=20.0)


@pytest.mark.parametrize('D', [1, 3])
def test_delayed_net_numpy_equals_c_ring(D):
    n, n_exc, pe, pi, V0, p = _net()
    T = 300
    ref = network.run_coba_lif(V0, pe, pi, p, n_exc, T, delay_steps=D)
    st = dict(V=V0.copy(), ge=np.zeros(n, F), gi=np.zeros(n, F), ref=np.zeros(n, np.int32),
              spk=np.zeros(n, np.uint8), in_e=np.zeros((D + 1) * n, F),
              in_i=np.zeros((D + 1) * n, F))
    counts = np.zeros(T, np.int32)
    cbuild.coba_lif_run(st, pe.idx, pi.idx, pe.w_scalar, pi.w_scalar, p, n_exc, 120,
                        nthreads=4, counts=counts[:120], delay=D)
    cbuild.coba_lif_run(st, pe.idx, pi.idx, pe.w_scalar, pi.w_scalar, p, n_exc, T - 120,
                        nthreads=4, counts=counts[120:], delay=D)
    assert ref['counts'].sum() > 1000
    np.testing.assert_array_equal(counts, ref['counts'])
    np.testing.assert_array_equal(st['V'], ref['V'])
    np.testing.assert_array_equal(st['ge'], ref['ge'])
    np.testing.assert_array_equal(st['spk'].astype(bool), ref['spk'])


@pytest.mark.parametrize('D', [0, 2, 5])
def test_first_input_arrives_at_s0_plus_1_plus_D(D):
    """Until the first spikes' inputs arrive the net runs as if uncoupled; they arrive at step
    s0 + 1 + D (s0 = the first step with spikes)."""
    n, n_exc, pe, pi, V0, p = _net()
    T = 60
    free = network.run_coba_lif(V0, network.Projection(0, n_exc, n, 80, 0.0, 3),
                                network.Projection(n_exc, n, n, 80, 0.0, 4), p, n_exc, T)
    s0 = int(np.flatnonzero(free['counts'])[0])
    assert s0 + 1 + 5 < T
    ge = []
    hist = None
    init = None
    for t in range(T):   # one step per call to see g_e after every step
        r = network.run_coba_lif(V0, pe, pi, p, n_exc, 1, init=init, delay_steps=D,
                                 delay_state=hist)
        init, hist = (r['V'], r['ge'], r['gi'], r['ref'], r['spk']), r['delay_state']
        ge.append(r['ge'].copy())
        if t < s0 + 1 + D:
            np.testing.assert_array_equal(r['spk'], free['raster'][t])
    first = min(t for t in range(T) if np.any(ge[t] != 0))
    assert first == s0 + 1 + D
