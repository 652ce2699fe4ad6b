"""Oracle network loops against the golden fixtures and the C restatement (CPU only)."""
import json
import os
import sys

import numpy as np
import pytest

from oracle import cbuild, network, neuron

F = np.float32
GOLD = os.path.join(os.path.dirname(__file__), 'golden')
sys.path.insert(0, GOLD)
import make_golden  # noqa: E402


def test_lif_notebook_kat():
    """docs/tutorials/brain_dynamics/04_building_an_snn.ipynb cell 5: one LIF step."""
    p = neuron.LIFParams(V_rest=-52., V_th=-50., V_reset=-60., tau=10., I_ext=8., dt=0.1)
    z = np.zeros(4, F)
    V, _, _, _, spk = neuron.coba_lif_step(np.full(4, -60., F), z, z, np.zeros(4, np.int32), z, z, p)
    assert np.all(V == F(-59.84079742)) and not spk.any()


def test_refractory_counts_steps_on_dt_grid():
    assert neuron.ref_steps(5.0, 0.1) == 49      # 0 < k*dt < 5 ms -> k = 1..49
    assert neuron.ref_steps(0.0, 0.1) == 0
    assert neuron.ref_steps(0.25, 0.1) == 2


def test_lif_refractory_and_reset():
    p = neuron.LIFParams(I_ext=0.)
    V = np.array([-49.0, -55.0], F)     # first above threshold after one step
    z = np.zeros(2, F)
    ref = np.zeros(2, np.int32)
    V, ge, gi, ref, spk = neuron.coba_lif_step(V, z, z, ref, z, z, p)
    assert spk.tolist() == [True, False] and V[0] == p.V_reset and ref[0] == p.ref_steps
    for _ in range(int(p.ref_steps)):
        V2, ge, gi, ref2, spk = neuron.coba_lif_step(V, ge, gi, ref, z, z, p)
        assert V2[0] == V[0] and not spk[0]
        V, ref = V2, ref2
    assert ref[0] == 0


def test_cuba_membrane_is_the_exact_linear_solution():
    """CUBA (brainpy.state CUBA, examples/400_CUBA_2005_bpu.py:42-58): the current does not
    depend on V, so dV/dt = (V_rest - V + R I) / tau is linear and exp-Euler is its exact
    solution V' = V_inf + (V - V_inf) exp(-dt / tau), V_inf = V_rest + R I, with
    I = I_ext + g_e s_e + g_i s_i (signed weights: g_i < 0 lowers I).  A Jacobian that kept
    a conductance term, or a wrong sign or scale, moves V' by far more than these few ulp."""
    rng = np.random.RandomState(4)
    n = 2000
    p = neuron.LIFParams(V_rest=-49., V_th=-50., V_reset=-60., tau=20., I_ext=20., out='cuba',
                         scale_e=1.0, scale_i=0.5)
    V = rng.uniform(-70, -40, n).astype(F)
    ge = rng.uniform(0, 3, n).astype(F)
    gi = -rng.uniform(0, 5, n).astype(F)
    got = neuron.lif_membrane(V, ge, gi, p).astype(np.float64)
    I = 20.0 + ge.astype(np.float64) * 1.0 + gi.astype(np.float64) * 0.5
    Vinf = -49.0 + I
    exact = Vinf + (V.astype(np.float64) - Vinf) * np.exp(-0.1 / 20.0)
    ulp = np.spacing(np.abs(exact).astype(F)).astype(np.float64)
    assert np.all(np.abs(got - exact) <= 8 * ulp)
    # zero conductances: CUBA and COBA are the same equation, bit for bit
    pc = neuron.LIFParams(V_rest=-49., V_th=-50., V_reset=-60., tau=20., I_ext=20.)
    z = np.zeros(n, F)
    assert np.array_equal(neuron.lif_membrane(V, z, z, p), neuron.lif_membrane(V, z, z, pc))
    # and with conductances they differ (the COBA current depends on V)
    assert not np.allclose(neuron.lif_membrane(V, ge, -gi, pc), got, atol=1e-3)


def test_soft_reset_subtracts_the_threshold_gap():
    """spk_reset='soft' (04_building_an_snn.ipynb cells 5, 11): a spiking neuron keeps its
    overshoot, V = V' - (V_th - V_reset); hard reset sets V_reset; below threshold both are
    the plain membrane step."""
    p_s = neuron.LIFParams(V_rest=-52., V_th=-50., V_reset=-60., tau=10., tau_ref=0.,
                           I_ext=30., out='cuba', spk_reset='soft')
    p_h = neuron.LIFParams(V_rest=-52., V_th=-50., V_reset=-60., tau=10., tau_ref=0.,
                           I_ext=30., out='cuba')
    V = np.array([-50.5, -49.0, -58.0, -45.0], F)
    z = np.zeros(4, F)
    r0 = np.zeros(4, np.int32)
    Vm = neuron.lif_membrane(V, z, z, p_s)
    Vs, _, _, rs, ss = neuron.coba_lif_step(V, z, z, r0, z, z, p_s)
    Vh, _, _, rh, sh = neuron.coba_lif_step(V, z, z, r0, z, z, p_h)
    assert np.array_equal(ss, Vm >= F(-50.)) and np.array_equal(ss, sh) and ss.sum() >= 2
    assert np.array_equal(Vs[ss], (Vm[ss] - F(10.)).astype(F))
    assert np.all(Vh[sh] == F(-60.)) and np.array_equal(Vs[~ss], Vm[~ss])
    assert np.all(rs == 0) and np.all(rh == 0)   # no refractory period (tau_ref = 0)


def test_tutorial_soft_reset_net_matches_golden():
    gold = json.load(open(os.path.join(GOLD, 'tut_lif_soft_500.json')))
    pe, pi, V0, p = make_golden.tut_net()
    res = network.run_coba_lif(V0, pe, pi, p, make_golden.TUT_NET['n_exc'],
                               make_golden.TUT_NET['steps'])
    assert res['counts'].tolist() == gold['counts']
    assert make_golden.sha(res['V']) == gold['final_V_sha256']
    assert 0 < sum(gold['counts'])


def test_hh_matches_float64_equations():
    """examples/100_hh_neuron_model.py:49-86 in float64 (libm exp) vs the fp32 oracle."""
    V = np.linspace(-90, 50, 2001)
    V = V[np.abs(V + 40) > 1e-6]
    V = V[np.abs(V + 55) > 1e-6]
    am = 0.1 * (V + 40) / (1 - np.exp(-(V + 40) / 10))
    bm = 4.0 * np.exp(-(V + 65) / 18)
    ah = 0.07 * np.exp(-(V + 65) / 20)
    bh = 1 / (1 + np.exp(-(V + 35) / 10))
    an = 0.01 * (V + 55) / (1 - np.exp(-(V + 55) / 10))
    bn = 0.125 * np.exp(-(V + 65) / 80)
    got = neuron.hh_rates(V.astype(F))
    for g, e in zip(got, (am, bm, ah, bh, an, bn)):
        np.testing.assert_allclose(g, e, rtol=5e-6)
    # steady state: the gate drifts vanish at x_inf
    m, h, n = neuron.hh_init(V.astype(F))
    for x, a, b in ((m, am, bm), (h, ah, bh), (n, an, bn)):
        assert np.max(np.abs(a * (1 - x) - b * x)) < 1e-5


def test_hh_rate_singular_points():
    # exprel makes the rates finite at V = -40 (m) and V = -55 (n): limits 1.0 and 0.1
    am, _, _, _, an, _ = neuron.hh_rates(np.array([-40.0, -55.0], F))
    assert am[0] == F(1.0) and an[1] == F(0.1)


def test_hh_step_float64_cross_check():
    rng = np.random.RandomState(3)
    n = 500
    V = rng.uniform(-75, -50, n).astype(F)
    m, h, ng = neuron.hh_init(V)
    ge = rng.exponential(0.1, n).astype(F)
    gi = rng.exponential(0.3, n).astype(F)
    p = neuron.HHParams(I_ext=6.5)
    Vn = neuron.hh_step(V, m, h, ng, ge, gi, np.zeros(n, F), np.zeros(n, F), p)[0]
    d = lambda a: a.astype(np.float64)
    ge64, gi64 = d(ge) * float(p.de), d(gi) * float(p.di)
    V64 = d(V)
    I = 6.5 + ge64 * (0 - V64) + gi64 * (-80 - V64)
    gna = 120 * d(m) ** 3 * d(h)
    gk = 36 * d(ng) ** 4
    f = -gna * (V64 - 50) - gk * (V64 + 77) - 0.03 * (V64 + 54.387) + I
    J = -gna - gk - 0.03 - ge64 - gi64
    z = 0.05 * J
    exact = V64 + 0.05 * np.expm1(z) / z * f
    np.testing.assert_allclose(Vn, exact, rtol=2e-5, atol=2e-5)


def test_coba_lif_4000_matches_golden():
    with open(os.path.join(GOLD, 'coba_lif_4000.json')) as f:
        gold = json.load(f)
    pe, pi, V0, p = make_golden.config1_net()
    res = network.run_coba_lif(V0, pe, pi, p, 3200, gold['config']['steps'])
    assert res['counts'].tolist() == gold['counts']
    assert make_golden.sha(np.packbits(res['raster'])) == gold['raster_sha256']
    assert [network.spike_hash(r) for r in res['raster']] == gold['hashes']


def test_coba_hh_2000_matches_golden():
    with open(os.path.join(GOLD, 'coba_hh_2000.json')) as f:
        gold = json.load(f)
    pe, pi, V0, p = make_golden.hh_net()
    res = network.run_coba_hh(V0, pe, pi, p, make_golden.HH_NET['n_exc'], gold['config']['steps'])
    assert res['counts'].tolist() == gold['counts']
    assert make_golden.sha(res['V']) == gold['final_V_sha256']


def test_cuba_lif_4000_matches_golden():
    """examples/400_CUBA_2005_bpu.py's E/I net (CUBA outputs, signed weights), 1000 steps."""
    gold = json.load(open(os.path.join(GOLD, 'cuba_lif_4000.json')))
    pe, pi, V0, p = make_golden.cuba_net()
    res = network.run_coba_lif(V0, pe, pi, p, make_golden.CUBA_NET['n_exc'],
                               make_golden.CUBA_NET['steps'])
    assert res['counts'].tolist() == gold['counts']
    assert make_golden.sha(np.packbits(res['raster'])) == gold['raster_sha256']
    assert make_golden.sha(res['V']) == gold['final_V_sha256']
    assert 0 < sum(gold['counts'])


def test_hh_single_trace_matches_golden():
    """examples/100_hh_neuron_model.py's neuron over 10,000 steps of random input."""
    gold = json.load(open(os.path.join(GOLD, 'hh_single_trace.json')))
    _, trace, spikes = make_golden.hh_single_trace()
    assert make_golden.sha(trace) == gold['trace_sha256'] and spikes == gold['spikes']
    assert len(spikes) > 0


@pytest.mark.parametrize('nthreads', [1, 4])
def test_c_restatement_equals_numpy_oracle(nthreads):
    with open(os.path.join(GOLD, 'coba_lif_4000.json')) as f:
        gold = json.load(f)
    pe, pi, V0, p = make_golden.config1_net()
    n = V0.size
    st = dict(V=V0.copy(), ge=np.zeros(n, F), gi=np.zeros(n, F), ref=np.zeros(n, np.int32),
              spk=np.zeros(n, np.uint8), in_e=np.zeros(n, F), in_i=np.zeros(n, F))
    T = gold['config']['steps']
    counts = np.zeros(T, np.int32)
    hashes = np.zeros(T, np.uint32)
    cbuild.coba_lif_run(st, pe.idx, pi.idx, pe.w_scalar, pi.w_scalar, p, 3200, T,
                        nthreads=nthreads, counts=counts, hashes=hashes)
    assert counts.tolist() == gold['counts']
    assert hashes.tolist() == gold['hashes']
    assert make_golden.sha(st['V']) == gold['final_V_sha256']


def test_spike_hash_matches_mix32_definition():
    spk = np.zeros(100, bool)
    spk[[3, 50]] = True
    def mix(x):
        x &= 0xFFFFFFFF
        x ^= x >> 16
        x = (x * 0x85EBCA6B) & 0xFFFFFFFF
        x ^= x >> 13
        x = (x * 0xC2B2AE35) & 0xFFFFFFFF
        x ^= x >> 16
        return x
    assert network.spike_hash(spk) == (mix(3) + mix(50)) & 0xFFFFFFFF
