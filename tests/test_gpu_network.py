"""GPU parity of the persistent whole-loop runners against the oracle network loops."""
import json
import os
import sys

import numpy as np
import pytest

from oracle import network, neuron

pytestmark = pytest.mark.gpu

F = np.float32
GOLD = os.path.join(os.path.dirname(__file__), 'golden')
sys.path.insert(0, GOLD)
import make_golden  # noqa: E402


@pytest.fixture(scope='module')
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail('GPU tests need a ROCm GPU')
    return torch


def say(*a):
    print('[case]', *a, flush=True)


def _lif_runner(torch, het, blocks_per_cu=0, delay_steps=0):
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    pe, pi, V0, _ = make_golden.config1_net()
    c = make_golden.CONFIG1
    return EINetRunner('lif', c['n'], c['n_exc'], pe.idx, pi.idx,
                       np.full(pe.idx.shape, F(c['w_e'])) if het else c['w_e'],
                       np.full(pi.idx.shape, F(c['w_i'])) if het else c['w_i'],
                       ops.lif_params(), V0, blocks_per_cu=blocks_per_cu,
                       delay_steps=delay_steps)


def _c_lif(idx_e, idx_i, w_e, w_i, p, n_exc, V0, T, D, nthreads=8):
    """C restatement with a D-step synaptic delay: per-step counts, hashes, final state."""
    from oracle import cbuild
    st = cbuild.lif_state(V0, delay=D)
    c = np.zeros(T, np.int32)
    h = np.zeros(T, np.uint32)
    cbuild.coba_lif_run(st, idx_e, idx_i, w_e, w_i, p, n_exc, T, nthreads=nthreads, counts=c,
                        hashes=h, delay=D)
    return c, h, st


def _c_hh(idx_e, idx_i, w_e, w_i, p, n_exc, V0, T, D=0, nthreads=16):
    from oracle import cbuild
    st = cbuild.hh_state(V0, delay=D)
    c = np.zeros(T, np.int32)
    h = np.zeros(T, np.uint32)
    cbuild.coba_hh_run(st, idx_e, idx_i, w_e, w_i, p, n_exc, T, nthreads=nthreads, counts=c,
                       hashes=h, delay=D)
    return c, h, st


def _host_threads():
    import os
    return max(1, min(16, len(os.sched_getaffinity(0))))


def _big_net(n, k, seed, weights):
    """Config [3]-shaped net: 80 % E, K fixed-num targets per neuron (numpy MT19937), V0 ~
    U(-60, -50).  weights: 'homo' (0.6 / 6.7), 'const' (0.6 / 6.7 stored per synapse, as
    bench.py) or 'normal' (N(0.6, 0.06) / N(6.7, 0.67) per synapse)."""
    n_exc = n * 4 // 5
    idx_e = np.random.RandomState(seed + 1).randint(0, n, size=(n_exc, k)).astype(np.int32)
    idx_i = np.random.RandomState(seed + 2).randint(0, n, size=(n - n_exc, k)).astype(np.int32)
    V0 = np.random.RandomState(seed + 3).uniform(-60., -50., n).astype(F)
    if weights == 'homo':
        w_e, w_i = 0.6, 6.7
    elif weights == 'const':
        w_e, w_i = np.full(idx_e.shape, F(0.6)), np.full(idx_i.shape, F(6.7))
    else:
        w_e = np.random.RandomState(seed + 4).normal(0.6, 0.06, idx_e.shape).astype(F)
        w_i = np.random.RandomState(seed + 5).normal(6.7, 0.67, idx_i.shape).astype(F)
    return n_exc, idx_e, idx_i, w_e, w_i, V0


def _run_chunks(torch, r, T, chunks):
    counts = torch.zeros(T, dtype=torch.int32, device='cuda')
    hashes = torch.zeros(T, dtype=torch.int32, device='cuda')
    t0 = 0
    for c in chunks:
        r.run(c, counts=counts[t0:t0 + c], hashes=hashes[t0:t0 + c])
        t0 += c
    r.check()
    return counts.cpu().numpy(), np.array([int(x) & 0xFFFFFFFF for x in hashes.cpu().numpy()],
                                          np.uint32)


@pytest.mark.parametrize('D,chunks', [(1, [1000]), (4, [300, 700]), (37, [1, 38, 961])])
def test_coba_lif_delay_matches_c_ring(torch_cuda, D, chunks):
    """Synaptic delay of D steps (inputs of step t from the spikes of step t-1-D): per-step
    counts and hashes, final V and spikes equal the C restatement's, across split runs."""
    torch = torch_cuda
    say('coba lif 4000 delay', D, chunks)
    pe, pi, V0, p = make_golden.config1_net()
    T = sum(chunks)
    c_ref, h_ref, st = _c_lif(pe.idx, pi.idx, pe.w_scalar, pi.w_scalar, p, 3200, V0, T, D)
    r = _lif_runner(torch, False, delay_steps=D)
    counts, hashes = _run_chunks(torch, r, T, chunks)
    assert c_ref.sum() > 1000
    assert counts.tolist() == c_ref.tolist()
    assert hashes.tolist() == h_ref.tolist()
    assert np.array_equal(r.state['V'].cpu().numpy(), st['V'])
    assert np.array_equal(r.spk.cpu().numpy(), st['spk'])


def test_coba_lif_delay_large_grid(torch_cuda):
    """262,144 neurons (256 workgroups, K = 100, as the 1M net per neuron): the ring of
    2(D+1) inbox slots under real cross-workgroup skew; counts, hashes and final V equal the
    C restatement's."""
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    from oracle import neuron
    torch = torch_cuda
    n, D, T = 262144, 3, 3000
    n_exc = n * 4 // 5
    say('coba lif delay large grid', n, D, T)
    idx_e = np.random.RandomState(101).randint(0, n, size=(n_exc, 100)).astype(np.int32)
    idx_i = np.random.RandomState(102).randint(0, n, size=(n - n_exc, 100)).astype(np.int32)
    V0 = np.random.RandomState(103).uniform(-60., -50., n).astype(F)
    c_ref, h_ref, st = _c_lif(idx_e, idx_i, F(0.6), F(6.7), neuron.LIFParams(), n_exc, V0, T, D,
                              nthreads=16)
    r = EINetRunner('lif', n, n_exc, idx_e, idx_i, 0.6, 6.7, ops.lif_params(), V0,
                    delay_steps=D)
    assert r.grid_blocks == 256
    counts, hashes = _run_chunks(torch, r, T, [T])
    assert c_ref.sum() > 10 * T
    assert counts.tolist() == c_ref.tolist()
    assert hashes.tolist() == h_ref.tolist()
    assert np.array_equal(r.state['V'].cpu().numpy(), st['V'])


def test_coba_hh_delay_matches_oracle(torch_cuda):
    """HH net with a 5-step synaptic delay against the numpy oracle's spike-history Delay."""
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    torch = torch_cuda
    c = make_golden.HH_NET
    D, T = 5, 600
    say('coba hh delay', D, T)
    pe, pi, V0, p = make_golden.hh_net()
    ref = network.run_coba_hh(V0, pe, pi, p, c['n_exc'], T, record_raster=False, delay_steps=D)
    r = EINetRunner('hh', c['n'], c['n_exc'], pe.idx, pi.idx, c['w_e'], c['w_i'],
                    ops.hh_params(I_ext=c['I_ext']), V0, delay_steps=D)
    counts, _ = _run_chunks(torch, r, T, [200, 400])
    assert ref['counts'].sum() > 100
    assert counts.tolist() == ref['counts'].tolist()
    assert np.array_equal(r.state['V'].cpu().numpy(), ref['V'])


@pytest.mark.parametrize('n,steps,weights,D', [
    (1_000_000, 1000, 'normal', 0),   # the bench's instantiation: 4 neurons per thread
    (1_000_000, 1000, 'const', 0),    # the bench's own weights
    (1_000_000, 600, 'homo', 0),      # event counts at the same instantiation
    (400_000, 1000, 'normal', 0),     # 2 neurons per thread
    (1_500_000, 600, 'normal', 0),    # 8 neurons per thread
    (1_000_000, 600, 'normal', 2),    # ring of inbox slots at the bench's instantiation
])
def test_coba_lif_large_matches_c(torch_cuda, n, steps, weights, D):
    """Config [3]-shaped nets (K = 100) at every neurons-per-thread instantiation of the
    persistent runner, including the one bench.py times: per-step spike counts and hashes, and
    the final V, g_e, g_i and refractory counters equal the C restatement's (same integer input
    sums, any thread schedule)."""
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    from oracle import neuron
    torch = torch_cuda
    say('coba lif large', n, steps, weights, D)
    n_exc, idx_e, idx_i, w_e, w_i, V0 = _big_net(n, 100, 100, weights)
    r = EINetRunner('lif', n, n_exc, idx_e, idx_i, w_e, w_i, ops.lif_params(), V0,
                    delay_steps=D)
    nb = r.grid_blocks
    npt = -(-n // (nb * 1024))
    assert {400_000: 2, 1_000_000: 4, 1_500_000: 8}[n] == 1 << (npt - 1).bit_length()
    counts, hashes = _run_chunks(torch, r, steps, [steps // 3, steps - steps // 3])
    say('  gpu done, running the C restatement on', _host_threads(), 'threads')
    c_ref, h_ref, st = _c_lif(idx_e, idx_i, w_e, w_i, neuron.LIFParams(), n_exc, V0, steps, D,
                              nthreads=_host_threads())
    assert c_ref.sum() > steps * n // 2000   # > 0.05 % of the neurons fire per step
    assert counts.tolist() == c_ref.tolist()
    assert hashes.tolist() == h_ref.tolist()
    for key in ('V', 'ge', 'gi', 'ref'):
        assert np.array_equal(r.state[key].cpu().numpy(), st[key]), key
    assert np.array_equal(r.spk.cpu().numpy(), st['spk'])


@pytest.mark.parametrize('model', ['lif', 'hh'])
def test_runner_per_neuron_input_matches_c(torch_cuda, model):
    """One external input per neuron (bs_net.I_ext) at the bench's instantiation (1M neurons,
    4 per thread, per-synapse weights): counts, hashes and final state equal the C
    restatement given the same array."""
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    from oracle import neuron
    torch = torch_cuda
    n, T = 1_000_000, 300
    say('runner per-neuron input', model, n, T)
    rs = np.random.RandomState(11)
    if model == 'lif':
        n_exc, idx_e, idx_i, w_e, w_i, V0 = _big_net(n, 100, 100, 'normal')
        I = rs.uniform(15., 25., n).astype(F)
        r = EINetRunner('lif', n, n_exc, idx_e, idx_i, w_e, w_i, ops.lif_params(I_ext=0.), V0,
                        I_ext=I)
    else:
        n_exc, idx_e, idx_i, w_e, w_i, V0 = _big_net(n, 80, 101, 'homo')
        w_e, w_i = 0.05, 0.3
        V0 = rs.uniform(-70., -50., n).astype(F)
        I = rs.uniform(0., 13., n).astype(F)
        r = EINetRunner('hh', n, n_exc, idx_e, idx_i, w_e, w_i, ops.hh_params(I_ext=0.), V0,
                        I_ext=I)
    counts, hashes = _run_chunks(torch, r, T, [T // 3, T - T // 3])
    say('  gpu done, running the C restatement on', _host_threads(), 'threads')
    if model == 'lif':
        from oracle import cbuild
        st = cbuild.lif_state(V0)
        st['I_ext'] = I
        c_ref = np.zeros(T, np.int32)
        h_ref = np.zeros(T, np.uint32)
        cbuild.coba_lif_run(st, idx_e, idx_i, w_e, w_i, neuron.LIFParams(I_ext=0.), n_exc, T,
                            nthreads=_host_threads(), counts=c_ref, hashes=h_ref)
        keys = ('V', 'ge', 'gi', 'ref')
    else:
        from oracle import cbuild
        st = cbuild.hh_state(V0)
        st['I_ext'] = I
        c_ref = np.zeros(T, np.int32)
        h_ref = np.zeros(T, np.uint32)
        cbuild.coba_hh_run(st, idx_e, idx_i, w_e, w_i, neuron.HHParams(I_ext=0.), n_exc, T,
                           nthreads=_host_threads(), counts=c_ref, hashes=h_ref)
        keys = ('V', 'm', 'h', 'n', 'ge', 'gi')
    assert c_ref.sum() > T * n // 5000
    assert counts.tolist() == c_ref.tolist()
    assert hashes.tolist() == h_ref.tolist()
    for key in keys:
        assert np.array_equal(r.state[key].cpu().numpy(), st[key]), key


@pytest.mark.parametrize('weights', ['const', 'normal'])
def test_coba_hh_1m_matches_c(torch_cuda, weights):
    """Config [5]: 1M COBA-HH neurons, K = 80 (4 neurons per thread), bench.py's drive (I_ext
    6.5, V0 ~ U(-70, -50), weights 0.05 / 0.3 or N(0.05, 0.005) / N(0.3, 0.03) per synapse):
    counts, hashes and the final V, m, h, n equal the C restatement's over 300 steps."""
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    from oracle import neuron
    torch = torch_cuda
    n, k, T = 1_000_000, 80, 300
    say('coba hh 1m', weights, T)
    n_exc = n * 4 // 5
    idx_e = np.random.RandomState(201).randint(0, n, size=(n_exc, k)).astype(np.int32)
    idx_i = np.random.RandomState(202).randint(0, n, size=(n - n_exc, k)).astype(np.int32)
    V0 = np.random.RandomState(203).uniform(-70., -50., n).astype(F)
    if weights == 'const':
        w_e, w_i = np.full(idx_e.shape, F(0.05)), np.full(idx_i.shape, F(0.3))
    else:
        w_e = np.random.RandomState(204).normal(0.05, 0.005, idx_e.shape).astype(F)
        w_i = np.random.RandomState(205).normal(0.3, 0.03, idx_i.shape).astype(F)
    r = EINetRunner('hh', n, n_exc, idx_e, idx_i, w_e, w_i, ops.hh_params(I_ext=6.5), V0)
    counts, hashes = _run_chunks(torch, r, T, [T])
    say('  gpu done, running the C restatement on', _host_threads(), 'threads')
    c_ref, h_ref, st = _c_hh(idx_e, idx_i, w_e, w_i, neuron.HHParams(I_ext=6.5), n_exc, V0, T,
                             nthreads=_host_threads())
    assert c_ref.sum() > 1000
    assert counts.tolist() == c_ref.tolist()
    assert hashes.tolist() == h_ref.tolist()
    for key in ('V', 'm', 'h', 'n', 'ge', 'gi'):
        assert np.array_equal(r.state[key].cpu().numpy(), st[key]), key


@pytest.mark.parametrize('chunks', [[1000], [1, 9, 90, 900]])
def test_coba_lif_4000_het_golden(torch_cuda, chunks):
    """Config [1] with random per-synapse weights N(0.6, 0.06) / N(6.7, 0.67): raster, counts,
    hashes and final V equal the oracle's golden run of the runner's fixed-point sums."""
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    torch = torch_cuda
    say('coba lif 4000 het', chunks)
    with open(os.path.join(GOLD, 'coba_lif_4000_het.json')) as f:
        gold = json.load(f)
    pe, pi, V0, _ = make_golden.config1_het_net()
    c = make_golden.CONFIG1_HET
    r = EINetRunner('lif', c['n'], c['n_exc'], pe.idx, pi.idx, pe.w, pi.w, ops.lif_params(), V0)
    T, n = c['steps'], c['n']
    raster = torch.zeros(T, n, dtype=torch.uint8, device='cuda')
    counts = torch.zeros(T, dtype=torch.int32, device='cuda')
    hashes = torch.zeros(T, dtype=torch.int32, device='cuda')
    t0 = 0
    for ch in chunks:
        r.run(ch, counts=counts[t0:t0 + ch], hashes=hashes[t0:t0 + ch], raster=raster[t0:t0 + ch])
        t0 += ch
    r.check()
    assert counts.cpu().numpy().tolist() == gold['counts']
    assert [int(h) & 0xFFFFFFFF for h in hashes.cpu().numpy()] == gold['hashes']
    assert make_golden.sha(np.packbits(raster.cpu().numpy().astype(bool))) == gold['raster_sha256']
    assert make_golden.sha(r.state['V'].cpu().numpy()) == gold['final_V_sha256']


@pytest.mark.parametrize('D', [1, 5])
def test_coba_lif_het_delay_matches_oracle(torch_cuda, D):
    """Random per-synapse weights with a synaptic delay: the numpy oracle's spike-history
    Delay with fixed-point sums, split runs."""
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    torch = torch_cuda
    say('coba lif het delay', D)
    pe, pi, V0, p = make_golden.config1_het_net()
    T = 400
    ref = network.run_coba_lif(V0, pe, pi, p, 3200, T, record_raster=False, delay_steps=D)
    r = EINetRunner('lif', 4000, 3200, pe.idx, pi.idx, pe.w, pi.w, ops.lif_params(), V0,
                    delay_steps=D)
    counts, _ = _run_chunks(torch, r, T, [D, T - D])
    assert ref['counts'].sum() > 500
    assert counts.tolist() == ref['counts'].tolist()
    assert np.array_equal(r.state['V'].cpu().numpy(), ref['V'])


def test_runner_rejects_non_finite_weights(torch_cuda):
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    idx_e = np.zeros((8, 4), np.int32)
    w = np.ones((8, 4), F)
    w[3, 1] = np.nan
    with pytest.raises(ValueError):
        EINetRunner('lif', 10, 8, idx_e, np.zeros((2, 4), np.int32), w, np.ones((2, 4), F),
                    ops.lif_params(), np.zeros(10, F))


@pytest.mark.parametrize('het,chunks', [(False, [1000]), (False, [1, 9, 90, 900])])
def test_coba_lif_4000_raster_bit_exact(torch_cuda, het, chunks):
    """Config [1]: 4000-neuron COBA net, 1000 steps; raster equal to the oracle's."""
    torch = torch_cuda
    say('coba lif 4000', het, chunks)
    with open(os.path.join(GOLD, 'coba_lif_4000.json')) as f:
        gold = json.load(f)
    r = _lif_runner(torch, het)
    T, n = make_golden.CONFIG1['steps'], make_golden.CONFIG1['n']
    raster = torch.zeros(T, n, dtype=torch.uint8, device='cuda')
    counts = torch.zeros(T, dtype=torch.int32, device='cuda')
    hashes = torch.zeros(T, dtype=torch.int32, device='cuda')
    t0 = 0
    for c in chunks:
        r.run(c, counts=counts[t0:t0 + c], hashes=hashes[t0:t0 + c], raster=raster[t0:t0 + c])
        t0 += c
    r.check()
    ras = raster.cpu().numpy().astype(bool)
    assert counts.cpu().numpy().tolist() == gold['counts']
    assert [int(h) & 0xFFFFFFFF for h in hashes.cpu().numpy()] == gold['hashes']
    assert make_golden.sha(np.packbits(ras)) == gold['raster_sha256']
    assert make_golden.sha(r.state['V'].cpu().numpy()) == gold['final_V_sha256']



@pytest.mark.parametrize('het', [False, True])
def test_cuba_lif_4000_raster_bit_exact(torch_cuda, het):
    """examples/400_CUBA_2005_bpu.py's net (CUBA outputs, signed weights) in the persistent
    runner: raster, counts and final V equal the oracle's golden run (one weight per
    projection), or the oracle's run of the fixed-point sums of the same weights stored per
    synapse (the negative I weights exercise the signed I field)."""
    torch = torch_cuda
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    say('cuba lif 4000', het)
    with open(os.path.join(GOLD, 'cuba_lif_4000.json')) as f:
        gold = json.load(f)
    c = make_golden.CUBA_NET
    pe, pi, V0, _ = make_golden.cuba_net()
    p = ops.lif_params(V_rest=c['V_rest'], V_th=c['V_th'], V_reset=c['V_reset'], tau=c['tau'],
                       tau_ref=c['tau_ref'], I_ext=c['I_ext'], out='cuba')
    r = EINetRunner('lif', c['n'], c['n_exc'], pe.idx, pi.idx,
                    np.full(pe.idx.shape, F(c['w_e'])) if het else c['w_e'],
                    np.full(pi.idx.shape, F(c['w_i'])) if het else c['w_i'], p, V0)
    T = c['steps']
    if het:
        ope = network.Projection(0, c['n_exc'], c['n'], c['p'], np.full(pe.idx.shape, F(c['w_e'])),
                                 seed=c['seed_e'], fixed=True)
        opi = network.Projection(c['n_exc'], c['n'], c['n'], c['p'],
                                 np.full(pi.idx.shape, F(c['w_i'])), seed=c['seed_i'], fixed=True)
        res = network.run_coba_lif(V0, ope, opi, make_golden.cuba_net()[3], c['n_exc'], T)
        gold = make_golden.run_records(res)
        assert opi.S is not None and res['counts'].sum() > 1000
    raster = torch.zeros(T, c['n'], dtype=torch.uint8, device='cuda')
    counts = torch.zeros(T, dtype=torch.int32, device='cuda')
    r.run(T, counts=counts, raster=raster)
    r.check()
    assert counts.cpu().numpy().tolist() == gold['counts']
    assert make_golden.sha(np.packbits(raster.cpu().numpy().astype(bool))) == gold['raster_sha256']
    assert make_golden.sha(r.state['V'].cpu().numpy()) == gold['final_V_sha256']


def test_tutorial_soft_reset_net_in_runner(torch_cuda):
    """04_building_an_snn.ipynb's E/I net (LIF without refractory period, soft reset, CUBA)
    in the persistent runner: counts and final V equal the oracle's golden run."""
    torch = torch_cuda
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    say('tutorial soft-reset net')
    with open(os.path.join(GOLD, 'tut_lif_soft_500.json')) as f:
        gold = json.load(f)
    c = make_golden.TUT_NET
    pe, pi, V0, _ = make_golden.tut_net()
    p = ops.lif_params(V_rest=c['V_rest'], V_th=c['V_th'], V_reset=c['V_reset'], tau=c['tau'],
                       tau_ref=0., tau_e=c['tau_e'], tau_i=c['tau_i'], I_ext=c['I_ext'],
                       out='cuba', spk_reset='soft')
    r = EINetRunner('lif', c['n'], c['n_exc'], pe.idx, pi.idx, c['w_e'], c['w_i'], p, V0)
    counts = torch.zeros(c['steps'], dtype=torch.int32, device='cuda')
    r.run(c['steps'], counts=counts)
    r.check()
    assert counts.cpu().numpy().tolist() == gold['counts']
    assert make_golden.sha(r.state['V'].cpu().numpy()) == gold['final_V_sha256']


def test_coba_lif_state_matches_oracle_midway(torch_cuda):
    torch = torch_cuda
    say('coba lif state')
    pe, pi, V0, p = make_golden.config1_net()
    res = network.run_coba_lif(V0, pe, pi, p, 3200, 137, record_raster=False)
    r = _lif_runner(torch, False)
    r.run(137)
    r.check()
    for k in ('V', 'ge', 'gi', 'ref'):
        assert np.array_equal(r.state[k].cpu().numpy(), res[k]), k
    assert np.array_equal(r.spk.cpu().numpy().astype(bool), res['spk'])


def test_coba_lif_long_run_across_launches(torch_cuda):
    """17000 steps: more than one cooperative launch (16384 steps each).  Per-step counts and
    spike hashes and the final state equal the C restatement's; the raster of one
    17000-step call equals that of a 1000 + 16000 split on a second runner."""
    from oracle import cbuild
    torch = torch_cuda
    say('coba lif 4000 long run', 17000)
    pe, pi, V0, p = make_golden.config1_net()
    n, T = V0.size, 17000
    st = dict(V=V0.copy(), ge=np.zeros(n, F), gi=np.zeros(n, F), ref=np.zeros(n, np.int32),
              spk=np.zeros(n, np.uint8), in_e=np.zeros(n, F), in_i=np.zeros(n, F))
    c_ref = np.zeros(T, np.int32)
    h_ref = np.zeros(T, np.uint32)
    cbuild.coba_lif_run(st, pe.idx, pi.idx, pe.w_scalar, pi.w_scalar, p, 3200, T, nthreads=4,
                        counts=c_ref, hashes=h_ref)
    r1 = _lif_runner(torch, False)
    r2 = _lif_runner(torch, False)
    ras1 = torch.zeros(T, n, dtype=torch.uint8, device='cuda')
    ras2 = torch.zeros(T, n, dtype=torch.uint8, device='cuda')
    counts = torch.zeros(T, dtype=torch.int32, device='cuda')
    hashes = torch.zeros(T, dtype=torch.int32, device='cuda')
    r1.run(T, counts=counts, hashes=hashes, raster=ras1)
    r2.run(1000, raster=ras2[:1000])
    r2.run(16000, raster=ras2[1000:])
    r1.check()
    r2.check()
    assert counts.cpu().numpy().tolist() == c_ref.tolist()
    assert [int(h) & 0xFFFFFFFF for h in hashes.cpu().numpy()] == h_ref.tolist()
    assert np.array_equal(r1.state['V'].cpu().numpy(), st['V'])
    assert torch.equal(ras1, ras2)
    assert int(ras1.sum().item()) == int(c_ref.sum())


@pytest.mark.parametrize('het,D', [(True, 0), (False, 4)])
def test_runner_rerun_and_reseed_on_one_workspace(torch_cuda, het, D):
    """Count words carry the step they belong to, so what an earlier run left on the
    workspace is never taken for a later run's.  On one runner: a rerun from step 0 repeats
    the first run bit for bit; for delay 0, a run seeded mid-way from another runner's state
    repeats that runner's remaining steps."""
    torch = torch_cuda
    say('rerun / reseed', het, D)
    T = 300
    r = _lif_runner(torch, het, delay_steps=D)
    init = {k: v.clone() for k, v in r.state.items()}

    def go(runner, steps):
        c = torch.zeros(steps, dtype=torch.int32, device='cuda')
        h = torch.zeros(steps, dtype=torch.int32, device='cuda')
        runner.run(steps, counts=c, hashes=h)
        runner.check()
        return c.cpu().numpy(), h.cpu().numpy()

    c1, h1 = go(r, T)
    V1 = r.state['V'].cpu().numpy()
    assert c1.sum() > 1000
    for k, v in init.items():
        r.state[k].copy_(v)
    r.spk.zero_()
    r.t = 0
    c2, h2 = go(r, T)
    assert np.array_equal(c1, c2) and np.array_equal(h1, h2)
    assert np.array_equal(r.state['V'].cpu().numpy(), V1)
    if D:
        return
    r2 = _lif_runner(torch, het)
    go(r2, 150)
    mid = {k: v.clone() for k, v in r2.state.items()}
    spk_mid = r2.spk.clone()
    c_ref, h_ref = go(r2, T - 150)
    for k, v in mid.items():  # r's workspace still holds the end of its own run
        r.state[k].copy_(v)
    r.seed(spk_mid, t0=150)
    c3, h3 = go(r, T - 150)
    assert np.array_equal(c3, c_ref) and np.array_equal(h3, h_ref)
    assert np.array_equal(c_ref, c1[150:])
    assert np.array_equal(r.state['V'].cpu().numpy(), r2.state['V'].cpu().numpy())


def test_coba_hh_2000_raster_bit_exact(torch_cuda):
    torch = torch_cuda
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    say('coba hh 2000')
    with open(os.path.join(GOLD, 'coba_hh_2000.json')) as f:
        gold = json.load(f)
    c = make_golden.HH_NET
    pe, pi, V0, _ = make_golden.hh_net()
    r = EINetRunner('hh', c['n'], c['n_exc'], pe.idx, pi.idx, c['w_e'], c['w_i'],
                    ops.hh_params(I_ext=c['I_ext']), V0)
    T = c['steps']
    raster = torch.zeros(T, c['n'], dtype=torch.uint8, device='cuda')
    counts = torch.zeros(T, dtype=torch.int32, device='cuda')
    r.run(T, counts=counts, raster=raster)
    r.check()
    assert counts.cpu().numpy().tolist() == gold['counts']
    assert make_golden.sha(np.packbits(raster.cpu().numpy().astype(bool))) == gold['raster_sha256']
    assert make_golden.sha(r.state['V'].cpu().numpy()) == gold['final_V_sha256']


def test_runner_rejects_bad_connectivity(torch_cuda):
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    idx = np.zeros((8, 4), np.int32)
    idx[0, 0] = 10
    with pytest.raises(ValueError):
        EINetRunner('lif', 10, 8, idx, np.zeros((2, 4), np.int32), 0.5, 1.0, ops.lif_params(),
                    np.zeros(10, F))


@pytest.mark.parametrize('soft,cuba,het,chunks', [
    (False, False, True, [1, 7, 192]),   # split runs: each starts from the deferred state
    (True, False, False, [200]),
    (False, True, True, [50, 150]),
    (True, True, False, [2, 198])])
def test_runner_deferred_reset_matches_c(torch_cuda, soft, cuba, het, chunks):
    """deferred_reset in the persistent runner: the state handed between runs keeps the
    crossed V of the last step's spiking neurons (reset at the start of the next run with the
    update's arithmetic; restored after a run from V before its last step).  Counts, hashes
    and final V, g and ref equal the C restatement's deferred steps at 4,000 neurons, hard
    and soft reset, COBA and CUBA, per-synapse and homogeneous weights, over split runs; the
    rasters equal those without deferral."""
    torch = torch_cuda
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    from oracle import neuron
    say('runner deferred reset', soft, cuba, het, chunks)
    T = sum(chunks)
    pe, pi, V0, _ = make_golden.config1_net()
    c = make_golden.CONFIG1
    if het:
        w_e, w_i = make_golden.config1_het_weights(pe.idx.shape, pi.idx.shape)
    else:
        w_e, w_i = c['w_e'], c['w_i']
    kw = dict(spk_reset='soft' if soft else 'hard')
    if cuba:
        kw.update(out='cuba', I_ext=14.)
    p_on = neuron.LIFParams(deferred_reset=True, **kw)
    c_on, h_on, st = _c_lif(pe.idx, pi.idx, F(w_e) if not het else w_e,
                            F(w_i) if not het else w_i, p_on, c['n_exc'], V0, T, 0)
    c_off, h_off, st_off = _c_lif(pe.idx, pi.idx, F(w_e) if not het else w_e,
                                  F(w_i) if not het else w_i, neuron.LIFParams(**kw),
                                  c['n_exc'], V0, T, 0)
    assert np.array_equal(c_on, c_off) and np.array_equal(h_on, h_off)
    assert int(c_on[-1]) > 0 and not np.array_equal(st['V'], st_off['V'])
    ok = dict(spk_reset=kw['spk_reset'], deferred_reset=True)
    if cuba:
        ok.update(out='cuba', I_ext=14.)
    r = EINetRunner('lif', c['n'], c['n_exc'], pe.idx, pi.idx, w_e, w_i,
                    ops.lif_params(**ok), V0)
    counts, hashes = _run_chunks(torch, r, T, chunks)
    assert np.array_equal(counts, c_on) and np.array_equal(hashes, h_on)
    assert np.array_equal(r.state['V'].cpu().numpy(), st['V'])
    assert np.array_equal(r.state['ge'].cpu().numpy(), st['ge'])
    assert np.array_equal(r.state['ref'].cpu().numpy(), st['ref'])
    assert np.array_equal(r.spk.cpu().numpy(), st['spk'])


def test_config3_full_length_matches_c(torch_cuda):
    """Config [3] for its whole run: 1M LIF neurons, K = 100, per-synapse weights
    N(0.6, 0.06) / N(6.7, 0.67), 10,000 steps in the bench's instantiation (4 neurons per
    thread), split over two runs: every step's spike count and hash and the final V, g_e, g_i,
    refractory counters and spikes equal the C restatement's."""
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    from oracle import neuron
    torch = torch_cuda
    n, T = 1_000_000, 10_000
    say('config [3] full length', n, T)
    n_exc, idx_e, idx_i, w_e, w_i, V0 = _big_net(n, 100, 300, 'normal')
    r = EINetRunner('lif', n, n_exc, idx_e, idx_i, w_e, w_i, ops.lif_params(), V0)
    counts, hashes = _run_chunks(torch, r, T, [3000, 7000])
    say('  gpu done, running the C restatement on', _host_threads(), 'threads')
    c_ref, h_ref, st = _c_lif(idx_e, idx_i, w_e, w_i, neuron.LIFParams(), n_exc, V0, T, 0,
                              nthreads=_host_threads())
    assert c_ref.sum() > T * 1000   # ~0.1-0.2 % of the neurons fire per step
    assert counts.tolist() == c_ref.tolist()
    assert hashes.tolist() == h_ref.tolist()
    for key in ('V', 'ge', 'gi', 'ref'):
        assert np.array_equal(r.state[key].cpu().numpy(), st[key]), key
    assert np.array_equal(r.spk.cpu().numpy(), st['spk'])


def test_config5_full_length_matches_c(torch_cuda):
    """Config [5] for its whole run: 1M COBA-HH neurons, K = 80, per-synapse weights
    N(0.05, 0.005) / N(0.3, 0.03), dt 0.05 ms, 4,000 steps: every step's spike count and hash
    and the final V, m, h, n, g_e, g_i equal the C restatement's."""
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    from oracle import neuron
    torch = torch_cuda
    n, k, T = 1_000_000, 80, 4000
    say('config [5] full length', n, T)
    n_exc = n * 4 // 5
    idx_e = np.random.RandomState(211).randint(0, n, size=(n_exc, k)).astype(np.int32)
    idx_i = np.random.RandomState(212).randint(0, n, size=(n - n_exc, k)).astype(np.int32)
    V0 = np.random.RandomState(213).uniform(-70., -50., n).astype(F)
    w_e = np.random.RandomState(214).normal(0.05, 0.005, idx_e.shape).astype(F)
    w_i = np.random.RandomState(215).normal(0.3, 0.03, idx_i.shape).astype(F)
    r = EINetRunner('hh', n, n_exc, idx_e, idx_i, w_e, w_i, ops.hh_params(I_ext=6.5), V0)
    counts, hashes = _run_chunks(torch, r, T, [T])
    say('  gpu done, running the C restatement on', _host_threads(), 'threads')
    c_ref, h_ref, st = _c_hh(idx_e, idx_i, w_e, w_i, neuron.HHParams(I_ext=6.5), n_exc, V0, T,
                             nthreads=_host_threads())
    assert c_ref.sum() > T * 100
    assert counts.tolist() == c_ref.tolist()
    assert hashes.tolist() == h_ref.tolist()
    for key in ('V', 'm', 'h', 'n', 'ge', 'gi'):
        assert np.array_equal(r.state[key].cpu().numpy(), st[key]), key


@pytest.mark.parametrize('model,deferred', [('lif', False), ('lif', True), ('hh', False)])
def test_runner_per_step_inputs(torch_cuda, model, deferred):
    """bs_coba_*_run_inputs: one launch whose steps each take their own external input equals
    the same steps run one launch each with that input in the parameters, bit for bit
    (raster, final state); the LIF runs also equal the oracle stepped with the same inputs."""
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    torch = torch_cuda
    T = 60
    say('runner per-step inputs', model, deferred, T)
    rng = np.random.RandomState(11)
    if model == 'lif':
        pe, pi, V0, _ = make_golden.config1_net()
        c = make_golden.CONFIG1
        I = (20.0 + rng.uniform(-4.0, 4.0, T)).astype(F)
        mk = lambda: EINetRunner('lif', c['n'], c['n_exc'], pe.idx, pi.idx, c['w_e'], c['w_i'],  # noqa: E731
                                 ops.lif_params(deferred_reset=deferred), V0)
    else:
        pe, pi, V0, _ = make_golden.hh_net()
        c = make_golden.HH_NET
        I = (c['I_ext'] + rng.uniform(-1.0, 1.0, T)).astype(F)
        mk = lambda: EINetRunner('hh', c['n'], c['n_exc'], pe.idx, pi.idx, c['w_e'], c['w_i'],  # noqa: E731
                                 ops.hh_params(I_ext=c['I_ext']), V0)
    ra, rb = mk(), mk()
    ras_a = torch.zeros(T, c['n'], dtype=torch.uint8, device='cuda')
    ras_b = torch.zeros_like(ras_a)
    ra.run(T, raster=ras_a, inputs=torch.from_numpy(I))
    for t in range(T):
        rb.params.I_ext = float(I[t])
        rb.run(1, raster=ras_b[t:t + 1])
    ra.check()
    rb.check()
    assert int(ras_a.sum()) > 0
    assert torch.equal(ras_a, ras_b)
    for k in ra.state:
        assert torch.equal(ra.state[k], rb.state[k]), k
    if model == 'lif':
        init = None
        rows = []
        for t in range(T):
            p = neuron.LIFParams(I_ext=float(I[t]), deferred_reset=deferred)
            res = network.run_coba_lif(V0, pe, pi, p, c['n_exc'], 1, init=init)
            init = (res['V'], res['ge'], res['gi'], res['ref'], res['spk'])
            rows.append(res['raster'][0])
        assert np.array_equal(ras_a.cpu().numpy() != 0, np.stack(rows))
        assert np.array_equal(ra.state['V'].cpu().numpy(), init[0])


def test_runner_per_step_inputs_rejects_per_neuron_inputs(torch_cuda):
    """Per-step inputs do not combine with a runner built with one input per neuron."""
    from brainstate_amd import _native as N, ops
    from brainstate_amd.runner import EINetRunner
    torch = torch_cuda
    pe, pi, V0, _ = make_golden.config1_net()
    c = make_golden.CONFIG1
    r = EINetRunner('lif', c['n'], c['n_exc'], pe.idx, pi.idx, c['w_e'], c['w_i'],
                    ops.lif_params(), V0, I_ext=np.full(c['n'], 20.0, F))
    with pytest.raises(N.NativeError, match='do not combine'):
        r.run(3, inputs=torch.full((3,), 20.0))
