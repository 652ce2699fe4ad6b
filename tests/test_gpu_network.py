"""GPU parity of the persistent whole-loop runners against the oracle network loops."""
import json
import os
import sys

import numpy as np
import pytest

from oracle import network

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
    n = V0.size
    st = dict(V=V0.copy(), ge=np.zeros(n, F), gi=np.zeros(n, F), ref=np.zeros(n, np.int32),
              spk=np.zeros(n, np.uint8), in_e=np.zeros((D + 1) * n, F),
              in_i=np.zeros((D + 1) * n, F))
    c = np.zeros(T, np.int32)
    h = np.zeros(T, np.uint32)
    cbuild.coba_lif_run(st, idx_e, idx_i, w_e, w_i, p, n_exc, T, nthreads=nthreads, counts=c,
                        hashes=h, delay=D)
    return c, h, st


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


@pytest.mark.parametrize('het,chunks', [(False, [1000]), (True, [1000]), (False, [1, 9, 90, 900])])
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
    runner: raster, counts and final V equal the oracle's golden run."""
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
