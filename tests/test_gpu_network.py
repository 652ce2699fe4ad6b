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


def _lif_runner(torch, het, blocks_per_cu=0):
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    pe, pi, V0, _ = make_golden.config1_net()
    c = make_golden.CONFIG1
    return EINetRunner('lif', c['n'], c['n_exc'], pe.idx, pi.idx,
                       np.full(pe.idx.shape, F(c['w_e'])) if het else c['w_e'],
                       np.full(pi.idx.shape, F(c['w_i'])) if het else c['w_i'],
                       ops.lif_params(), V0, blocks_per_cu=blocks_per_cu)


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
