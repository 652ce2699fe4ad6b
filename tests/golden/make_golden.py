"""Writes the golden fixtures in tests/golden/ from the oracle (run from the repo root).

    python tests/golden/make_golden.py

* conn_digests.json -- SHA-256 of the int32 index arrays that
  ``RandomState(seed).randint(0, n_post, (n_pre, K))`` produces for the seeds and shapes
  used by the parity configs (brainstate/nn/_event_fixedprob.py:165-171).
* coba_lif_4000.json -- config [1]: 4000-neuron COBA E/I net, 1000 steps; per-step spike
  counts, per-step order-free spike digests and SHA-256 of the raster / final state.
* coba_lif_4000_het.json -- the same net with random per-synapse weights summed in the
  persistent runner's fixed-point arithmetic (the exponents S_e, S_i recorded too).
* cuba_lif_4000.json -- examples/400_CUBA_2005_bpu.py's CUBA E/I net, 1000 steps, same records.
* tut_lif_soft_500.json -- the SNN tutorial's E/I net (LIF, soft reset, CUBA), 2000 steps.
* coba_hh_2000.json -- a 2000-neuron COBA-HH net, 600 steps, same records.
* hh_single_trace.json -- examples/100_hh_neuron_model.py's neuron (dt 0.01 ms, 10,000 steps,
  random input per step): SHA-256 of the V trace, its spike steps, V every 1000 steps.
* matvec_2000.json -- config [2] at 2000 x 2000, K = 100: SHA-256 of the homogeneous sums
  (order-free), of the sequential per-synapse sums and of the fixed-point sums, per density.
The reference itself is not imported (it needs JAX, brainevent and brainunit, which are
absent); these fixtures freeze the oracle so that any drift in it is caught.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import conn, event, neuron, network  # noqa: E402

CONFIG1 = dict(n=4000, n_exc=3200, p=0.02, w_e=0.6, w_i=6.7, seed_e=1, seed_i=2, seed_v=3,
               steps=1000)
# examples/400_CUBA_2005_bpu.py:36-66 (V0 ~ N(-55, 2) drawn with numpy; 1000 of its steps)
CUBA_NET = dict(n=4000, n_exc=3200, p=0.02, w_e=1.62, w_i=-9.0, seed_e=21, seed_i=22,
                seed_v=23, steps=1000, V_rest=-49., V_th=-50., V_reset=-60., tau=20.,
                tau_ref=5., I_ext=20.)
# docs/tutorials/brain_dynamics/04_building_an_snn.ipynb cells 11-14: LIF (no refractory
# period, soft reset) with CUBA outputs, balanced weights +-1/sqrt(p N), input 3 (V0 drawn
# with numpy)
TUT_NET = dict(n=500, n_exc=400, p=0.1, w_e=float(np.float32(1.0 / np.sqrt(40.0))),
               w_i=float(np.float32(-1.0 / np.sqrt(10.0))), seed_e=31, seed_i=32, seed_v=33,
               steps=2000, V_rest=-52., V_th=-50., V_reset=-60., tau=10., tau_e=2., tau_i=2.,
               I_ext=3.)
# examples/100_hh_neuron_model.py:96-112: 10 HH neurons, dt = 0.01 ms, 100 ms, input
# uniform(1, 10) per step (drawn with numpy)
HH_SINGLE = dict(n=10, dt=0.01, steps=10000, seed_in=7, V0=-65.)
# config [2] at reduced size: 2000 x 2000, K = 100, w ~ N(0.5, 0.1), spikes at three densities
MATVEC = dict(n_pre=2000, n_post=2000, k=100, seed_idx=41, seed_w=42, seed_spk=43,
              p=[0.001, 0.01, 0.1], w_homo=0.6)
HH_NET = dict(n=2000, n_exc=1600, k=80, w_e=0.05, w_i=0.3, seed_e=11, seed_i=12, seed_v=13,
              steps=600, I_ext=6.5)
# config [1] with per-synapse weights w_e ~ N(0.6, 0.06), w_i ~ N(6.7, 0.67) (numpy seeds),
# summed as the persistent runner sums them (fixed point, oracle.network.fixed_point_input)
CONFIG1_HET = dict(CONFIG1, seed_we=4, seed_wi=5, sd_e=0.06, sd_i=0.67)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def config1_net():
    c = CONFIG1
    pe = network.Projection(0, c['n_exc'], c['n'], c['p'], c['w_e'], seed=c['seed_e'])
    pi = network.Projection(c['n_exc'], c['n'], c['n'], c['p'], c['w_i'], seed=c['seed_i'])
    V0 = np.random.RandomState(c['seed_v']).uniform(-60., -50., c['n']).astype(np.float32)
    return pe, pi, V0, neuron.LIFParams()


def config1_het_weights(shape_e, shape_i):
    c = CONFIG1_HET
    we = np.random.RandomState(c['seed_we']).normal(c['w_e'], c['sd_e'], shape_e)
    wi = np.random.RandomState(c['seed_wi']).normal(c['w_i'], c['sd_i'], shape_i)
    return we.astype(np.float32), wi.astype(np.float32)


def config1_het_net():
    """Config [1] with random per-synapse weights, runner (fixed-point) sums."""
    c = CONFIG1_HET
    pe0, pi0, V0, p = config1_net()
    we, wi = config1_het_weights(pe0.idx.shape, pi0.idx.shape)
    pe = network.Projection(0, c['n_exc'], c['n'], c['p'], we, seed=c['seed_e'], fixed=True)
    pi = network.Projection(c['n_exc'], c['n'], c['n'], c['p'], wi, seed=c['seed_i'], fixed=True)
    return pe, pi, V0, p


def cuba_net():
    c = CUBA_NET
    pe = network.Projection(0, c['n_exc'], c['n'], c['p'], c['w_e'], seed=c['seed_e'])
    pi = network.Projection(c['n_exc'], c['n'], c['n'], c['p'], c['w_i'], seed=c['seed_i'])
    V0 = np.random.RandomState(c['seed_v']).normal(-55., 2., c['n']).astype(np.float32)
    p = neuron.LIFParams(V_rest=c['V_rest'], V_th=c['V_th'], V_reset=c['V_reset'],
                         tau=c['tau'], tau_ref=c['tau_ref'], I_ext=c['I_ext'], out='cuba')
    return pe, pi, V0, p


def tut_net():
    c = TUT_NET
    pe = network.Projection(0, c['n_exc'], c['n'], c['p'], c['w_e'], seed=c['seed_e'])
    pi = network.Projection(c['n_exc'], c['n'], c['n'], c['p'], c['w_i'], seed=c['seed_i'])
    V0 = np.random.RandomState(c['seed_v']).normal(-60., 10., c['n']).astype(np.float32)
    p = neuron.LIFParams(V_rest=c['V_rest'], V_th=c['V_th'], V_reset=c['V_reset'],
                         tau=c['tau'], tau_ref=0., tau_e=c['tau_e'], tau_i=c['tau_i'],
                         I_ext=c['I_ext'], out='cuba', spk_reset='soft')
    return pe, pi, V0, p


def hh_net():
    c = HH_NET
    pe = network.Projection(0, c['n_exc'], c['n'], c['k'], c['w_e'], seed=c['seed_e'])
    pi = network.Projection(c['n_exc'], c['n'], c['n'], c['k'], c['w_i'], seed=c['seed_i'])
    V0 = np.random.RandomState(c['seed_v']).uniform(-70., -50., c['n']).astype(np.float32)
    return pe, pi, V0, neuron.HHParams(I_ext=c['I_ext'])


def hh_single_trace():
    """V of neuron 0 after every step, and the steps at which it spikes."""
    c = HH_SINGLE
    inp = np.random.RandomState(c['seed_in']).uniform(1., 10., c['steps']).astype(np.float32)
    V = np.full(c['n'], c['V0'], np.float32)
    m, h, ng = neuron.hh_init(V)
    z = np.zeros(c['n'], np.float32)
    ge, gi = z.copy(), z.copy()
    trace = np.zeros(c['steps'], np.float32)
    spikes = []
    for t in range(c['steps']):
        p = neuron.HHParams(I_ext=float(inp[t]), dt=c['dt'])
        V, m, h, ng, ge, gi, spk = neuron.hh_step(V, m, h, ng, ge, gi, z, z, p)
        trace[t] = V[0]
        if spk[0]:
            spikes.append(t)
    return inp, trace, spikes


def matvec_case(p_spk):
    """(spk, idx, w) of the reduced config-[2] mat-vec at spike density p_spk."""
    c = MATVEC
    idx = np.random.RandomState(c['seed_idx']).randint(0, c['n_post'], (c['n_pre'], c['k']))
    w = np.random.RandomState(c['seed_w']).normal(0.5, 0.1, idx.shape).astype(np.float32)
    rs = np.random.RandomState(c['seed_spk'] + int(round(p_spk * 1000)))
    spk = (rs.rand(c['n_pre']) < p_spk).astype(np.uint8)
    return spk, idx.astype(np.int32), w


def run_records(res):
    return dict(counts=res['counts'].tolist(),
                hashes=[network.spike_hash(r) for r in res['raster']],
                raster_sha256=sha(np.packbits(res['raster'])),
                final_V_sha256=sha(res['V']))


def main():
    digests = []
    for n_pre, n_post, k, seed in [(3200, 4000, 80, 1), (800, 4000, 80, 2), (20, 30, 6, 11),
                                   (1600, 2000, 80, 11), (400, 2000, 80, 12)]:
        idx, _ = conn.fixed_num_indices(n_pre, n_post, k, seed)
        digests.append(dict(n_pre=n_pre, n_post=n_post, k=k, seed=seed, sha256=sha(idx)))
    with open(os.path.join(HERE, 'conn_digests.json'), 'w') as f:
        json.dump(digests, f, indent=1)

    pe, pi, V0, p = config1_net()
    res = network.run_coba_lif(V0, pe, pi, p, CONFIG1['n_exc'], CONFIG1['steps'])
    rec = dict(config=CONFIG1, **run_records(res))
    with open(os.path.join(HERE, 'coba_lif_4000.json'), 'w') as f:
        json.dump(rec, f)
    print('coba_lif_4000: total spikes', int(res['counts'].sum()))

    pe, pi, V0, p = config1_het_net()
    res = network.run_coba_lif(V0, pe, pi, p, CONFIG1_HET['n_exc'], CONFIG1_HET['steps'])
    rec = dict(config=CONFIG1_HET, qexp=[pe.S, pi.S], **run_records(res))
    with open(os.path.join(HERE, 'coba_lif_4000_het.json'), 'w') as f:
        json.dump(rec, f)
    print('coba_lif_4000_het: total spikes', int(res['counts'].sum()))

    pe, pi, V0, p = cuba_net()
    res = network.run_coba_lif(V0, pe, pi, p, CUBA_NET['n_exc'], CUBA_NET['steps'])
    rec = dict(config=CUBA_NET, **run_records(res))
    with open(os.path.join(HERE, 'cuba_lif_4000.json'), 'w') as f:
        json.dump(rec, f)
    print('cuba_lif_4000: total spikes', int(res['counts'].sum()))

    pe, pi, V0, p = tut_net()
    res = network.run_coba_lif(V0, pe, pi, p, TUT_NET['n_exc'], TUT_NET['steps'])
    rec = dict(config=TUT_NET, **run_records(res))
    with open(os.path.join(HERE, 'tut_lif_soft_500.json'), 'w') as f:
        json.dump(rec, f)
    print('tut_lif_soft_500: total spikes', int(res['counts'].sum()))

    inp, trace, spikes = hh_single_trace()
    rec = dict(config=HH_SINGLE, trace_sha256=sha(trace), spikes=spikes,
               V_every_1000=[float(v) for v in trace[999::1000]])
    with open(os.path.join(HERE, 'hh_single_trace.json'), 'w') as f:
        json.dump(rec, f)
    print('hh_single_trace: spikes', len(spikes))

    cases = []
    for p_spk in MATVEC['p']:
        spk, idx, w = matvec_case(p_spk)
        homo = event.scatter_fixed(spk, idx, np.float32(MATVEC['w_homo']), MATVEC['n_post'])
        het = event.scatter_fixed(spk, idx, w, MATVEC['n_post'])
        S = event.bucket_qexp(w, idx, MATVEC['n_post'])
        indptr = np.arange(MATVEC['n_pre'] + 1, dtype=np.int64) * MATVEC['k']
        fixed = event.scatter_fixed_point(spk, indptr, idx.reshape(-1), w, MATVEC['n_post'], S)
        cases.append(dict(p=p_spk, active=int(spk.sum()), homo_sha256=sha(homo),
                          het_sequential_sha256=sha(het), fixed_point_S=S,
                          fixed_point_sha256=sha(fixed)))
    with open(os.path.join(HERE, 'matvec_2000.json'), 'w') as f:
        json.dump(dict(config=MATVEC, cases=cases), f, indent=1)
    print('matvec_2000:', [c['active'] for c in cases])

    pe, pi, V0, p = hh_net()
    res = network.run_coba_hh(V0, pe, pi, p, HH_NET['n_exc'], HH_NET['steps'])
    rec = dict(config=HH_NET, **run_records(res))
    with open(os.path.join(HERE, 'coba_hh_2000.json'), 'w') as f:
        json.dump(rec, f)
    print('coba_hh_2000: total spikes', int(res['counts'].sum()))


if __name__ == '__main__':
    main()
