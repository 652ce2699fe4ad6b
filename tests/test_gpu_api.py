"""GPU tests of the brainstate-compatible layer: the reference's own layer tests, and an
E/I network built from modules, stepped eagerly and fused, against the oracle."""
import json
import os
import sys

import numpy as np
import pytest

from oracle import event, network, neuron

pytestmark = pytest.mark.gpu

F = np.float32


def ops_chunks(batch, n_in, n_out):
    """(S, L) of bs_event_dense_f32's summation order for this shape."""
    from brainstate_amd import ops
    return ops.event_dense_chunks(batch, n_in, n_out)
GOLD = os.path.join(os.path.dirname(__file__), 'golden')
sys.path.insert(0, GOLD)
import make_golden  # noqa: E402


@pytest.fixture(scope='module')
def bs():
    import torch
    if not torch.cuda.is_available():
        pytest.fail('GPU tests need a ROCm GPU')
    import brainstate_amd
    return brainstate_amd


def test_event_update_matches_dense_reference(bs):
    """brainstate/nn/_event_fixedprob_test.py:247-260."""
    import torch
    print('[case] fixedprob np.add.at', flush=True)
    n_in, n_out = 20, 30
    fn = bs.nn.EventFixedProb(n_in, n_out, 0.2, 1.5, seed=11)
    spk = np.random.RandomState(0).rand(n_in) < 0.3
    out = fn(torch.tensor(spk.astype(np.float32), device='cuda')).cpu().numpy()
    indices = fn.conn.indices.cpu().numpy()
    ref = np.zeros((n_out,))
    for i in range(n_in):
        np.add.at(ref, indices[i], 1.5 * float(spk[i]))
    assert np.allclose(out, ref, rtol=1e-4, atol=1e-4)
    assert np.array_equal(indices, np.random.RandomState(11).randint(0, n_out, (n_in, 6)))


def test_fixedprob_heterogeneous_and_batched(bs):
    import torch
    print('[case] fixedprob het batched', flush=True)
    m = bs.nn.EventFixedProb(300, 200, 40, bs.nn.init.Normal(0.5, 0.1, seed=3), seed=5)
    spk = np.random.RandomState(1).rand(3, 300) < 0.2
    out = m(torch.tensor(spk, device='cuda')).cpu().numpy()
    w = np.asarray(m.weight.value, F)
    idx = m.conn.indices.cpu().numpy()
    for b in range(3):
        np.testing.assert_allclose(out[b], event.scatter_fixed(spk[b], idx, w, 200),
                                   rtol=1e-5, atol=1e-6)


def test_fixedprob_afferent_ratio_csr(bs):
    import torch
    print('[case] fixedprob csr', flush=True)
    m = bs.nn.EventFixedProb(500, 400, 30, 0.7, seed=9, afferent_ratio=0.5)
    from oracle import conn
    indptr, indices, sel = conn.csr_afferent(500, 400, 30, 9, 0.5)
    assert np.array_equal(m.conn.indptr.cpu().numpy(), indptr)
    spk = np.random.RandomState(2).rand(500) < 0.3
    out = m(torch.tensor(spk, device='cuda')).cpu().numpy()
    assert np.array_equal(out, event.scatter_csr(spk, indptr, indices, F(0.7), 400))


def test_fixedprob_zero_conn_returns_zeros(bs):
    import torch
    m = bs.nn.EventFixedProb(10, 7, 0.0, 1.0)
    out = m(torch.ones(4, 10, device='cuda'))
    assert out.shape == (4, 7) and float(out.abs().sum()) == 0.0


@pytest.mark.parametrize('bool_x', [True, False])
@pytest.mark.parametrize('homo_w', [True, False])
def test_event_linear_reference_test1(bs, homo_w, bool_x):     # _event_linear_test.py:26-40
    import torch
    print('[case] event linear', homo_w, bool_x, flush=True)
    x = np.random.RandomState(4).rand(20) < 0.1
    x = x if bool_x else x.astype(F)
    m = bs.nn.EventLinear(20, 40, 1.5 if homo_w else bs.nn.init.Uniform(-0.5, 0.5, seed=1),
                          float_as_event=bool_x)
    y = m(torch.tensor(x, device='cuda')).cpu().numpy()
    W = m.weight.value
    expect = x.sum() * W * np.ones(40) if homo_w else x.astype(F) @ W
    assert np.allclose(y, expect, rtol=1e-5)


@pytest.mark.parametrize('float_as_event', [True, False])
def test_event_linear_homogeneous_matches_dense_nonbinary(bs, float_as_event):  # :127-162
    import torch
    spk = torch.tensor([0., 2., 0., 3., 0., 0., 1., 0., 0., 5.], device='cuda')
    homo = bs.nn.EventLinear(10, 8, 1.5, float_as_event=float_as_event)
    dense = bs.nn.EventLinear(10, 8, bs.nn.init.Constant(1.5), float_as_event=float_as_event)
    yh, yd = homo(spk).cpu().numpy(), dense(spk).cpu().numpy()
    assert np.allclose(yh, yd)
    assert np.allclose(yh, np.ones(8) * (4 if float_as_event else 11) * 1.5)


def test_event_linear_batched_bit_exact(bs):
    import torch
    print('[case] event linear batched', flush=True)
    rng = np.random.RandomState(7)
    spk = rng.rand(64, 512) < 0.05
    W = rng.normal(0, 0.125, (512, 256)).astype(F)
    m = bs.nn.EventLinear(512, 256, W, event_kernel='stream')
    y = m(torch.tensor(spk, device='cuda')).cpu().numpy()
    _, L = ops_chunks(64, 512, 256)
    assert np.array_equal(y, event.event_linear(spk, W, chunk_rows=L))
    p = bs.nn.EventLinear(512, 256, W)   # 'auto': packed, exact per-column fixed point
    assert np.array_equal(p(torch.tensor(spk, device='cuda')).cpu().numpy(),
                          event.event_dense_fixed_point(spk, W))


class _EINet:
    """examples/105_COBA_HH_2007_braincell.py:54-82 with config-[1] LIF parameters."""

    def __init__(self, bs, w_e=0.6, w_i=6.7, **lif):
        c = make_golden.CONFIG1
        self.bs = bs
        self.n_exc, self.num = c['n_exc'], c['n']
        V0 = np.random.RandomState(c['seed_v']).uniform(-60., -50., c['n']).astype(F)
        kw = dict(V_rest=-60., V_th=-50., V_reset=-60., tau=20., tau_ref=5.)
        kw.update(lif)   # e.g. per-neuron parameter arrays
        self.N = bs.nn.LIFRef(self.num, V_initializer=lambda s: V0, **kw)
        self.E = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(self.n_exc, self.num, conn_num=0.02, conn_weight=w_e,
                                      seed=c['seed_e']),
            syn=bs.nn.Expon.desc(self.num, tau=5.), out=bs.nn.COBA.desc(E=0.), post=self.N)
        self.I = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(self.num - self.n_exc, self.num, conn_num=0.02,
                                      conn_weight=w_i, seed=c['seed_i']),
            syn=bs.nn.Expon.desc(self.num, tau=10.), out=bs.nn.COBA.desc(E=-80.), post=self.N)
        for m in (self.E.syn, self.I.syn, self.N):
            m.init_state()

    def update(self, t):
        with self.bs.environ.context(t=t):
            spk = self.N.get_spike() != 0.
            self.E(spk[:self.n_exc])
            self.I(spk[self.n_exc:])
            self.N(20.)
            return self.N.get_spike()


def _for_loop_paths(bs, make_step, T, dt=0.1):
    """for_loop(step, times) on a fresh net twice: stepped eagerly, then the default that
    hands the loop to the persistent runner after two recorded steps.  Returns
    [(raster, net), ...] and checks which path each took."""
    import torch
    res = []
    for fused in (False, True):
        bs.transform.fuse_loops = fused
        try:
            with bs.environ.context(dt=dt):
                step, net = make_step()
                # the fused pass with a progress bar, as examples/105_COBA_HH_2007_braincell.py:91
                pbar = bs.transform.ProgressBar(10) if fused and T >= 10 else None
                res.append((bs.transform.for_loop(step, torch.arange(T) * dt, pbar=pbar), net))
        finally:
            bs.transform.fuse_loops = True
        assert bs.transform.last_loop == ('fused' if fused else 'eager')
    return res


@pytest.mark.parametrize('het', [False, True])
def test_for_loop_chunks_reuse_the_runner(bs, het):
    """Loops run in chunks on one net keep its persistent runner (no new set-up) and reload
    the modules' state each time: chunks of 60, 40 and 50 steps with the state changed
    between chunks (V shifted, the E conductances scaled) equal the same chunks stepped
    eagerly with the same changes; a new weight value builds a new runner.  With per-synapse
    weights (N(0.6, 0.06) / N(6.7, 0.67)) the eager steps use the runner's fixed-point sums,
    so both paths stay bit-equal."""
    import torch
    print('[case] for_loop chunks reuse the runner', het, flush=True)
    res = []
    for fused in (False, True):
        bs.transform.fuse_loops = fused
        try:
            with bs.environ.context(dt=0.1):
                if het:
                    net = _EINet(bs, w_e=bs.nn.init.Normal(0.6, 0.06, seed=5),
                                 w_i=bs.nn.init.Normal(6.7, 0.67, seed=6))
                else:
                    net = _EINet(bs)
                outs, runners = [], []
                for i, T in enumerate((60, 40, 50)):
                    if i == 1:
                        net.N.V.value = net.N.V.value + 0.25
                        net.E.syn.g.value = net.E.syn.g.value * 1.5
                    if i == 2:
                        w = net.E.comm.weight.value
                        net.E.comm.weight.value = (np.asarray(w) * F(1.1)).astype(F) if het \
                            else 0.7
                    outs.append(bs.transform.for_loop(net.update, torch.arange(T) * 0.1))
                    assert bs.transform.last_loop == ('fused' if fused else 'eager')
                    r = getattr(net.N, '_fused_runner', None)
                    runners.append(None if r is None else r[1])
                if fused:
                    assert runners[1] is runners[0] and runners[2] is not runners[1]
                res.append((torch.cat(outs), net))
        finally:
            bs.transform.fuse_loops = True
    (a, na), (b, nb) = res
    assert int(a.sum()) > 0
    assert torch.equal(a, b)
    assert torch.equal(na.N.V.value, nb.N.V.value)
    assert torch.equal(na.E.syn.g.value, nb.E.syn.g.value)
    assert torch.equal(na.N.ref.value, nb.N.ref.value)


def test_module_ei_network_matches_oracle(bs):
    """The reference's E/I script shape (examples/105_COBA_HH_2007_braincell.py:76-91):
    for_loop(net.update, times) stepped eagerly and through the persistent runner; both
    rasters and final states equal the oracle's."""
    print('[case] module E/I net for_loop eager + fused', flush=True)
    T = 300
    pe, pi, V0, p = make_golden.config1_net()
    p.deferred_reset = True   # LIFRef's default reset_timing='next'
    ref = network.run_coba_lif(V0, pe, pi, p, 3200, T)

    def make():
        net = _EINet(bs)
        return net.update, net
    for spikes, net in _for_loop_paths(bs, make, T):
        assert spikes.dtype == net.N.get_spike().dtype and spikes.shape == (T, 4000)
        assert np.array_equal(spikes.cpu().numpy() != 0, ref['raster'])
        assert np.array_equal(net.N.V.value.cpu().numpy(), ref['V'])
        assert np.array_equal(net.E.syn.g.value.cpu().numpy(), ref['ge'])
        assert np.array_equal(net.N.ref.value.cpu().numpy(), ref['ref'])
        assert np.array_equal(net.N.spike.value.cpu().numpy(), ref['spk'])


def test_module_ei_network_per_neuron_input(bs):
    """The same script with one external input per neuron (N(x), x of shape [n]): eager
    steps and the persistent runner (for_loop hands the loop over with the array) both equal
    the oracle given that array."""
    import torch
    print('[case] module E/I net, per-neuron input', flush=True)
    T = 300
    pe, pi, V0, p = make_golden.config1_net()
    I = (20. + np.random.RandomState(5).uniform(-3., 3., V0.size)).astype(F)
    ref = network.run_coba_lif(V0, pe, pi, neuron.LIFParams(I_ext=I, deferred_reset=True),
                               3200, T)
    dI = torch.as_tensor(I, device='cuda')

    def make():
        net = _EINet(bs)

        def step(t):
            spk = net.N.get_spike() != 0.
            net.E(spk[:net.n_exc])
            net.I(spk[net.n_exc:])
            return net.N(dI)
        return step, net
    for spikes, net in _for_loop_paths(bs, make, T):
        assert np.array_equal(spikes.cpu().numpy() != 0, ref['raster'])
        assert np.array_equal(net.N.V.value.cpu().numpy(), ref['V'])
        assert np.array_equal(net.N.ref.value.cpu().numpy(), ref['ref'])


@pytest.mark.parametrize('kernel', ['auto', 'bucket'])
def test_for_loop_1m_fused_equals_eager(bs, kernel):
    """A 1M-neuron module net (K = 100, homogeneous weights): for_loop handed to the runner
    equals the loop stepped eagerly.  The eager mat-vecs take the atomic kernel under 'auto'
    (82 buckets of 1M posts hold ~1.2 of a row's 100 synapses each: too few for the bucketed
    layout) and the bucketed layout under 'bucket'; the fused loop's recorded steps take the
    one-launch kernel (no layout built)."""
    import torch
    print('[case] 1M module net, for_loop fused = eager', kernel, flush=True)
    n, k, T = 1_000_000, 100, 40
    n_exc = n * 4 // 5
    V0 = np.random.RandomState(3).uniform(-60., -50., n).astype(F)

    def make():
        N = bs.nn.LIFRef(n, V_rest=-60., V_th=-50., V_reset=-60., tau=20., tau_ref=5.,
                         V_initializer=lambda s: V0)
        E = bs.nn.AlignPostProj(comm=bs.nn.EventFixedProb(n_exc, n, k, 0.6, seed=1,
                                                           event_kernel=kernel),
                                syn=bs.nn.Expon.desc(n, tau=5.), out=bs.nn.COBA.desc(E=0.),
                                post=N)
        I = bs.nn.AlignPostProj(comm=bs.nn.EventFixedProb(n - n_exc, n, k, 6.7, seed=2,
                                                           event_kernel=kernel),
                                syn=bs.nn.Expon.desc(n, tau=10.), out=bs.nn.COBA.desc(E=-80.),
                                post=N)
        for m in (E.syn, I.syn, N):
            m.init_state()

        def step(t):
            spk = N.get_spike() != 0.
            E(spk[:n_exc])
            I(spk[n_exc:])
            return N(20.)
        return step, (N, E)
    (eager, (Ne, Ee)), (fused, (Nf, Ef)) = _for_loop_paths(bs, make, T)
    assert (Ee.comm._bucket is not None) == (kernel == 'bucket') and Ef.comm._bucket is None
    assert int(eager.sum()) > T * 500
    assert torch.equal(eager, fused)
    assert torch.equal(Ne.V.value, Nf.V.value)


def test_module_ei_network_per_neuron_parameters(bs):
    """LIFRef with array-valued V_th, tau and tau_ref (one value per neuron): the eager step
    (bs_coba_lif_step_arr) equals the oracle given the same arrays (tau as its fp32
    reciprocal, tau_ref as each neuron's refractory steps); for_loop keeps such a net eager
    (the runner's parameters are scalars) and fuse() says so."""
    import torch
    print('[case] module E/I net, per-neuron parameters', flush=True)
    T = 200
    c = make_golden.CONFIG1
    pe, pi, V0, p = make_golden.config1_net()
    rs = np.random.RandomState(12)
    V_th = rs.uniform(-52., -48., c['n']).astype(F)
    tau = rs.uniform(15., 25., c['n']).astype(F)
    tau_ref = rs.choice([2., 5., 8.], c['n']).astype(F)
    p.V_th, p.tau = V_th, tau
    p.inv_tau = (F(1.0) / tau).astype(F)
    p.ref_steps = np.array([neuron.ref_steps(x, 0.1) for x in tau_ref], np.int32)
    p.deferred_reset = True
    ref = network.run_coba_lif(V0, pe, pi, p, 3200, T)
    with bs.environ.context(dt=0.1):
        net = _EINet(bs, V_th=V_th, tau=tau, tau_ref=tau_ref)
        N = net.N

        def step(t):
            spk = N.get_spike() != 0.
            net.E(spk[:net.n_exc])
            net.I(spk[net.n_exc:])
            return N(20.)
        spikes = bs.transform.for_loop(step, torch.arange(T) * 0.1)
        assert bs.transform.last_loop == 'eager'
        with pytest.raises(NotImplementedError, match='per-neuron parameters'):
            bs.nn.fuse(N, net.E, net.I, n_exc=3200, inp=20.)
    assert np.array_equal(spikes.cpu().numpy() != 0, ref['raster'])
    assert np.array_equal(N.V.value.cpu().numpy(), ref['V'])
    assert np.array_equal(N.ref.value.cpu().numpy(), ref['ref'])
    assert ref['counts'].sum() > 100


def test_hh_module_network_for_loop(bs):
    """A COBA-HH E/I net (the shape of examples/105_COBA_HH_2007_braincell.py) built from the
    modules: for_loop eagerly and through the runner, both equal to the oracle's golden run."""
    print('[case] HH module net for_loop', flush=True)
    c = make_golden.HH_NET
    with open(os.path.join(GOLD, 'coba_hh_2000.json')) as f:
        gold = json.load(f)
    V0 = np.random.RandomState(c['seed_v']).uniform(-70., -50., c['n']).astype(F)

    def make():
        N = bs.nn.HH(c['n'], V_initializer=lambda s: V0)
        E = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(c['n_exc'], c['n'], c['k'], c['w_e'], seed=c['seed_e']),
            syn=bs.nn.Expon.desc(c['n'], tau=5.), out=bs.nn.COBA.desc(E=0.), post=N)
        I = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(c['n'] - c['n_exc'], c['n'], c['k'], c['w_i'],
                                      seed=c['seed_i']),
            syn=bs.nn.Expon.desc(c['n'], tau=10.), out=bs.nn.COBA.desc(E=-80.), post=N)
        bs.nn.init_all_states(N)
        for m in (E.syn, I.syn):
            m.init_state()

        def step(t):
            spk = N.get_spike() != 0.
            E(spk[:c['n_exc']])
            I(spk[c['n_exc']:])
            return N(c['I_ext'])
        return step, N
    for spikes, N in _for_loop_paths(bs, make, c['steps'], dt=0.05):
        ras = spikes.cpu().numpy() != 0
        assert ras.sum(1).tolist() == gold['counts']
        assert make_golden.sha(np.packbits(ras)) == gold['raster_sha256']
        assert make_golden.sha(N.V.value.cpu().numpy()) == gold['final_V_sha256']


def test_hh_module_network_for_loop_in_chunks(bs):
    """The HH net of the previous test run through the runner in three for_loop chunks: one
    runner kept and reloaded between them, and the concatenated raster and the final V equal
    the oracle's single golden run."""
    import torch
    print('[case] HH module net for_loop in chunks', flush=True)
    c = make_golden.HH_NET
    with open(os.path.join(GOLD, 'coba_hh_2000.json')) as f:
        gold = json.load(f)
    V0 = np.random.RandomState(c['seed_v']).uniform(-70., -50., c['n']).astype(F)
    with bs.environ.context(dt=0.05):
        N = bs.nn.HH(c['n'], V_initializer=lambda s: V0)
        E = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(c['n_exc'], c['n'], c['k'], c['w_e'], seed=c['seed_e']),
            syn=bs.nn.Expon.desc(c['n'], tau=5.), out=bs.nn.COBA.desc(E=0.), post=N)
        I = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(c['n'] - c['n_exc'], c['n'], c['k'], c['w_i'],
                                      seed=c['seed_i']),
            syn=bs.nn.Expon.desc(c['n'], tau=10.), out=bs.nn.COBA.desc(E=-80.), post=N)
        bs.nn.init_all_states(N)
        for m in (E.syn, I.syn):
            m.init_state()

        def step(t):
            spk = N.get_spike() != 0.
            E(spk[:c['n_exc']])
            I(spk[c['n_exc']:])
            return N(c['I_ext'])
        T = c['steps']
        cuts = [0, T * 2 // 5, T * 3 // 4, T]
        outs, runners = [], []
        for a, b in zip(cuts[:-1], cuts[1:]):
            outs.append(bs.transform.for_loop(step, torch.arange(a, b) * 0.05))
            assert bs.transform.last_loop == 'fused'
            runners.append(N._fused_runner[1])
        assert runners[0] is runners[1] is runners[2]
    ras = torch.cat(outs).cpu().numpy() != 0
    assert ras.sum(1).tolist() == gold['counts']
    assert make_golden.sha(np.packbits(ras)) == gold['raster_sha256']
    assert make_golden.sha(N.V.value.cpu().numpy()) == gold['final_V_sha256']


def test_hh_module_network_per_neuron_parameters(bs):
    """HH with array-valued gL, gK and V_th (one value per neuron): the eager steps
    (bs_coba_hh_step_arr) equal the oracle given the same arrays; for_loop stays eager."""
    import torch
    print('[case] HH module net, per-neuron parameters', flush=True)
    c = make_golden.HH_NET
    T = 300
    pe, pi, V0, p = make_golden.hh_net()
    rs = np.random.RandomState(14)
    gL = rs.uniform(0.02, 0.04, c['n']).astype(F)
    gK = rs.uniform(30., 40., c['n']).astype(F)
    V_th = rs.uniform(15., 25., c['n']).astype(F)
    p.gL, p.gK, p.V_th = gL, gK, V_th
    ref = network.run_coba_hh(V0, pe, pi, p, c['n_exc'], T)
    with bs.environ.context(dt=0.05):
        N = bs.nn.HH(c['n'], gL=gL, gK=gK, V_th=V_th, V_initializer=lambda s: V0)
        E = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(c['n_exc'], c['n'], c['k'], c['w_e'], seed=c['seed_e']),
            syn=bs.nn.Expon.desc(c['n'], tau=5.), out=bs.nn.COBA.desc(E=0.), post=N)
        I = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(c['n'] - c['n_exc'], c['n'], c['k'], c['w_i'],
                                      seed=c['seed_i']),
            syn=bs.nn.Expon.desc(c['n'], tau=10.), out=bs.nn.COBA.desc(E=-80.), post=N)
        bs.nn.init_all_states(N)
        for m in (E.syn, I.syn):
            m.init_state()

        def step(t):
            spk = N.get_spike() != 0.
            E(spk[:c['n_exc']])
            I(spk[c['n_exc']:])
            return N(c['I_ext'])
        spikes = bs.transform.for_loop(step, torch.arange(T) * 0.05)
        assert bs.transform.last_loop == 'eager'
    assert np.array_equal(spikes.cpu().numpy() != 0, ref['raster'])
    assert np.array_equal(N.V.value.cpu().numpy(), ref['V'])
    assert ref['counts'].sum() > 50


def test_for_loop_input_changing_every_step(bs):
    """A step whose input changes every step (20 + t) is recorded step by step and run in the
    runner with one launch per step; it equals the loop stepped eagerly."""
    import torch
    print('[case] for_loop time-varying input', flush=True)
    outs, nets = [], []
    for fused in (False, True):
        bs.transform.fuse_loops = fused
        try:
            with bs.environ.context(dt=0.1):
                net = _EINet(bs)

                def step(t):
                    spk = net.N.get_spike() != 0.
                    net.E(spk[:net.n_exc])
                    net.I(spk[net.n_exc:])
                    return net.N(20. + float(t))

                outs.append(bs.transform.for_loop(step, torch.arange(50) * 0.1))
                nets.append(net)
        finally:
            bs.transform.fuse_loops = True
        assert bs.transform.last_loop == ('fused' if fused else 'eager')
    assert int(outs[0].sum()) > 0
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(nets[0].N.V.value, nets[1].N.V.value)
    assert torch.equal(nets[0].E.syn.g.value, nets[1].E.syn.g.value)


def _switch_oracle(T, t_switch, I_on, I_off):
    """The oracle's run of the config-[1] net with input I_on for steps [0, t_switch) and
    I_off after, continuing one run's state in the next."""
    pe, pi, V0, _ = make_golden.config1_net()
    a = network.run_coba_lif(V0, pe, pi, neuron.LIFParams(I_ext=I_on, deferred_reset=True),
                             3200, t_switch)
    init = (a['V'], a['ge'], a['gi'], a['ref'], a['spk'])
    b = network.run_coba_lif(V0, pe, pi, neuron.LIFParams(I_ext=I_off, deferred_reset=True),
                             3200, T - t_switch, init=init)
    b['raster'] = np.concatenate([a['raster'], b['raster']])
    return b


def test_for_loop_drive_switch(bs):
    """for_loop(lambda t: net.update(20 if t < 5 ms else 0), times): the step uses its
    argument, so every step is recorded with its value; the inputs form two runs of equal
    input, run as two launches, and the loop equals the loop stepped eagerly and the oracle
    (input 20 for 50 steps, then 0) -- raster, final V, conductances, refractory counts."""
    import torch
    print('[case] for_loop drive switching at 5 ms', flush=True)
    T = 300
    ref = _switch_oracle(T, 50, 20., 0.)
    assert ref['raster'][:50].sum() > 0 and ref['raster'].sum() > ref['raster'][:50].sum()

    class Net(_EINet):
        def update(self, t):
            with self.bs.environ.context(t=t):
                spk = self.N.get_spike() != 0.
                self.E(spk[:self.n_exc])
                self.I(spk[self.n_exc:])
                return self.N(20. if t < 5. else 0.)

    def make():
        net = Net(bs)
        return net.update, net
    for spikes, net in _for_loop_paths(bs, make, T):
        assert spikes.dtype == torch.bool and spikes.shape == (T, 4000)
        assert np.array_equal(spikes.cpu().numpy(), ref['raster'])
        assert np.array_equal(net.N.V.value.cpu().numpy(), ref['V'])
        assert np.array_equal(net.E.syn.g.value.cpu().numpy(), ref['ge'])
        assert np.array_equal(net.I.syn.g.value.cpu().numpy(), ref['gi'])
        assert np.array_equal(net.N.ref.value.cpu().numpy(), ref['ref'])
        assert np.array_equal(net.N.spike.value.cpu().numpy(), ref['spk'])


def test_for_loop_input_from_xs(bs):
    """The input passed straight from the loop's own argument (for_loop(step, times,
    inputs) with N(inp)): taken from xs without calling the step per step, one launch per
    run of equal values; equals eager stepping and the oracle."""
    import torch
    print('[case] for_loop input from xs', flush=True)
    T = 200
    ref = _switch_oracle(T, 120, 20., 14.)
    inputs = torch.cat([torch.full((120,), 20.), torch.full((80,), 14.)])

    def make():
        net = _EINet(bs)

        def step(t, inp):
            spk = net.N.get_spike() != 0.
            net.E(spk[:net.n_exc])
            net.I(spk[net.n_exc:])
            return net.N(inp)
        return step, net
    res = []
    for fused in (False, True):
        bs.transform.fuse_loops = fused
        try:
            with bs.environ.context(dt=0.1):
                step, net = make()
                res.append((bs.transform.for_loop(step, torch.arange(T) * 0.1, inputs), net))
        finally:
            bs.transform.fuse_loops = True
        assert bs.transform.last_loop == ('fused' if fused else 'eager')
    for spikes, net in res:
        assert np.array_equal(spikes.cpu().numpy(), ref['raster'])
        assert np.array_equal(net.N.V.value.cpu().numpy(), ref['V'])


@pytest.mark.parametrize('kind', ['assign_state', 'state_as_input', 'reduce_spikes',
                                  'extra_module', 'late_change'])
def test_for_loop_steps_the_runner_cannot_take_stay_eager(bs, kind):
    """Steps with an effect the runner would not reproduce run eagerly and equal the loop
    stepped eagerly: a State assigned outside the modules (V clamped), the neuron's state fed
    back as its input, the spikes used for anything but the projections, another module
    called, and a step whose structure changes after some steps (an extra call from step 7)."""
    import torch
    print('[case] for_loop stays eager:', kind, flush=True)
    T = 40
    res = []
    for fused in (False, True):
        bs.transform.fuse_loops = fused
        try:
            with bs.environ.context(dt=0.1):
                net = _EINet(bs)
                other = bs.nn.LIFRef(10, V_initializer=0.)
                other.init_state()
                log = []

                def step(t):
                    spk = net.N.get_spike() != 0.
                    net.E(spk[:net.n_exc])
                    net.I(spk[net.n_exc:])
                    if kind == 'assign_state':
                        net.N.V.value = torch.clamp(net.N.V.value, max=-50.5)
                        out = net.N(20.)
                    elif kind == 'state_as_input':
                        out = net.N(net.N.V.value * 0. + 20.)
                    elif kind == 'reduce_spikes':
                        log.append(spk.sum())
                        out = net.N(20.)
                    elif kind == 'extra_module':
                        other(1.)
                        out = net.N(20.)
                    else:
                        if float(t) > 0.65:
                            other(1.)
                        out = net.N(20.)
                    return out

                res.append((bs.transform.for_loop(step, torch.arange(T) * 0.1), net))
        finally:
            bs.transform.fuse_loops = True
        assert bs.transform.last_loop == 'eager', kind
    (a, na), (b, nb) = res
    assert torch.equal(a, b)
    assert torch.equal(na.N.V.value, nb.N.V.value)


def _het_module_oracle(T):
    pe, pi, V0, p = make_golden.config1_het_net()
    p.deferred_reset = True
    return pe, pi, network.run_coba_lif(V0, pe, pi, p, 3200, T)


def test_for_loop_per_synapse_weights_4000(bs):
    """A module net with per-synapse weights N(0.6, 0.06) / N(6.7, 0.67) (the weights of the
    coba_lif_4000_het fixture): eager steps take the bucketed operator, whose fixed-point
    exponent is the runner's, so stepping eagerly, for_loop through the runner and the
    oracle's fixed-point sums agree bit for bit; eager stepping twice gives the same bits."""
    import torch
    print('[case] module net, per-synapse weights, 4000', flush=True)
    T = 300
    pe, pi, ref = _het_module_oracle(T)
    assert ref['counts'].sum() > 500

    def make():
        net = _EINet(bs, w_e=pe.w, w_i=pi.w)
        return net.update, net
    runs = _for_loop_paths(bs, make, T) + _for_loop_paths(bs, make, T)[:1]
    for spikes, net in runs:
        assert np.array_equal(spikes.cpu().numpy() != 0, ref['raster'])
        assert np.array_equal(net.N.V.value.cpu().numpy(), ref['V'])
        assert np.array_equal(net.E.syn.g.value.cpu().numpy(), ref['ge'])
        assert np.array_equal(net.I.syn.g.value.cpu().numpy(), ref['gi'])
    assert torch.equal(runs[0][0], runs[2][0])


def test_for_loop_per_synapse_weights_1m(bs):
    """The same at 1M neurons (K = 100, weights N(0.6, 0.06) / N(6.7, 0.67)): eager module
    steps, for_loop through the runner and the C restatement's fixed-point sums agree bit
    for bit over 60 steps."""
    import torch
    from oracle import cbuild
    print('[case] module net, per-synapse weights, 1M', flush=True)
    n, k, T = 1_000_000, 100, 60
    n_exc = n * 4 // 5
    V0 = np.random.RandomState(3).uniform(-60., -50., n).astype(F)
    rs = np.random.RandomState(8)
    w_e = rs.normal(0.6, 0.06, (n_exc, k)).astype(F)
    w_i = rs.normal(6.7, 0.67, (n - n_exc, k)).astype(F)

    def make():
        N = bs.nn.LIFRef(n, V_rest=-60., V_th=-50., V_reset=-60., tau=20., tau_ref=5.,
                         V_initializer=lambda s: V0)
        E = bs.nn.AlignPostProj(comm=bs.nn.EventFixedProb(n_exc, n, k, w_e, seed=1),
                                syn=bs.nn.Expon.desc(n, tau=5.), out=bs.nn.COBA.desc(E=0.),
                                post=N)
        I = bs.nn.AlignPostProj(comm=bs.nn.EventFixedProb(n - n_exc, n, k, w_i, seed=2),
                                syn=bs.nn.Expon.desc(n, tau=10.), out=bs.nn.COBA.desc(E=-80.),
                                post=N)
        for m in (E.syn, I.syn, N):
            m.init_state()

        def step(t):
            spk = N.get_spike() != 0.
            E(spk[:n_exc])
            I(spk[n_exc:])
            return N(20.)
        return step, (N, E)
    (eager, (Ne, Ee)), (fused, (Nf, Ef)) = _for_loop_paths(bs, make, T)
    idx_e = Ee.comm.conn.indices.cpu().numpy()
    idx_i = Ne._channels[1].comm.conn.indices.cpu().numpy()
    st = cbuild.lif_state(V0)
    c = np.zeros(T, np.int32)
    p = neuron.LIFParams(deferred_reset=True)
    cbuild.coba_lif_run(st, idx_e, idx_i, w_e, w_i, p, n_exc, T, counts=c)
    assert int(c.sum()) > T * 300
    assert eager.sum(1).cpu().numpy().tolist() == c.tolist()
    assert torch.equal(eager, fused)
    assert np.array_equal(Ne.V.value.cpu().numpy(), st['V'])
    assert np.array_equal(Nf.V.value.cpu().numpy(), st['V'])
    assert np.array_equal(Nf.spike.value.cpu().numpy().astype(np.uint8), st['spk'])


def test_deferred_reset_state_after_a_spike_step(bs):
    """LIFRef's default reset_timing='next' (brainpy.state's order): after a spike step V
    keeps the value that crossed V_th and get_spike() is set exactly where V >= V_th; the next
    step starts from V_reset (hard) or V - (V_th - V_reset) (soft).  reset_timing='same'
    gives V_reset right away, and both give the same spikes, conductances and refractory
    counts step by step; the oracle's deferred step gives the same V."""
    import torch
    print('[case] deferred reset', flush=True)
    n = 64
    V0 = np.linspace(-50.6, -49.9, n).astype(F)   # some cross V_th = -50 at once
    for soft in (False, True):
        kw = dict(V_rest=-60., V_th=-50., V_reset=-60., tau=20., tau_ref=0.3,
                  V_initializer=lambda s: V0, spk_reset='soft' if soft else 'hard')
        with bs.environ.context(dt=0.1):
            Nn = bs.nn.LIFRef(n, reset_timing='next', **kw)
            Ns = bs.nn.LIFRef(n, reset_timing='same', **kw)
            Nn.init_state()
            Ns.init_state()
            p = neuron.LIFParams(V_rest=-60., V_th=-50., V_reset=-60., tau=20., tau_ref=0.3,
                                 I_ext=15., spk_reset='soft' if soft else 'hard',
                                 deferred_reset=True)
            V, ge, gi, ref = V0.copy(), np.zeros(n, F), np.zeros(n, F), np.zeros(n, np.int32)
            spk = np.zeros(n, bool)
            seen = 0
            for t in range(12):
                sn, ss = Nn(15.), Ns(15.)
                V, ge, gi, ref, spk = neuron.coba_lif_step(V, ge, gi, ref, np.zeros(n, F),
                                                           np.zeros(n, F), p, spk)
                assert torch.equal(sn, ss) and torch.equal(Nn.ref.value, Ns.ref.value)
                s = sn.cpu().numpy()
                vn, vs = Nn.V.value.cpu().numpy(), Ns.V.value.cpu().numpy()
                assert np.array_equal(s, spk) and np.array_equal(vn, V)
                assert np.array_equal(Nn.get_spike().cpu().numpy(), s)
                assert np.all(vn[s] >= -50.) and np.all(vn[~s] == vs[~s])
                want = (vn[s] - F(10.)).astype(F) if soft else np.full(s.sum(), F(-60.))
                assert np.array_equal(vs[s], want)
                seen += int(s.sum())
            assert seen > n // 4


def test_array_tau_ref_counts_like_the_scalar(bs):
    """Per-neuron tau_ref arrays give the refractory steps of the scalar value (kept in
    float64 before dividing by dt): 0.3 ms and 4.9 ms at dt = 0.1 ms, 'open' and 'closed'."""
    from brainstate_amd import ops
    print('[case] tau_ref arrays', flush=True)
    with bs.environ.context(dt=0.1):
        for rule in ('open', 'closed'):
            for tr in (0.3, 0.6, 0.7, 1.1, 2.3, 4.9, 5.0):
                N = bs.nn.LIFRef(4, tau_ref=np.full(4, tr), ref_rule=rule)
                N.init_state()
                got = N._param_arrays(N.V.value)['ref_steps'].cpu().numpy()
                assert np.all(got == ops.refractory_steps(tr, 0.1, rule)), (rule, tr)


def test_fused_network_continues_eager_state(bs):
    import torch
    print('[case] module E/I net fused', flush=True)
    T = 300
    pe, pi, V0, p = make_golden.config1_net()
    p.deferred_reset = True
    ref = network.run_coba_lif(V0, pe, pi, p, 3200, T)
    with bs.environ.context(dt=0.1):
        net = _EINet(bs)
        r = bs.nn.fuse(net.N, net.E, net.I, n_exc=net.n_exc, inp=20.)
        raster = torch.zeros(T, net.num, dtype=torch.uint8, device='cuda')
        r.run(T, raster=raster)
        r.check()
        r.write_back()
    assert np.array_equal(raster.cpu().numpy().astype(bool), ref['raster'])
    assert np.array_equal(net.N.V.value.cpu().numpy(), ref['V'])
    assert np.array_equal(net.E.syn.g.value.cpu().numpy(), ref['ge'])



class _CUBANet:
    """examples/400_CUBA_2005_bpu.py:36-66: LIFRef with Expon synapses and CUBA outputs
    (scale 1 V), signed weights 1.62 / -9.0, external input 20."""

    def __init__(self, bs):
        c = make_golden.CUBA_NET
        self.bs = bs
        self.n_exc, self.num = c['n_exc'], c['n']
        V0 = np.random.RandomState(c['seed_v']).normal(-55., 2., c['n']).astype(F)
        self.N = bs.nn.LIFRef(self.num, V_rest=c['V_rest'], V_th=c['V_th'], V_reset=c['V_reset'],
                              tau=c['tau'], tau_ref=c['tau_ref'], V_initializer=lambda s: V0)
        self.E = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(self.n_exc, self.num, conn_num=c['p'],
                                      conn_weight=c['w_e'], seed=c['seed_e']),
            syn=bs.nn.Expon.desc(self.num, tau=5.), out=bs.nn.CUBA.desc(scale=1.0), post=self.N)
        self.I = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(self.num - self.n_exc, self.num, conn_num=c['p'],
                                      conn_weight=c['w_i'], seed=c['seed_i']),
            syn=bs.nn.Expon.desc(self.num, tau=10.), out=bs.nn.CUBA.desc(scale=1.0), post=self.N)
        for m in (self.E.syn, self.I.syn, self.N):
            m.init_state()

    def update(self, t):
        with self.bs.environ.context(t=t):
            spk = self.N.get_spike() != 0.
            self.E(spk[:self.n_exc])
            self.I(spk[self.n_exc:])
            self.N(make_golden.CUBA_NET['I_ext'])
            return self.N.get_spike()


def test_cuba_module_network_eager_and_fused(bs):
    """The reference's CUBA example through the module API: stepped eagerly (200 steps), and
    a fresh copy handed to the persistent runner with fuse() (500 steps).  Rasters and final
    states equal the oracle's."""
    import torch
    print('[case] module CUBA net eager + fused', flush=True)
    pe, pi, V0, p = make_golden.cuba_net()
    p.deferred_reset = True
    ref = network.run_coba_lif(V0, pe, pi, p, make_golden.CUBA_NET['n_exc'], 500)
    assert ref['counts'].sum() > 100
    def make():
        net = _CUBANet(bs)
        return net.update, net
    for spikes, _ in _for_loop_paths(bs, make, 200):
        assert np.array_equal(spikes.cpu().numpy() != 0, ref['raster'][:200])
    with bs.environ.context(dt=0.1):
        net = _CUBANet(bs)
        r = bs.nn.fuse(net.N, net.E, net.I, n_exc=net.n_exc, inp=make_golden.CUBA_NET['I_ext'])
        raster = torch.zeros(500, net.num, dtype=torch.uint8, device='cuda')
        r.run(500, raster=raster)
        r.check()
        r.write_back()
    assert np.array_equal(raster.cpu().numpy().astype(bool), ref['raster'])
    assert np.array_equal(net.N.V.value.cpu().numpy(), ref['V'])
    assert np.array_equal(net.I.syn.g.value.cpu().numpy(), ref['gi'])


def test_tutorial_network_modules_soft_reset(bs):
    """docs/tutorials/brain_dynamics/04_building_an_snn.ipynb cells 11-14 through the module
    API: LIF(spk_reset='soft') with Expon + CUBA projections, stepped eagerly (300 steps) and
    fused (the whole 2000 steps); both equal the oracle."""
    import torch
    print('[case] tutorial net modules', flush=True)
    c = make_golden.TUT_NET
    pe, pi, V0, p = make_golden.tut_net()
    p.deferred_reset = True
    ref = network.run_coba_lif(V0, pe, pi, p, c['n_exc'], c['steps'])

    def build():
        N = bs.nn.LIF(c['n'], V_rest=c['V_rest'], V_th=c['V_th'], V_reset=c['V_reset'],
                      tau=c['tau'], V_initializer=lambda s: V0, spk_reset='soft')
        E = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(c['n_exc'], c['n'], c['p'], c['w_e'], seed=c['seed_e']),
            syn=bs.nn.Expon.desc(c['n'], tau=c['tau_e']), out=bs.nn.CUBA.desc(), post=N)
        I = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(c['n'] - c['n_exc'], c['n'], c['p'], c['w_i'],
                                      seed=c['seed_i']),
            syn=bs.nn.Expon.desc(c['n'], tau=c['tau_i']), out=bs.nn.CUBA.desc(), post=N)
        for m in (E.syn, I.syn, N):
            m.init_state()
        return N, E, I

    def make():
        N, E, I = build()

        def step(t):
            spk = N.get_spike() != 0.
            E(spk[:c['n_exc']])
            I(spk[c['n_exc']:])
            return N(c['I_ext'])
        return step, N
    for spikes, N_ in _for_loop_paths(bs, make, c['steps']):
        assert np.array_equal(spikes.cpu().numpy() != 0, ref['raster'])
        assert np.array_equal(N_.V.value.cpu().numpy(), ref['V'])
    with bs.environ.context(dt=0.1):
        N, E, I = build()
        r = bs.nn.fuse(N, E, I, n_exc=c['n_exc'], inp=c['I_ext'])
        raster = torch.zeros(c['steps'], c['n'], dtype=torch.uint8, device='cuda')
        r.run(c['steps'], raster=raster)
        r.check()
        r.write_back()
    assert np.array_equal(raster.cpu().numpy().astype(bool), ref['raster'])
    assert np.array_equal(N.V.value.cpu().numpy(), ref['V'])


def test_cuba_and_coba_channels_do_not_mix(bs):
    with bs.environ.context(dt=0.1):
        N = bs.nn.LIFRef(10)
        bs.nn.AlignPostProj(comm=bs.nn.EventFixedProb(10, 10, conn_num=2, conn_weight=1.0,
                                                      seed=1),
                            syn=bs.nn.Expon.desc(10, tau=5.), out=bs.nn.CUBA.desc(), post=N)
        with pytest.raises(NotImplementedError):
            bs.nn.AlignPostProj(comm=bs.nn.EventFixedProb(10, 10, conn_num=2, conn_weight=1.0,
                                                          seed=2),
                                syn=bs.nn.Expon.desc(10, tau=5.), out=bs.nn.COBA.desc(E=0.),
                                post=N)

def test_hh_module_step_matches_oracle(bs):
    import torch
    print('[case] HH module', flush=True)
    n = 1000
    rng = np.random.RandomState(5)
    V0 = rng.uniform(-70, -50, n).astype(F)
    with bs.environ.context(dt=0.05):
        hh = bs.nn.HH(n, V_initializer=lambda s: V0)
        hh.init_state()
        out = []
        for _ in range(50):
            out.append(hh(6.5).cpu().numpy())
    V, m, h, nn_ = V0.copy(), *neuron.hh_init(V0)
    ge, gi = np.zeros(n, F), np.zeros(n, F)
    p = neuron.HHParams(I_ext=6.5, tau_e=1.0, tau_i=1.0)
    z = np.zeros(n, F)
    for t in range(50):
        V, m, h, nn_, ge, gi, spk = neuron.hh_step(V, m, h, nn_, ge, gi, z, z, p)
        assert np.array_equal(out[t], spk)
    assert np.array_equal(hh.V.value.cpu().numpy(), V)


def test_hh_single_neuron_trace_matches_fixture(bs):
    """examples/100_hh_neuron_model.py through the module API: 10 HH neurons, dt = 0.01 ms,
    10,000 steps of random input; the V trace and spike steps equal the committed fixture."""
    import hashlib
    import json
    import os
    import torch
    print('[case] HH single-neuron trace', flush=True)
    gold = json.load(open(os.path.join(GOLD, 'hh_single_trace.json')))
    c = gold['config']
    inp = np.random.RandomState(c['seed_in']).uniform(1., 10., c['steps']).astype(F)
    Vs, spk = [], []
    with bs.environ.context(dt=c['dt']):
        hh = bs.nn.HH(c['n'], V_initializer=c['V0'])
        hh.init_state()
        for t in range(c['steps']):
            spk.append(hh(float(inp[t]))[0].clone())
            Vs.append(hh.V.value[0].clone())   # the state tensor is updated in place
    trace = torch.stack(Vs).cpu().numpy()
    assert hashlib.sha256(trace.tobytes()).hexdigest() == gold['trace_sha256']
    assert np.flatnonzero(torch.stack(spk).cpu().numpy()).tolist() == gold['spikes']
    assert [float(v) for v in trace[999::1000]] == gold['V_every_1000']


@pytest.mark.parametrize('k,bucketed', [(50, False), (100, True)])
def test_event_fixed_prob_auto_homogeneous_choice(bs, k, bucketed):
    """'auto' with a homogeneous weight onto 200,000 neurons (17 buckets): the bucketed
    layout when a row averages at least 4 synapses per bucket (K >= 68), else the atomic
    kernel; both give the sequential scatter's sums of one repeated value."""
    import torch
    print('[case] auto homogeneous choice', k, flush=True)
    n_pre, n_post = 1000, 200_000
    auto = bs.nn.EventFixedProb(n_pre, n_post, conn_num=k, conn_weight=0.6, seed=7)
    spk = torch.from_numpy(np.random.RandomState(4).rand(n_pre) < 0.3).cuda()
    got = auto(spk).cpu().numpy()
    assert (auto._bucket is not None) == bucketed
    idx = auto.conn.indices.cpu().numpy()
    cnt = np.bincount(idx[spk.cpu().numpy()].reshape(-1), minlength=n_post)
    want = np.zeros(n_post, F)
    for c in range(1, int(cnt.max()) + 1):
        want = np.where(cnt >= c, (want + F(0.6)).astype(F), want).astype(F)
    assert np.array_equal(got, want)


@pytest.mark.parametrize('het,ratio', [(True, 1.0), (False, 1.0), (True, 0.6)])
def test_event_fixed_prob_bucketed_path(bs, het, ratio):
    """event_kernel='auto' on a wide output (> 16,384 posts) runs the bucketed operator; it
    matches the atomic path (bit for bit for a homogeneous weight, within the atomic-path
    tolerance otherwise), follows a new weight value, and autodiff still goes through the
    differentiable path."""
    import torch
    print('[case] event fixed prob bucketed', het, ratio, flush=True)
    n_pre, n_post = 3000, 40_000
    w = bs.nn.init.Normal(0.5, 0.1) if het else 0.6
    kw = dict(conn_num=0.002, conn_weight=w, seed=42, afferent_ratio=ratio)
    torch.manual_seed(0)
    auto = bs.nn.EventFixedProb(n_pre, n_post, **kw)
    atomic = bs.nn.EventFixedProb(n_pre, n_post, event_kernel='atomic', **kw)
    atomic.weight.value = auto.weight.value
    spk = torch.from_numpy(np.random.RandomState(3).rand(n_pre) < 0.2).cuda()
    a = auto(spk).cpu().numpy()
    assert auto._bucket is not None and atomic._bucket is None
    b = atomic(spk).cpu().numpy()
    if het:
        assert np.allclose(a, b, rtol=1e-5, atol=1e-6)
    else:
        assert np.array_equal(a, b)
    if het:  # a new weight value rebuilds the layout
        auto.weight.value = auto.weight.value * 2
        atomic.weight.value = auto.weight.value
        assert np.allclose(auto(spk).cpu().numpy(), atomic(spk).cpu().numpy(), rtol=1e-5,
                           atol=1e-6)
        wv = torch.as_tensor(np.asarray(auto.weight.value), dtype=torch.float32,
                             device='cuda').clone().requires_grad_(True)
        auto.weight.value = wv
        y = auto(spk.to(torch.float32))   # float spikes: value path, differentiable
        y.sum().backward()
        assert wv.grad is not None and torch.isfinite(wv.grad).all()
