"""GPU tests of batched simulation: the batched event / value mat-vec kernels
(bs_event_matvec_batch_f32, bs_value_matvec_batch_f32), module nets initialised with
init_all_states(batch_size=B) (states [B, n]), and their fusion into one runner over the
block-diagonal union of the replicas -- every replica against its own oracle run."""
import os
import sys

import numpy as np
import pytest

from oracle import event, network

pytestmark = pytest.mark.gpu
F = np.float32
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


def say(*a):
    print('[case]', *a, flush=True)


@pytest.mark.parametrize('homo,csr', [(True, False), (False, False), (True, True), (False, True)])
def test_batched_event_matvec_rows(bs, homo, csr):
    import torch
    say('batched matvec', homo, csr)
    rs = np.random.RandomState(3)
    B, n_pre, n_post, k = 37, 3000, 2500, 40
    idx = rs.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = F(0.7) if homo else rs.randn(n_pre, k).astype(F)
    spk = rs.rand(B, n_pre) < 0.05
    dev = torch.device('cuda')
    it = torch.from_numpy(idx).to(dev)
    wt = w if homo else torch.from_numpy(w).to(dev)
    if csr:
        indptr = torch.arange(0, (n_pre + 1) * k, k, dtype=torch.int32, device=dev)
        out = bs.ops.event_matvec(torch.from_numpy(spk).to(dev), it.reshape(-1), wt if homo
                                  else wt.reshape(-1), n_post, indptr=indptr)
    else:
        out = bs.ops.event_matvec(torch.from_numpy(spk).to(dev), it, wt, n_post)
    assert tuple(out.shape) == (B, n_post)
    got = out.cpu().numpy()
    for b in range(B):
        want = event.scatter_fixed(spk[b], idx, w, n_post)
        if homo:
            assert np.array_equal(got[b], want), b
        else:
            assert np.allclose(got[b], want, rtol=1e-5, atol=1e-6), b
    x = (rs.randn(B, n_pre) * (rs.rand(B, n_pre) < 0.1)).astype(F)
    outv = bs.ops.value_matvec(torch.from_numpy(x).to(dev), it, wt, n_post).cpu().numpy()
    for b in range(B):
        assert np.allclose(outv[b], event.value_matvec(x[b], idx, w, n_post), rtol=1e-5,
                           atol=1e-5), b


def test_batched_module_and_gradients(bs):
    """EventFixedProb on [B, n_pre] inputs (one launch) equals its rows; the batched VJP /
    JVP equal the sums of the per-row derivatives."""
    import torch
    say('batched module grads')
    rs = np.random.RandomState(4)
    B, n_pre, n_post = 6, 400, 300
    m = bs.nn.EventFixedProb(n_pre, n_post, 20, rs.randn(n_pre, 20).astype(F), seed=5)
    x = torch.from_numpy((rs.rand(B, n_pre) < 0.2).astype(F)).cuda().requires_grad_(True)
    y = m(x)
    rows = torch.stack([m(x[b]) for b in range(B)])
    assert torch.allclose(y, rows, rtol=1e-5, atol=1e-6)
    g = torch.from_numpy(rs.randn(B, n_post).astype(F)).cuda()
    gx, = torch.autograd.grad((y * g).sum(), x)
    for b in range(B):
        gxb, = torch.autograd.grad((m(x[b]) * g[b]).sum(), x)
        assert torch.allclose(gx[b], gxb[b], rtol=1e-5, atol=1e-5)
    xs = (rs.rand(B, n_pre) < 0.2).astype(F)
    w = m.weight.value
    w = w.detach().cpu().numpy() if torch.is_tensor(w) else np.asarray(w, F)
    fn = lambda xx: m(xx)                      # noqa: E731
    t = torch.from_numpy(rs.randn(B, n_pre).astype(F)).cuda()
    _, jv = torch.func.jvp(fn, (torch.from_numpy(xs).cuda(),), (t,))
    want = np.stack([event.value_matvec(t[b].cpu().numpy(), m.conn.indices.cpu().numpy(),
                                        w, n_post) for b in range(B)])
    assert np.allclose(jv.cpu().numpy(), want, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize('het,csr,sdt', [(True, False, 'u8'), (True, True, 'f32'),
                                         (False, False, 'u8'), (True, False, 'f32')])
def test_batched_vjp_kernel_equals_rows(bs, het, csr, sdt):
    """bs_event_matvec_vjp_batch_f32: grad_spk row b equals bs_event_matvec_vjp_f32 on row b
    bit for bit, and per-synapse grad_w equals the per-row gradients added in row order (bit
    for bit); a homogeneous grad_w equals their sum within fp32 rounding."""
    import torch
    from brainstate_amd import ops
    say('batched vjp kernel', het, csr, sdt)
    rs = np.random.RandomState(9)
    B, n_pre, n_post, k = 7, 3000, 2500, 40
    idx = rs.randint(-3, n_post, (n_pre, k)).astype(np.int32)   # a few out-of-range targets
    indptr = None
    if csr:
        lens = rs.randint(0, 2 * k, n_pre)
        indptr = torch.as_tensor(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32),
                                 device='cuda')
        idx = rs.randint(0, n_post, int(lens.sum())).astype(np.int32)
    d_idx = torch.as_tensor(idx, device='cuda')
    w = torch.as_tensor(rs.randn(*idx.shape).astype(F), device='cuda') if het else \
        torch.tensor(0.7, device='cuda')
    act = rs.rand(B, n_pre) < 0.3
    spk = torch.as_tensor(act.astype(np.uint8) if sdt == 'u8' else
                          np.where(act, rs.rand(B, n_pre), 0).astype(F), device='cuda')
    g = torch.as_tensor(rs.randn(B, n_post).astype(F), device='cuda')
    gs, gw = ops.event_matvec_vjp_batch(spk, d_idx, w, n_post, g, indptr=indptr)
    gw_sum = None
    for b in range(B):
        gs_b, gw_b = ops.event_matvec_vjp(spk[b], d_idx, w, n_post, g[b].contiguous(),
                                          indptr=indptr)
        assert torch.equal(gs[b], gs_b), b
        gw_sum = gw_b if gw_sum is None else gw_sum + gw_b
    if het:
        assert torch.equal(gw, gw_sum)
    else:
        assert torch.allclose(gw, gw_sum, rtol=1e-5)
    assert float(gs.abs().sum()) > 0


class _BatchedEINet:
    """Config [1]'s E/I net (examples/105_COBA_HH_2007_braincell.py:54-82) with states
    [B, n]: replica b starts from its own V0."""

    def __init__(self, bs, V0s, w_e=0.6, w_i=6.7):
        c = make_golden.CONFIG1
        self.bs = bs
        self.n_exc, self.num = c['n_exc'], c['n']
        self.N = bs.nn.LIFRef(self.num, V_rest=-60., V_th=-50., V_reset=-60., tau=20.,
                              tau_ref=5., V_initializer=V0s)
        self.E = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(self.n_exc, self.num, conn_num=0.02, conn_weight=w_e,
                                      seed=c['seed_e']),
            syn=bs.nn.Expon.desc(self.num, tau=5.), out=bs.nn.COBA.desc(E=0.), post=self.N)
        self.I = bs.nn.AlignPostProj(
            comm=bs.nn.EventFixedProb(self.num - self.n_exc, self.num, conn_num=0.02,
                                      conn_weight=w_i, seed=c['seed_i']),
            syn=bs.nn.Expon.desc(self.num, tau=10.), out=bs.nn.COBA.desc(E=-80.), post=self.N)
        for m in (self.E.syn, self.I.syn, self.N):
            m.init_state(batch_size=V0s.shape[0])

    def update(self, t):
        with self.bs.environ.context(t=t):
            spk = self.N.get_spike() != 0.
            self.E(spk[..., :self.n_exc])
            self.I(spk[..., self.n_exc:])
            self.N(20.)
            return self.N.get_spike()


def _replica_V0(B):
    return np.stack([np.random.RandomState(300 + b).uniform(-60., -50., 4000).astype(F)
                     for b in range(B)])


def test_batched_module_net_eager(bs):
    import torch
    B, T = 4, 150
    say('batched module net eager', B, T)
    V0s = _replica_V0(B)
    pe, pi, _, p = make_golden.config1_net()
    p.deferred_reset = True   # LIFRef's default reset_timing='next'
    with bs.environ.context(dt=0.1):
        net = _BatchedEINet(bs, V0s)
        assert tuple(net.N.V.value.shape) == (B, 4000)
        spikes = bs.transform.for_loop(net.update, torch.arange(T) * 0.1).cpu().numpy()
    assert spikes.shape == (T, B, 4000)
    for b in range(B):
        ref = network.run_coba_lif(V0s[b], pe, pi, p, 3200, T)
        assert np.array_equal(spikes[:, b], ref['raster']), b
        assert np.array_equal(net.N.V.value[b].cpu().numpy(), ref['V']), b


def test_batched_net_fused_union_runner(bs):
    import torch
    B, T = 8, 300
    say('batched fused union', B, T)
    V0s = _replica_V0(B)
    pe, pi, _, p = make_golden.config1_net()
    p.deferred_reset = True
    with bs.environ.context(dt=0.1):
        net = _BatchedEINet(bs, V0s)
        r = bs.nn.fuse(net.N, net.E, net.I, n_exc=3200, inp=20.)
        assert r.n == B * 4000
        raster = torch.zeros(T, B * 4000, dtype=torch.uint8, device='cuda')
        r.run(T, raster=raster)
        r.check()
        r.write_back()
    ras = raster.cpu().numpy().astype(bool)[:, r.replica_index]   # [T, B, n]
    for b in range(B):
        ref = network.run_coba_lif(V0s[b], pe, pi, p, 3200, T)
        assert np.array_equal(ras[:, b], ref['raster']), b
        assert np.array_equal(net.N.V.value[b].cpu().numpy(), ref['V']), b
        assert np.array_equal(net.E.syn.g.value[b].cpu().numpy(), ref['ge']), b


def test_batched_net_per_replica_input(bs):
    """A sweep over the drive: replica b gets its own external input (N(x) with x of shape
    [B, 1], broadcast over its neurons) -- eager for_loop, the loop handed to the union runner,
    and fuse() with the array; every replica equals its own oracle run with that input."""
    import torch
    from oracle import neuron
    B, T = 4, 200
    say('batched net, per-replica input', B, T)
    V0s = _replica_V0(B)
    pe, pi, _, _ = make_golden.config1_net()
    I = np.array([16., 19., 22., 25.], F)[:, None]
    dI = torch.as_tensor(I, device='cuda')
    refs = [network.run_coba_lif(V0s[b], pe, pi,
                                 neuron.LIFParams(I_ext=I[b, 0], deferred_reset=True), 3200, T)
            for b in range(B)]
    assert len({int(r['counts'].sum()) for r in refs}) == B   # the inputs matter
    for fused in (False, True):
        bs.transform.fuse_loops = fused
        try:
            with bs.environ.context(dt=0.1):
                net = _BatchedEINet(bs, V0s)

                def step(t):
                    spk = net.N.get_spike() != 0.
                    net.E(spk[..., :net.n_exc])
                    net.I(spk[..., net.n_exc:])
                    return net.N(dI)
                spikes = bs.transform.for_loop(step, torch.arange(T) * 0.1).cpu().numpy()
        finally:
            bs.transform.fuse_loops = True
        assert bs.transform.last_loop == ('fused' if fused else 'eager')
        for b in range(B):
            assert np.array_equal(spikes[:, b] != 0, refs[b]['raster']), (fused, b)
            assert np.array_equal(net.N.V.value[b].cpu().numpy(), refs[b]['V']), (fused, b)
    with bs.environ.context(dt=0.1):
        net = _BatchedEINet(bs, V0s)
        r = bs.nn.fuse(net.N, net.E, net.I, n_exc=3200, inp=dI)
        r.run(T)
        r.check()
        r.write_back()
    for b in range(B):
        assert np.array_equal(net.N.V.value[b].cpu().numpy(), refs[b]['V']), b


def test_batched_net_per_synapse_weights(bs):
    """Replicas sharing per-synapse weights N(0.6, 0.06) / N(6.7, 0.67): the eager batched step
    takes the bucketed operator row by row (the runner's fixed-point sums), so stepping eagerly,
    for_loop through the union runner and each replica's oracle run agree bit for bit."""
    import torch
    B, T = 3, 200
    say('batched net, per-synapse weights', B, T)
    V0s = _replica_V0(B)
    pe, pi, _, p = make_golden.config1_het_net()
    p.deferred_reset = True
    refs = [network.run_coba_lif(V0s[b], pe, pi, p, 3200, T) for b in range(B)]
    assert all(int(r['counts'].sum()) > 300 for r in refs)
    out = {}
    for fused in (False, True):
        bs.transform.fuse_loops = fused
        try:
            with bs.environ.context(dt=0.1):
                net = _BatchedEINet(bs, V0s, w_e=pe.w, w_i=pi.w)
                spikes = bs.transform.for_loop(net.update, torch.arange(T) * 0.1)
        finally:
            bs.transform.fuse_loops = True
        assert bs.transform.last_loop == ('fused' if fused else 'eager')
        out[fused] = spikes
        for b in range(B):
            assert np.array_equal(spikes[:, b].cpu().numpy() != 0, refs[b]['raster']), (fused, b)
            assert np.array_equal(net.N.V.value[b].cpu().numpy(), refs[b]['V']), (fused, b)
            assert np.array_equal(net.I.syn.g.value[b].cpu().numpy(), refs[b]['gi']), (fused, b)
    assert torch.equal(out[False], out[True])


def test_batched_for_loop_chunks_reuse_the_runner(bs):
    """A batched net (B = 3 replicas, one union runner) run in three for_loop chunks keeps
    its runner between them and equals the same chunks stepped eagerly."""
    import torch
    B = 3
    say('batched for_loop chunks', B)
    res = []
    for fused in (False, True):
        bs.transform.fuse_loops = fused
        try:
            with bs.environ.context(dt=0.1):
                net = _BatchedEINet(bs, _replica_V0(B))
                outs, runners = [], []
                for T in (50, 30, 40):
                    outs.append(bs.transform.for_loop(net.update, torch.arange(T) * 0.1))
                    assert bs.transform.last_loop == ('fused' if fused else 'eager')
                    r = getattr(net.N, '_fused_runner', None)
                    runners.append(None if r is None else r[1])
                if fused:
                    assert runners[0] is runners[1] is runners[2]
                res.append((torch.cat(outs), net))
        finally:
            bs.transform.fuse_loops = True
    (a, na), (b, nb) = res
    assert int(a.sum()) > 0
    assert torch.equal(a, b)
    assert torch.equal(na.N.V.value, nb.N.V.value)
    assert torch.equal(na.I.syn.g.value, nb.I.syn.g.value)
