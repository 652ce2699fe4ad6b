"""GPU: reverse and forward mode of the event operators against the oracle's float64
derivatives, and the reference's own gradient tests restated
(brainstate/nn/_event_fixedprob_test.py:56-126, brainstate/nn/_event_linear_test.py:42-125)."""
import numpy as np
import pytest

from oracle import event

pytestmark = pytest.mark.gpu
F = np.float32
RT, AT = 1e-5, 1e-5


@pytest.fixture(scope='module')
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail('GPU tests need a ROCm GPU')
    return torch


def say(*a):
    print('[case]', *a, flush=True)


def _net(seed, n_pre, n_post, k, p_spk, csr=False):
    rs = np.random.RandomState(seed)
    idx = rs.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = rs.randn(n_pre, k).astype(F)
    spk = (rs.rand(n_pre) < p_spk)
    g = rs.randn(n_post).astype(F)
    indptr = None
    if csr:  # drop some rows to get variable lengths
        keep = rs.rand(n_pre) < 0.7
        lens = np.where(keep, k, 0)
        indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        idx = idx[keep].reshape(-1)
        w = w[keep].reshape(-1)
    return rs, idx, w, spk, g, indptr


@pytest.mark.parametrize('csr', [False, True])
@pytest.mark.parametrize('homo', [False, True])
@pytest.mark.parametrize('dtype', ['bool', 'f32'])
def test_event_matvec_vjp_matches_oracle(torch_cuda, csr, homo, dtype):
    torch = torch_cuda
    from brainstate_amd import ops
    say('matvec vjp', csr, homo, dtype)
    rs, idx, w, spk, g, indptr = _net(7, 3000, 2000, 40, 0.1, csr)
    x = spk.astype(F) if dtype == 'f32' else spk
    wv = F(0.37) if homo else w
    tw = float(wv) if homo else torch.from_numpy(w).cuda()
    ti = torch.from_numpy(idx).cuda()
    tp = None if indptr is None else torch.from_numpy(indptr).cuda()
    gs, gw = ops.event_matvec_vjp(torch.from_numpy(np.asarray(x)).cuda(), ti, tw, 2000,
                                  torch.from_numpy(g).cuda(), k=40, indptr=tp)
    rx, rw = event.matvec_vjp(spk.astype(F), idx, wv, 2000, g, indptr=indptr)
    assert np.allclose(gs.cpu().numpy(), rx, rtol=RT, atol=AT)
    assert np.allclose(gw.cpu().numpy(), rw, rtol=RT, atol=1e-4 if homo else AT)


@pytest.mark.parametrize('homo', [False, True])
def test_value_matvec_matches_oracle(torch_cuda, homo):
    torch = torch_cuda
    from brainstate_amd import ops
    say('value matvec', homo)
    rs, idx, w, spk, g, _ = _net(11, 3000, 2000, 40, 0.3)
    x = (rs.randn(3000) * spk).astype(F)
    wv = F(-0.8) if homo else w
    out = ops.value_matvec(torch.from_numpy(x).cuda(), torch.from_numpy(idx).cuda(),
                           float(wv) if homo else torch.from_numpy(w).cuda(), 2000)
    assert np.allclose(out.cpu().numpy(), event.value_matvec(x, idx, wv, 2000), rtol=RT, atol=AT)


@pytest.mark.parametrize('shape', [(64, 512, 300), (5, 96, 64), (1, 33, 17), (70, 100, 160),
                                   (64, 1024, 4096)])
@pytest.mark.parametrize('dtype', ['bool', 'f32'])
def test_event_dense_vjp_matches_oracle(torch_cuda, shape, dtype):
    torch = torch_cuda
    from brainstate_amd import ops
    B, n_in, n_out = shape
    say('dense vjp', shape, dtype)
    rs = np.random.RandomState(3)
    spk = rs.rand(B, n_in) < 0.1
    x = (rs.rand(B, n_in) * spk).astype(F) if dtype == 'f32' else spk
    W = rs.randn(n_in, n_out).astype(F)
    g = rs.randn(B, n_out).astype(F)
    gs, gW = ops.event_dense_vjp(torch.from_numpy(np.asarray(x)).cuda(), torch.from_numpy(W).cuda(),
                                 torch.from_numpy(g).cuda())
    rx, rW = event.dense_vjp(np.asarray(x, F), W, g)
    # grad_spk sums n_out fp32 products in an unspecified order (the matrix-core path adds
    # 16-wide blocks per wave, then the waves' partials): its error is bounded by the fp32
    # rounding of such a sum, 4 sqrt(n_out) 2^-24 sum_j |g W| (a dropped block or a
    # transposed tile misses it by orders of magnitude), on top of rtol / 1e-4
    err = np.abs(gs.cpu().numpy() - rx)
    bound = 1e-4 + RT * np.abs(rx) + 4 * np.sqrt(n_out) * 2.0 ** -24 * (np.abs(g) @ np.abs(W).T)
    say('  grad_spk max error / bound', float((err / bound).max()))
    assert np.all(err <= bound)
    assert np.allclose(gW.cpu().numpy(), rW, rtol=RT, atol=AT)


# ---- the reference's module-level tests, restated ----

@pytest.mark.parametrize('homo_w', [True, False])
def test_event_fixedprob_vjp_reference(torch_cuda, homo_w):
    """brainstate/nn/_event_fixedprob_test.py:56-88."""
    torch = torch_cuda
    import brainstate_amd as bs
    say('fixedprob vjp', homo_w)
    n_in, n_out = 20, 30
    x = torch.from_numpy((np.random.RandomState(1).rand(n_in) < 0.3).astype(F)).cuda()
    w0 = 1.5 if homo_w else np.random.RandomState(2).uniform(-0.5, 0.5, (n_in, 3)).astype(F)
    fn = bs.nn.EventFixedProb(n_in, n_out, 0.1, w0, seed=123)
    w = torch.as_tensor(np.asarray(fn.weight.value, F)).cuda()

    def f(x, w):
        fn.weight.value = w
        return fn(x).sum()

    r = bs.transform.grad(f, argnums=(0, 1))(x, w)
    idx = fn.conn.indices.cpu().numpy()
    g = np.ones(n_out)
    rx, rw = event.matvec_vjp(x.cpu().numpy(), idx, float(w0) if homo_w else w0, n_out, g)
    assert np.allclose(r[0].cpu().numpy(), rx, rtol=RT, atol=AT)
    assert np.allclose(r[1].cpu().numpy(), rw, rtol=RT, atol=AT)


@pytest.mark.parametrize('homo_w', [True, False])
def test_event_fixedprob_jvp_reference(torch_cuda, homo_w):
    """brainstate/nn/_event_fixedprob_test.py:90-126 (forward mode, tangents of ones)."""
    torch = torch_cuda
    import brainstate_amd as bs
    say('fixedprob jvp', homo_w)
    n_in, n_out = 20, 30
    x = torch.from_numpy((np.random.RandomState(4).rand(n_in) < 0.3).astype(F)).cuda()
    w0 = 1.5 if homo_w else np.random.RandomState(5).uniform(-0.5, 0.5, (n_in, 3)).astype(F)
    fn = bs.nn.EventFixedProb(n_in, n_out, 0.1, w0, seed=123)
    w = torch.as_tensor(np.asarray(fn.weight.value, F)).cuda()

    def f(x, w):
        fn.weight.restore_value(w)
        return fn(x)

    o1, t1 = torch.func.jvp(f, (x, w), (torch.ones_like(x), torch.ones_like(w)))
    idx = fn.conn.indices.cpu().numpy()
    xn, wn = x.cpu().numpy(), (float(w0) if homo_w else w0)
    o2 = event.value_matvec(xn, idx, wn, n_out)
    t2 = event.matvec_jvp(xn, np.ones(n_in), idx, wn, 1.0 if homo_w else np.ones_like(w0), n_out)
    assert np.allclose(o1.cpu().numpy(), o2, rtol=RT, atol=AT)
    assert np.allclose(t1.cpu().numpy(), t2, rtol=1e-4, atol=1e-4)


def test_event_linear_grad_of_bool_raises(torch_cuda):
    """brainstate/nn/_event_linear_test.py:42-49: differentiating w.r.t. bool spikes fails."""
    torch = torch_cuda
    import brainstate_amd as bs
    fn = bs.nn.EventLinear(20, 30, np.random.RandomState(0).randn(20, 30).astype(F))
    x = torch.from_numpy(np.random.RandomState(1).rand(20) < 0.3).cuda()
    with pytest.raises(TypeError):
        bs.transform.grad(lambda x: fn(x).sum())(x)


@pytest.mark.parametrize('bool_x', [True, False])
@pytest.mark.parametrize('homo_w', [True, False])
def test_event_linear_vjp_reference(torch_cuda, bool_x, homo_w):
    """brainstate/nn/_event_linear_test.py:51-89: gradients of x @ W (x @ (ones * w))."""
    torch = torch_cuda
    import brainstate_amd as bs
    say('linear vjp', bool_x, homo_w)
    n_in, n_out = 20, 30
    rs = np.random.RandomState(6)
    xn = (rs.rand(n_in) < 0.3).astype(F) if bool_x else rs.rand(n_in).astype(F)
    w0 = 1.5 if homo_w else rs.uniform(-0.4, 0.4, (n_in, n_out)).astype(F)
    fn = bs.nn.EventLinear(n_in, n_out, w0, float_as_event=bool_x)
    w = torch.as_tensor(np.asarray(fn.weight.value, F)).cuda()

    def f(x, w):
        fn.weight.value = w
        return fn(x).sum()

    r = bs.transform.grad(f, argnums=(0, 1))(torch.from_numpy(xn).cuda(), w)
    Wd = np.ones((n_in, n_out)) * w0
    rx, rW = event.dense_vjp(xn[None], Wd, np.ones((1, n_out)))
    assert np.allclose(r[0].cpu().numpy(), rx[0], rtol=RT, atol=AT)
    want_w = rW.sum() if homo_w else rW
    assert np.allclose(r[1].cpu().numpy(), want_w, rtol=RT, atol=AT)


@pytest.mark.parametrize('bool_x', [True, False])
@pytest.mark.parametrize('homo_w', [True, False])
def test_event_linear_jvp_reference(torch_cuda, bool_x, homo_w):
    """brainstate/nn/_event_linear_test.py:91-125 (tangents of ones)."""
    torch = torch_cuda
    import brainstate_amd as bs
    say('linear jvp', bool_x, homo_w)
    n_in, n_out = 20, 30
    rs = np.random.RandomState(8)
    xn = (rs.rand(n_in) < 0.3).astype(F) if bool_x else rs.rand(n_in).astype(F)
    w0 = 1.5 if homo_w else rs.uniform(-0.4, 0.4, (n_in, n_out)).astype(F)
    fn = bs.nn.EventLinear(n_in, n_out, w0, float_as_event=bool_x)
    w = torch.as_tensor(np.asarray(fn.weight.value, F)).cuda()

    def f(x, w):
        fn.weight.restore_value(w)
        return fn(x)

    x = torch.from_numpy(xn).cuda()
    o1, t1 = torch.func.jvp(f, (x, w), (torch.ones_like(x), torch.ones_like(w)))
    Wd = np.ones((n_in, n_out)) * w0
    o2 = xn.astype(np.float64) @ Wd
    t2 = np.ones(n_in) @ Wd + xn.astype(np.float64) @ (np.ones((n_in, n_out)) if not homo_w
                                                        else np.ones((n_in, n_out)))
    assert np.allclose(o1.cpu().numpy(), o2, rtol=RT, atol=AT)
    assert np.allclose(t1.cpu().numpy(), t2, rtol=RT, atol=1e-4)


@pytest.mark.parametrize('homo_w', [True, False])
def test_fixednumconn_value_inputs(torch_cuda, homo_w):
    """FixedNumConn.update on float inputs is the value-weighted mat-vec x @ conn
    (brainstate/nn/_event_fixedprob.py:202-209); EventFixedNumConn counts events instead."""
    torch = torch_cuda
    import brainstate_amd as bs
    say('fixednumconn values', homo_w)
    rs = np.random.RandomState(12)
    w0 = 0.7 if homo_w else rs.randn(200, 20).astype(F)
    fn = bs.nn.FixedNumConn(200, 150, 20, w0, seed=9)
    xn = (rs.randn(200) * (rs.rand(200) < 0.3)).astype(F)
    y = fn(torch.from_numpy(xn).cuda())
    want = event.value_matvec(xn, fn.conn.indices.cpu().numpy(), w0, 150)
    assert np.allclose(y.detach().cpu().numpy(), want, rtol=RT, atol=AT)
    ev = bs.nn.EventFixedNumConn(200, 150, 20, w0, seed=9)(torch.from_numpy(xn).cuda())
    want_ev = event.value_matvec((xn != 0).astype(F), fn.conn.indices.cpu().numpy(), w0, 150)
    assert np.allclose(ev.detach().cpu().numpy(), want_ev, rtol=RT, atol=AT)
