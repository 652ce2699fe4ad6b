"""GPU parity of the packed EventLinear product (bs_event_dense_pack, bs_event_dense_packed_f32)
against the oracle's per-column fixed-point restatement (bit-exact) and the sequential fp32
sum of brainstate/nn/_event_linear.py:99-100 (rtol 1e-5, atol 1e-6 scaled by the largest
weight)."""
import sys

import numpy as np
import pytest

from oracle import event

pytestmark = pytest.mark.gpu

F = np.float32


@pytest.fixture(scope='module')
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail('GPU tests need a ROCm GPU')
    from brainstate_amd import _native
    _native.load_library()
    return torch


def say(*a):
    print('[case]', *a, flush=True)
    sys.stdout.flush()


def dev(t, a):
    return t.from_numpy(np.ascontiguousarray(a)).cuda()


def run(torch, spk, W):
    from brainstate_amd import ops
    P = ops.pack_dense(dev(torch, W))
    return P, ops.event_dense_packed(dev(torch, spk), P).cpu().numpy()


@pytest.mark.parametrize('B,n_in,n_out,p,sdt', [
    (1, 64, 16, 0.3, 'u8'), (3, 17, 5, 0.5, 'u8'), (64, 4096, 4096, 0.05, 'u8'),
    (65, 100, 33, 0.2, 'u8'), (130, 1000, 257, 0.05, 'bool'), (5, 20000, 70, 0.02, 'u8'),
    (7, 96, 40, 0.4, 'f32'), (64, 512, 256, 0.05, 'f32'), (2, 65536, 16, 0.01, 'u8'),
    (16, 1, 3, 0.9, 'u8')])
def test_packed_matches_oracle(torch_cuda, B, n_in, n_out, p, sdt):
    """Bit-exact against the fixed-point restatement; within tolerance of the sequential
    fp32 sum.  Byte spikes hold values other than 1 and float spikes arbitrary nonzero
    values: any nonzero is one event."""
    torch = torch_cuda
    say('packed', B, n_in, n_out, p, sdt)
    rng = np.random.RandomState(B + n_in + n_out)
    W = rng.normal(0, 0.125, (n_in, n_out)).astype(F)
    s = rng.rand(B, n_in) < p
    if sdt == 'u8':
        spk = s.astype(np.uint8) * rng.randint(1, 256, (B, n_in)).astype(np.uint8)
    elif sdt == 'bool':
        spk = s
    else:
        spk = np.where(s, rng.normal(0, 2, (B, n_in)), 0).astype(F)
        spk[s & (spk == 0)] = 1.0
    P, got = run(torch, spk, W)
    assert P['finite'] and P['L'] == event.dense_digits(n_in)
    want = event.event_dense_fixed_point(spk, W)
    assert np.array_equal(got, want)
    if n_in * B <= 200_000:
        seq = event.event_linear(spk != 0, W)
        assert np.allclose(got, seq, rtol=1e-5, atol=1e-6 * float(np.abs(W).max()))


def test_packed_unaligned_spikes_and_repack(torch_cuda):
    """A spike view that starts one byte into its buffer (byte-load path) gives the same
    bits; packing a second W into the same buffer leaves nothing of the first behind."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('packed unaligned + repack')
    rng = np.random.RandomState(3)
    B, n_in, n_out = 9, 640, 48
    W1 = rng.normal(0, 1, (n_in, n_out)).astype(F)
    W2 = (rng.normal(0, 1e-3, (n_in, n_out)) * (rng.rand(n_in, n_out) < 0.5)).astype(F)
    spk = (rng.rand(B, n_in) < 0.2).astype(np.uint8)
    raw = torch.zeros(B * n_in + 1, dtype=torch.uint8, device='cuda')
    raw[1:] = dev(torch, spk.reshape(-1))
    view = raw[1:].view(B, n_in)
    P = ops.pack_dense(dev(torch, W1))
    got1 = ops.event_dense_packed(view, P).cpu().numpy()
    assert np.array_equal(got1, event.event_dense_fixed_point(spk, W1))
    buf = P['packed']
    from brainstate_amd import _native as N
    N.check(N.lib().bs_event_dense_pack(N.ptr(dev(torch, W2)), n_in, n_out, N.ptr(buf),
                                        buf.numel(), N.stream_handle(buf.device)), 'pack')
    got2 = ops.event_dense_packed(dev(torch, spk), P).cpu().numpy()
    assert np.array_equal(got2, event.event_dense_fixed_point(spk, W2))
    again = ops.event_dense_packed(dev(torch, spk), P).cpu().numpy()
    assert np.array_equal(got2, again)


def test_packed_column_scales_zero_columns_and_ties(torch_cuda):
    """Columns 2^60 apart keep their own scale; a column of zeros gives +0; the half-way
    weights of the oracle's tie pins round to even on the device too."""
    torch = torch_cuda
    say('packed scales')
    rng = np.random.RandomState(8)
    n_in, n_out, B = 64, 20, 6
    W = rng.normal(0, 1, (n_in, n_out)).astype(F)
    W[:, 1] *= F(2.0 ** -60)
    W[:, 2] *= F(2.0 ** 60)
    W[:, 3] = 0
    W[:, 4] = 0
    W[:4, 4] = [1.0, 2.0 ** -30, 3 * 2.0 ** -30, 5 * 2.0 ** -30]
    W[:, 5] = rng.normal(0, 1, n_in).astype(F) * F(1e-40)  # subnormal column
    spk = (rng.rand(B, n_in) < 0.5).astype(np.uint8)
    spk[0, :4] = [0, 1, 0, 0]
    spk[1, :4] = [0, 0, 1, 0]
    spk[2, :4] = [0, 0, 0, 1]
    _, got = run(torch, spk, W)
    want = event.event_dense_fixed_point(spk, W)
    assert np.array_equal(got, want)
    assert np.all(got[:, 3] == 0) and not np.any(np.signbit(got[:, 3]))
    assert got[0, 4] == 0.0 and got[1, 4] == F(2.0 ** -28) and got[2, 4] == F(2.0 ** -28)


def test_packed_non_finite_weight_flags(torch_cuda):
    """A weight that is inf or NaN sets the status word; every output is then NaN."""
    torch = torch_cuda
    say('packed non-finite')
    rng = np.random.RandomState(2)
    W = rng.normal(0, 1, (128, 32)).astype(F)
    W[5, 7] = np.inf
    spk = (rng.rand(4, 128) < 0.3).astype(np.uint8)
    P, got = run(torch, spk, W)
    assert not P['finite'] and np.all(np.isnan(got))


def test_packed_empty_shapes(torch_cuda):
    """n_in = 0 gives zeros; batch 0 writes nothing."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('packed empty')
    P = ops.pack_dense(torch.zeros(0, 7, device='cuda'))
    out = ops.event_dense_packed(torch.zeros(3, 0, dtype=torch.uint8, device='cuda'), P)
    assert out.shape == (3, 7) and torch.all(out == 0)
    P = ops.pack_dense(dev(torch, np.ones((32, 16), F)))
    out = ops.event_dense_packed(torch.zeros(0, 32, dtype=torch.uint8, device='cuda'), P)
    assert out.shape == (0, 16)


def test_event_linear_module_routes(torch_cuda):
    """nn.EventLinear ('auto') uses the packed form for event inputs without autodiff,
    repacks when a torch weight changes in place, and streams value inputs or on request."""
    torch = torch_cuda
    import brainstate_amd as bs
    say('EventLinear routes')
    rng = np.random.RandomState(12)
    W = rng.normal(0, 0.125, (512, 256)).astype(F)
    spk = rng.rand(64, 512) < 0.05
    m = bs.nn.EventLinear(512, 256, dev(torch, W))
    x = torch.tensor(spk, device='cuda')
    with torch.no_grad():
        y = m(x).cpu().numpy()
    assert np.array_equal(y, event.event_dense_fixed_point(spk, W))
    with torch.no_grad():
        m.weight.value.mul_(2.0)   # in place: version bump -> repack
        y2 = m(x).cpu().numpy()
    assert np.array_equal(y2, event.event_dense_fixed_point(spk, W * 2))
    for it in range(3):   # a new tensor each time, the previous one released
        m.weight.value = dev(torch, W * F(it + 3))
        with torch.no_grad():
            y3 = m(x).cpu().numpy()
        assert np.array_equal(y3, event.event_dense_fixed_point(spk, W * F(it + 3)))
    s = bs.nn.EventLinear(512, 256, W, event_kernel='stream')
    with torch.no_grad():
        ys = s(x).cpu().numpy()
    from brainstate_amd import ops
    _, L = ops.event_dense_chunks(64, 512, 256)
    assert np.array_equal(ys, event.event_linear(spk, W, chunk_rows=L))
    v = bs.nn.EventLinear(512, 256, W, float_as_event=False)
    xf = np.where(spk, 0.5, 0).astype(F)
    with torch.no_grad():
        yv = v(dev(torch, xf)).cpu().numpy()
    assert np.array_equal(yv, event.event_linear(xf, W, float_as_event=False, chunk_rows=L))


@pytest.mark.parametrize('inh', [False, True])
def test_fused_lif_step_recurrent(torch_cuda, inh):
    """Four recurrent steps (the spikes of one step are the next step's input) of the fused
    packed EventLinear + COBA-LIF launch equal, bit for bit, the oracle's fixed-point product
    followed by its COBA-LIF step, and the unfused pair of device calls."""
    torch = torch_cuda
    from brainstate_amd import ops
    from oracle import neuron
    say('fused lif step', inh)
    rng = np.random.RandomState(31 + inh)
    B, n = 70, 512
    W = rng.normal(0.4 if not inh else 0.8, 0.3, (n, n)).astype(F)
    spk = rng.rand(B, n) < 0.1
    V = rng.uniform(-60, -50, (B, n)).astype(F).reshape(-1)
    ge = np.zeros(B * n, F)
    gi = np.zeros(B * n, F)
    ref = rng.choice([0, 0, 0, 2], B * n).astype(np.int32)
    p = neuron.LIFParams()
    P = ops.pack_dense(dev(torch, W))
    dV, dge, dgi, dref = (dev(torch, a) for a in (V, ge, gi, ref))
    uV, uge, ugi, uref = (dev(torch, a) for a in (V, ge, gi, ref))
    x = dev(torch, spk.astype(np.uint8))
    ux = x.clone()
    fired = 0
    for step in range(4):
        cur = event.event_dense_fixed_point(spk, W).reshape(-1)
        z = np.zeros_like(cur)
        V, ge, gi, ref, s_new = neuron.coba_lif_step(V, ge, gi, ref, z if inh else cur,
                                                     cur if inh else z, p)
        cur_d = torch.empty(B, n, device='cuda')
        spk_d = torch.empty(B, n, dtype=torch.uint8, device='cuda')
        ops.event_dense_packed_lif_step(x, P, dV, dge, dgi, dref, ops.lif_params(), inh=inh,
                                        cur_out=cur_d, spk_out=spk_d)
        ucur = ops.event_dense_packed(ux, P)
        zero = torch.zeros_like(ucur)
        us = ops.coba_lif_step(uV, uge, ugi, uref, (zero if inh else ucur).view(-1),
                               (ucur if inh else zero).view(-1), ops.lif_params())
        assert np.array_equal(cur_d.cpu().numpy().reshape(-1), cur)
        for d, e in ((dV, V), (dge, ge), (dgi, gi), (dref, ref)):
            assert np.array_equal(d.cpu().numpy(), e)
        for d, u in ((dV, uV), (dge, uge), (dgi, ugi), (dref, uref)):
            assert torch.equal(d, u)
        assert np.array_equal(spk_d.cpu().numpy().reshape(-1).astype(bool), s_new)
        assert torch.equal(spk_d.view(-1), us)
        spk = s_new.reshape(B, n)
        x, ux = spk_d, us.view(B, n)
        fired += int(s_new.sum())
    assert fired > 100 or inh


def test_packed_config4_against_float64_sum(torch_cuda):
    """Config [4] (spikes [64, 4096] at 5 %, W [4096, 4096] ~ N(0, 1/64)): every output within
    abs 1e-6 + rel 1e-5 of the float64 sum (the north_star tolerance, fixed, not scaled by
    max|W|), and within the packed form's own bound 2^-24 max|W[:, j]| + half an ulp."""
    torch = torch_cuda
    say('packed config [4] vs float64')
    rng = np.random.RandomState(11)
    W = rng.normal(0, 0.125, (4096, 4096)).astype(F)
    spk = (rng.rand(64, 4096) < 0.05).astype(np.uint8)
    _, got = run(torch, spk, W)
    exact = (spk != 0).astype(np.float64) @ W.astype(np.float64)
    err = np.abs(got.astype(np.float64) - exact)
    assert np.all(err <= 1e-6 + 1e-5 * np.abs(exact))
    bound = 2.0 ** -24 * np.abs(W).max(0)[None, :] + 0.5 * np.spacing(np.abs(exact).astype(F))
    assert np.all(err <= bound)


def test_packed_lif_step_rejects_overlapping_outputs(torch_cuda):
    """An output that shares memory with the spike input is refused by the wrapper and by
    the C entry point (workgroups would read spikes another one already overwrote)."""
    torch = torch_cuda
    from brainstate_amd import _native as N
    from brainstate_amd import ops
    say('packed lif step overlap')
    B, n = 4, 64
    W = torch.from_numpy(np.random.RandomState(2).normal(0, 0.1, (n, n)).astype(F)).cuda()
    P = ops.pack_dense(W)
    buf = torch.zeros(B, n, dtype=torch.uint8, device='cuda')
    V = torch.full((B * n,), -60.0, device='cuda')
    ge, gi = torch.zeros(B * n, device='cuda'), torch.zeros(B * n, device='cuda')
    ref = torch.zeros(B * n, dtype=torch.int32, device='cuda')
    with pytest.raises(ValueError):
        ops.event_dense_packed_lif_step(buf, P, V, ge, gi, ref, ops.lif_params(), spk_out=buf)
    rc = N.lib().bs_event_dense_packed_lif_step(
        N.ptr(buf), N.BS_SPK_U8, B, n, N.ptr(P['packed']), n, 0, N.ptr(V), N.ptr(ge), N.ptr(gi),
        N.ptr(ref), ops.ctypes_ref(ops.lif_params()), None, N.ptr(buf),
        N.stream_handle(buf.device))
    assert rc == N.BS_ERR_INVALID and b'overlaps' in N.lib().bs_last_error()
    out = torch.empty(B, n, dtype=torch.uint8, device='cuda')
    ops.event_dense_packed_lif_step(buf, P, V, ge, gi, ref, ops.lif_params(), spk_out=out)
    torch.cuda.synchronize()
