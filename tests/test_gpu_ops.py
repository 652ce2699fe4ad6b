"""GPU parity of each operator through the C ABI against the oracle."""
import json
import os
import sys

import numpy as np
import pytest

from oracle import conn, event, neuron, network

pytestmark = pytest.mark.gpu

F = np.float32
GOLD = os.path.join(os.path.dirname(__file__), 'golden')


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


# ---------------------------------------------------------------- N1 compaction

@pytest.mark.parametrize('n,p,dtype', [(0, 0.1, 'u8'), (1, 1.0, 'u8'), (100, 0.3, 'u8'),
                                       (4096, 0.05, 'u8'), (4097, 0.5, 'f32'),
                                       (100_000, 0.001, 'u8'), (1_000_000, 0.0015, 'u8'),
                                       (1_000_003, 1.0, 'f32'), (300_000, 0.0, 'u8'),
                                       (16384, 1.0, 'u8'), (16385, 0.5, 'f32'),
                                       (4_000_037, 0.3, 'u8')])   # 245 tiles: look-back rounds
def test_compact(torch_cuda, n, p, dtype):
    torch = torch_cuda
    from brainstate_amd import ops
    say('compact', n, p, dtype)
    rng = np.random.RandomState(n % 1000 + 1)
    spk = rng.rand(n) < p
    arr = spk.astype(np.uint8) if dtype == 'u8' else np.where(spk, rng.rand(n) + 0.5, 0).astype(F)
    ref, c = event.compact(arr)
    for _ in range(2):   # second call reuses the workspace (epoch advance)
        idx, cnt = ops.spike_compact(dev(torch, arr))
        torch.cuda.synchronize()
        assert int(cnt.item()) == c
        assert np.array_equal(idx[:c].cpu().numpy(), ref)


def test_compact_epoch_wraps_without_a_zero_tag(torch_cuda):
    """Status words are tagged epoch + 1, and a cleared word is 0: across the epoch's wrap
    (2^32 - 2 -> 0) no call may use tag 0, or the tiles a larger call reaches for the first
    time would read as published with count 0.  A workspace at epoch 2^32 - 2 compacts 2 tiles,
    then 40 (38 never written), then 40 again."""
    torch = torch_cuda
    from brainstate_amd import _native as N
    say('compact epoch wrap')
    dev_ = torch.device('cuda')
    ws = torch.zeros(int(N.lib().bs_spike_compact_workspace_size(40 * 16384)),
                     dtype=torch.uint8, device=dev_)
    ws.view(torch.int32)[2] = -2                  # epoch 0xFFFFFFFE
    rng = np.random.RandomState(17)
    for n in (2 * 16384, 40 * 16384, 40 * 16384):
        arr = (rng.rand(n) < 0.1).astype(np.uint8)
        ref, c = event.compact(arr)
        spk = dev(torch, arr)
        idx = torch.empty(n, dtype=torch.int32, device=dev_)
        cnt = torch.empty(1, dtype=torch.int32, device=dev_)
        N.check(N.lib().bs_spike_compact(N.ptr(spk), N.BS_SPK_U8, n, N.ptr(idx), N.ptr(cnt),
                                         N.ptr(ws), N.stream_handle(dev_)), 'bs_spike_compact')
        assert int(cnt.item()) == c
        assert np.array_equal(idx[:c].cpu().numpy(), ref)
    assert int(ws.view(torch.int32)[2]) == 2     # 0xFFFFFFFE -> 0 -> 1 -> 2


@pytest.mark.parametrize('dtype', ['u8', 'f32'])
def test_compact_unaligned_view(torch_cuda, dtype):
    """A spike view that starts one element into its buffer takes the element-wise loads
    (tiles are no longer 16-byte aligned); the list is the same."""
    torch = torch_cuda
    from brainstate_amd import ops
    n = 70_001
    say('compact unaligned', n, dtype)
    rng = np.random.RandomState(9)
    spk = rng.rand(n + 1) < 0.2
    arr = spk.astype(np.uint8) if dtype == 'u8' else np.where(spk, 1.0, 0.0).astype(F)
    ref, c = event.compact(arr[1:])
    idx, cnt = ops.spike_compact(dev(torch, arr)[1:])
    assert int(cnt.item()) == c
    assert np.array_equal(idx[:c].cpu().numpy(), ref)


# ---------------------------------------------------------------- N2a scatter

@pytest.mark.parametrize('n_pre,n_post,k,p,het', [
    (20, 30, 6, 0.3, False), (3200, 4000, 80, 0.02, False), (3200, 4000, 80, 0.5, True),
    (100_000, 100_000, 1000, 0.001, True), (100_000, 100_000, 1000, 0.01, False),
    (100_000, 100_000, 1000, 0.01, True), (5000, 7, 3, 0.9, True), (1000, 500, 0, 0.5, True)])
def test_scatter_fixed(torch_cuda, n_pre, n_post, k, p, het):
    torch = torch_cuda
    from brainstate_amd import ops
    say('scatter', n_pre, n_post, k, p, het)
    rng = np.random.RandomState(k + 3)
    idx = rng.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = rng.normal(0.5, 0.1, (n_pre, k)).astype(F) if het else F(0.6)
    spk = rng.rand(n_pre) < p
    ref = event.scatter_fixed(spk, idx, w, n_post)
    act, cnt = ops.spike_compact(dev(torch, spk.astype(np.uint8)))
    out = ops.event_scatter(act, cnt, dev(torch, idx), dev(torch, w) if het else float(w), n_post)
    got = out.cpu().numpy()
    if het:
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)
    else:   # one repeated weight value: order-free, bit-exact
        assert np.array_equal(got, ref)


def test_scatter_csr_afferent(torch_cuda):
    torch = torch_cuda
    from brainstate_amd import ops
    say('scatter csr')
    indptr, indices, sel = conn.csr_afferent(2000, 1500, 60, seed=4, afferent_ratio=0.6)
    rng = np.random.RandomState(4)
    w = rng.normal(0.5, 0.1, indices.size).astype(F)
    spk = rng.rand(2000) < 0.1
    ref = event.scatter_csr(spk, indptr, indices, w, 1500)
    act, cnt = ops.spike_compact(dev(torch, spk.astype(np.uint8)))
    out = ops.event_scatter(act, cnt, dev(torch, indices), dev(torch, w), 1500,
                            indptr=dev(torch, indptr))
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- N2b gather

@pytest.mark.parametrize('n_pre,n_post,k,p,het', [
    (20, 30, 6, 0.3, True), (3200, 4000, 80, 0.02, False), (3000, 4001, 80, 0.3, True),
    (100_000, 100_000, 1000, 0.01, True), (100_000, 100_000, 1000, 0.1, False)])
def test_gather_bit_exact(torch_cuda, n_pre, n_post, k, p, het):
    torch = torch_cuda
    from brainstate_amd import ops
    say('gather', n_pre, n_post, k, p, het)
    rng = np.random.RandomState(k + 5)
    idx = rng.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = rng.normal(0.5, 0.1, (n_pre, k)).astype(F) if het else F(0.6)
    spk = rng.rand(n_pre) < p
    indptr, flat = conn.fixed_to_csr(idx)
    sell = ops.build_sell(indptr, flat, n_pre, n_post, w=w if het else None,
                          w_homo=0.0 if het else float(w), device='cuda')
    got = ops.event_gather(dev(torch, spk.astype(np.uint8)), sell).cpu().numpy()
    if n_pre * k <= 400_000:
        ref = event.scatter_fixed(spk, idx, w, n_post)
    else:   # the oracle's sequential sum in (pre, k) order, via the post-major restatement
        post_ptr, pre_of, syn_of = conn.to_post_major(indptr, flat, n_post)
        ref = event.gather_post_major(spk, post_ptr, pre_of,
                                      w.reshape(-1)[syn_of] if het else w, n_post)
    assert np.array_equal(got, ref)
    got2 = ops.event_gather(dev(torch, spk.astype(np.uint8)), sell).cpu().numpy()
    assert np.array_equal(got, got2)     # deterministic


# ---------------------------------------------------------------- N2c event x dense

@pytest.mark.parametrize('B,n_in,n_out,p,fae,sdt', [
    (1, 20, 40, 0.1, True, 'u8'), (64, 4096, 4096, 0.05, True, 'u8'),
    (3, 100, 37, 0.3, True, 'f32'), (4, 64, 128, 0.3, False, 'f32'), (2, 10, 8, 0.5, True, 'u8'),
    (5, 3000, 130, 0.1, True, 'u8'), (3, 2500, 66, 0.2, False, 'f32'),
    (130, 1000, 70, 0.05, True, 'u8'), (70, 4097, 200, 0.05, False, 'u8'),
    (1, 40000, 64, 0.01, True, 'u8')])
def test_event_dense(torch_cuda, B, n_in, n_out, p, fae, sdt):
    """Bit-exact against the oracle summed in the kernel's documented chunk order."""
    torch = torch_cuda
    from brainstate_amd import ops
    S, L = ops.event_dense_chunks(B, n_in, n_out)
    say('dense', B, n_in, n_out, p, fae, sdt, 'chunks', S, L)
    rng = np.random.RandomState(n_in)
    s = rng.rand(B, n_in) < p
    spk = s.astype(np.uint8) if sdt == 'u8' else np.where(s, rng.rand(B, n_in) * 3, 0).astype(F)
    W = rng.normal(0, 0.125, (n_in, n_out)).astype(F)
    ds, dW = dev(torch, spk), dev(torch, W)
    got = ops.event_dense(ds, dW, float_as_event=fae).cpu().numpy()
    ref = event.event_linear(spk, W, float_as_event=fae, chunk_rows=L)
    assert np.array_equal(got, ref)
    # the workspace is left ready: a second call (another spike pattern) is exact too
    s2 = np.roll(spk, 1, axis=1)
    got2 = ops.event_dense(dev(torch, s2), dW, float_as_event=fae).cpu().numpy()
    assert np.array_equal(got2, event.event_linear(s2, W, float_as_event=fae, chunk_rows=L))


# ---------------------------------------------------------------- N3 neuron steps

def test_lif_step_bit_exact(torch_cuda):
    torch = torch_cuda
    from brainstate_amd import ops
    say('lif step')
    n = 200_003
    rng = np.random.RandomState(1)
    V = rng.uniform(-62, -48, n).astype(F)
    ge = rng.exponential(0.5, n).astype(F)
    gi = rng.exponential(2.0, n).astype(F)
    ref_c = rng.choice([0, 0, 0, 1, 7, 49], n).astype(np.int32)
    in_e = (rng.rand(n) < 0.1).astype(F) * F(0.6)
    in_i = (rng.rand(n) < 0.05).astype(F) * F(6.7)
    p = neuron.LIFParams()
    eV, ege, egi, eref, espk = neuron.coba_lif_step(V, ge, gi, ref_c, in_e, in_i, p)
    tV, tge, tgi, tref = (dev(torch, a) for a in (V, ge, gi, ref_c))
    spk = ops.coba_lif_step(tV, tge, tgi, tref, dev(torch, in_e), dev(torch, in_i),
                            ops.lif_params())
    assert np.array_equal(tV.cpu().numpy(), eV)
    assert np.array_equal(tge.cpu().numpy(), ege) and np.array_equal(tgi.cpu().numpy(), egi)
    assert np.array_equal(tref.cpu().numpy(), eref)
    assert np.array_equal(spk.cpu().numpy().astype(bool), espk)
    assert espk.sum() > 100



@pytest.mark.parametrize('reset', ['hard', 'soft'])
def test_cuba_lif_step_bit_exact(torch_cuda, reset):
    """bs_coba_lif_step with CUBA output (cuba = 1, signed conductances), hard or soft reset,
    equals the oracle."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('cuba lif step', reset)
    n = 100_003
    rng = np.random.RandomState(2)
    V = rng.uniform(-62, -48, n).astype(F)
    ge = rng.exponential(0.5, n).astype(F)
    gi = -rng.exponential(2.0, n).astype(F)
    ref_c = rng.choice([0, 0, 0, 1, 7, 49], n).astype(np.int32)
    in_e = (rng.rand(n) < 0.1).astype(F) * F(1.62)
    in_i = (rng.rand(n) < 0.05).astype(F) * F(-9.0)
    p = neuron.LIFParams(V_rest=-49., V_th=-50., V_reset=-60., tau=20., I_ext=20., out='cuba',
                         scale_e=1.0, scale_i=0.75, spk_reset=reset)
    eV, ege, egi, eref, espk = neuron.coba_lif_step(V, ge, gi, ref_c, in_e, in_i, p)
    tV, tge, tgi, tref = (dev(torch, a) for a in (V, ge, gi, ref_c))
    spk = ops.coba_lif_step(tV, tge, tgi, tref, dev(torch, in_e), dev(torch, in_i),
                            ops.lif_params(V_rest=-49., V_th=-50., V_reset=-60., tau=20.,
                                           I_ext=20., out='cuba', scale_e=1.0, scale_i=0.75,
                                           spk_reset=reset))
    assert np.array_equal(tV.cpu().numpy(), eV)
    assert np.array_equal(tge.cpu().numpy(), ege) and np.array_equal(tgi.cpu().numpy(), egi)
    assert np.array_equal(tref.cpu().numpy(), eref)
    assert np.array_equal(spk.cpu().numpy().astype(bool), espk)
    assert espk.sum() > 100

def test_lif_reference_kat_on_gpu(torch_cuda):
    """docs/tutorials/brain_dynamics/04_building_an_snn.ipynb cell 5: -59.84079742 mV."""
    torch = torch_cuda
    from brainstate_amd import ops
    p = ops.lif_params(V_rest=-52., V_th=-50., V_reset=-60., tau=10., tau_ref=0., I_ext=8.,
                       dt=0.1)
    V = torch.full((4,), -60.0, device='cuda')
    z = torch.zeros(4, device='cuda')
    spk = ops.coba_lif_step(V, z.clone(), z.clone(), torch.zeros(4, dtype=torch.int32,
                                                                 device='cuda'), None, None, p)
    assert np.all(V.cpu().numpy() == F(-59.84079742)) and spk.sum().item() == 0


def test_hh_init_and_step_bit_exact(torch_cuda):
    torch = torch_cuda
    from brainstate_amd import ops
    say('hh step')
    n = 100_001
    rng = np.random.RandomState(2)
    V = rng.uniform(-80, 40, n).astype(F)
    V[:5] = [-40.0, -55.0, -65.0, -35.0, 20.0]   # exprel singular points of the rates
    m, h, ng = neuron.hh_init(V)
    tV = dev(torch, V)
    tm, th, tn = (torch.empty(n, device='cuda') for _ in range(3))
    ops.hh_init(tV, tm, th, tn)
    assert np.array_equal(tm.cpu().numpy(), m) and np.array_equal(th.cpu().numpy(), h)
    assert np.array_equal(tn.cpu().numpy(), ng)
    ge = rng.exponential(0.1, n).astype(F)
    gi = rng.exponential(0.3, n).astype(F)
    in_e = (rng.rand(n) < 0.1).astype(F) * F(0.05)
    in_i = (rng.rand(n) < 0.05).astype(F) * F(0.3)
    p = neuron.HHParams(I_ext=6.5)
    exp = neuron.hh_step(V, m, h, ng, ge, gi, in_e, in_i, p)
    tge, tgi = dev(torch, ge), dev(torch, gi)
    spk = ops.coba_hh_step(tV, tm, th, tn, tge, tgi, dev(torch, in_e), dev(torch, in_i),
                           ops.hh_params(I_ext=6.5))
    got = [tV, tm, th, tn, tge, tgi]
    for g, e in zip(got, exp[:6]):
        assert np.array_equal(g.cpu().numpy(), e)
    assert np.array_equal(spk.cpu().numpy().astype(bool), exp[6])


def test_step_kernels_take_per_neuron_input(torch_cuda):
    """bs_coba_lif_step_in / bs_coba_hh_step_in: one external input per neuron in place of
    the parameters' I_ext, bit-exact against the oracle given the same array (the neuron
    called with an input array of its shape)."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('step kernels, per-neuron input')
    n = 50_001
    rng = np.random.RandomState(3)
    I = rng.uniform(10., 30., n).astype(F)
    V = rng.uniform(-62, -48, n).astype(F)
    ge, gi = rng.exponential(0.5, n).astype(F), rng.exponential(2.0, n).astype(F)
    ref_c = rng.choice([0, 0, 0, 1, 7], n).astype(np.int32)
    in_e = (rng.rand(n) < 0.1).astype(F) * F(0.6)
    in_i = (rng.rand(n) < 0.05).astype(F) * F(6.7)
    eV, ege, egi, eref, espk = neuron.coba_lif_step(V, ge, gi, ref_c, in_e, in_i,
                                                    neuron.LIFParams(I_ext=I))
    tV, tge, tgi, tref = (dev(torch, a) for a in (V, ge, gi, ref_c))
    spk = ops.coba_lif_step(tV, tge, tgi, tref, dev(torch, in_e), dev(torch, in_i),
                            ops.lif_params(I_ext=0.), I_ext=dev(torch, I))
    assert np.array_equal(tV.cpu().numpy(), eV) and np.array_equal(tref.cpu().numpy(), eref)
    assert np.array_equal(spk.cpu().numpy().astype(bool), espk) and espk.sum() > 100
    # HH
    V = rng.uniform(-75, -50, n).astype(F)
    m, h, ng = neuron.hh_init(V)
    I = rng.uniform(0., 12., n).astype(F)
    ge, gi = rng.exponential(0.1, n).astype(F), rng.exponential(0.3, n).astype(F)
    exp = neuron.hh_step(V, m, h, ng, ge, gi, in_e * F(0.1), in_i * F(0.05),
                         neuron.HHParams(I_ext=I))
    t = [dev(torch, a) for a in (V, m, h, ng, ge, gi)]
    spk = ops.coba_hh_step(*t, dev(torch, in_e * F(0.1)), dev(torch, in_i * F(0.05)),
                           ops.hh_params(I_ext=0.), I_ext=dev(torch, I))
    for g, e in zip(t, exp[:6]):
        assert np.array_equal(g.cpu().numpy(), e)
    assert np.array_equal(spk.cpu().numpy().astype(bool), exp[6])


# ---------------------------------------------------------------- fused spike-vector mat-vec

@pytest.mark.parametrize('n_pre,n_post,k,p,het,csr', [
    (3200, 4000, 80, 0.02, False, False),     # config [1] E projection, direct atomics
    (3200, 4000, 80, 0.9, True, False),       # dense activity, LDS-aggregated path
    (3200, 4000, 80, 0.9, False, False),      # dense, homogeneous: direct (bit-exact)
    (100_000, 100_000, 1000, 0.01, True, False),
    (2000, 1500, 60, 0.5, True, True),        # CSR (afferent ratio)
    (50, 10, 3, 1.0, True, False)])
def test_event_matvec_fused(torch_cuda, n_pre, n_post, k, p, het, csr):
    torch = torch_cuda
    from brainstate_amd import ops
    say('matvec fused', n_pre, n_post, k, p, het, csr)
    rng = np.random.RandomState(k + 11)
    if csr:
        indptr, indices, _ = conn.csr_afferent(n_pre, n_post, k, seed=5, afferent_ratio=0.6)
        w = rng.normal(0.5, 0.1, indices.size).astype(F) if het else F(0.6)
        spk = rng.rand(n_pre) < p
        ref = event.scatter_csr(spk, indptr, indices, w, n_post)
        out = ops.event_matvec(dev(torch, spk.astype(np.uint8)), dev(torch, indices),
                               dev(torch, w) if het else float(w), n_post,
                               indptr=dev(torch, indptr))
    else:
        idx = rng.randint(0, n_post, (n_pre, k)).astype(np.int32)
        w = rng.normal(0.5, 0.1, (n_pre, k)).astype(F) if het else F(0.6)
        spk = rng.rand(n_pre) < p
        ref = event.scatter_fixed(spk, idx, w, n_post)
        out = ops.event_matvec(dev(torch, spk.astype(np.uint8)), dev(torch, idx),
                               dev(torch, w) if het else float(w), n_post)
    got = out.cpu().numpy()
    if het:   # the north_star tolerance of the atomic path
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)
    else:
        assert np.array_equal(got, ref)


def test_gather_global_bitmap_path(torch_cuda):
    """n_pre > 524288: the spike bitmap is read from global memory instead of LDS."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('gather global bitmap')
    n_pre, n_post, k = 600_000, 20_000, 20
    rng = np.random.RandomState(3)
    idx = rng.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = rng.normal(0.5, 0.1, (n_pre, k)).astype(F)
    spk = rng.rand(n_pre) < 0.01
    indptr, flat = conn.fixed_to_csr(idx)
    sell = ops.build_sell(indptr, flat, n_pre, n_post, w=w, device='cuda')
    got = ops.event_gather(dev(torch, spk.astype(np.uint8)), sell).cpu().numpy()
    post_ptr, pre_of, syn_of = conn.to_post_major(indptr, flat, n_post)
    ref = event.gather_post_major(spk, post_ptr, pre_of, w.reshape(-1)[syn_of], n_post)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize('n', [1, 63, 64, 65, 1000, 100_003])
def test_spike_pack(torch_cuda, n):
    torch = torch_cuda
    from brainstate_amd import ops
    spk = np.random.RandomState(n).rand(n) < 0.3
    bits = ops.spike_pack(dev(torch, spk.astype(np.uint8))).cpu().numpy().view(np.uint32)
    ref = np.zeros((n + 31) // 32, np.uint32)
    for i in np.flatnonzero(spk):
        ref[i // 32] |= np.uint32(1) << np.uint32(i % 32)
    assert np.array_equal(bits[:ref.size], ref)
