"""GPU parity of the destination-bucketed event mat-vec (bs_bucket_build, bs_event_bucket_f32)
against the oracle's sequential scatter (brainstate/nn/_event_fixedprob.py:202-209,249-252;
closed form of _event_fixedprob_test.py:247-260)."""
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


def expected_layout(indptr, indices, n_post, nb, P):
    """The layout contract of bs_bucket_build, restated row by row with a stable sort."""
    n_pre = indptr.size - 1
    seg = np.zeros((n_pre, nb + 1), np.int64)
    lidx = np.zeros(indices.size, np.int64)
    for i in range(n_pre):
        lo, hi = int(indptr[i]), int(indptr[i + 1])
        t = indices[lo:hi].astype(np.int64)
        valid = (t >= 0) & (t < n_post)
        b = np.where(valid, t // P, nb)
        order = np.argsort(b, kind='stable')
        lidx[lo:hi] = np.where(valid, t - b * P, 0)[order]
        counts = np.bincount(b[valid], minlength=nb)
        seg[i, :nb] = lo + np.concatenate([[0], np.cumsum(counts)[:-1]])
        seg[i, nb] = lo + valid.sum()
    return seg, lidx


@pytest.mark.parametrize('n_pre,n_post,k,het', [(300, 1000, 17, True), (70, 5, 9, False),
                                                (513, 200_003, 40, True)])
def test_layout_matches_contract(torch_cuda, n_pre, n_post, k, het):
    torch = torch_cuda
    from brainstate_amd import ops
    say('bucket layout', n_pre, n_post, k, het)
    rng = np.random.RandomState(n_pre)
    idx = rng.randint(-2, n_post + 2, (n_pre, k)).astype(np.int32)  # some out of range
    w = rng.rand(n_pre, k).astype(F) if het else None
    L = ops.build_buckets(dev(torch, idx), n_post, w=w, w_homo=0.5)
    nb, P = L['nb'], L['P']
    assert nb * P >= n_post > (nb - 1) * P and P <= 16384
    indptr = np.arange(n_pre + 1, dtype=np.int64) * k
    seg, lidx = expected_layout(indptr, idx.reshape(-1), n_post, nb, P)
    got_seg = L['seg'][:n_pre * (nb + 1)].cpu().numpy().reshape(n_pre, nb + 1)
    assert np.array_equal(got_seg, seg)
    got = L['lidx'].cpu().numpy().view(np.uint16).astype(np.int64)[:idx.size]
    for i in range(n_pre):  # valid synapses (out-of-range ones follow, never read)
        lo, hi = seg[i, 0], seg[i, nb]
        assert np.array_equal(got[lo:hi], lidx[lo:hi])
    if het:
        # weights travel with their synapse: the bucketed sums reproduce the row sums
        got_w = L['w'].cpu().numpy()[:idx.size]
        for i in range(0, n_pre, 37):
            lo, hi = seg[i, 0], seg[i, nb]
            row = idx[i]
            valid = (row >= 0) & (row < n_post)
            assert np.isclose(got_w[lo:hi].astype(np.float64).sum(),
                              w[i][valid].astype(np.float64).sum(), rtol=1e-6)


@pytest.mark.parametrize('n_pre,n_post,k,p,het,sdt', [
    (2000, 3000, 50, 0.1, True, 'u8'), (2000, 3000, 50, 0.1, False, 'u8'),
    (20_000, 100_000, 200, 0.01, True, 'u8'), (20_000, 100_000, 200, 0.1, False, 'u8'),
    (5000, 150_000, 100, 0.05, True, 'f32'), (64, 10, 3, 0.5, True, 'u8'),
    (1000, 1000, 10, 0.0, True, 'u8'), (100_000, 100_000, 1000, 0.001, True, 'u8')])
def test_bucket_matvec_matches_oracle(torch_cuda, n_pre, n_post, k, p, het, sdt):
    """Per-synapse weights: bit-exact against the oracle's fixed-point restatement and within
    rtol 1e-5 / atol 1e-6 of the sequential fp32 scatter; homogeneous weights bit-exact
    against the sequential scatter (counted events, one chain of additions)."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('bucket matvec', n_pre, n_post, k, p, het, sdt)
    rng = np.random.RandomState(k + n_pre)
    idx = rng.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = rng.normal(0.5, 0.1, (n_pre, k)).astype(F) if het else F(0.6)
    s = rng.rand(n_pre) < p
    spk = s.astype(np.uint8) if sdt == 'u8' else np.where(s, rng.rand(n_pre) + 0.5, 0).astype(F)
    L = ops.build_buckets(dev(torch, idx), n_post, w=w if het else None, w_homo=0.6)
    got = ops.event_bucket(dev(torch, spk), L).cpu().numpy()
    ref = event.scatter_fixed(spk, idx, w, n_post)
    if het:
        S = int(L['qexp'].item())
        assert S == event.bucket_qexp(w, idx, n_post)
        indptr = np.arange(n_pre + 1, dtype=np.int64) * k
        exact = event.scatter_fixed_point(spk, indptr, idx.reshape(-1), w, n_post, S)
        assert np.array_equal(got, exact)                      # the documented arithmetic
        assert np.allclose(got, ref, rtol=1e-5, atol=1e-6)     # the sequential fp32 scatter
        again = ops.event_bucket(dev(torch, spk), L).cpu().numpy()
        assert np.array_equal(got, again)                      # deterministic
    else:
        assert np.array_equal(got, ref)
    # accumulate adds onto what is there
    base = rng.rand(n_post).astype(F)
    acc = ops.event_bucket(dev(torch, spk), L, out=dev(torch, base.copy()), accumulate=True)
    assert np.allclose(acc.cpu().numpy(), base + ref, rtol=1e-5, atol=1e-5)


def test_bucket_csr_ragged_and_out_of_range(torch_cuda):
    """CSR rows of varying length (some empty) with out-of-range targets, which contribute
    nothing (as in the scatter)."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('bucket csr')
    rng = np.random.RandomState(5)
    n_pre, n_post = 3000, 40_000
    lens = rng.randint(0, 90, n_pre)
    lens[::17] = 0
    indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    indices = rng.randint(-5, n_post + 5, indptr[-1]).astype(np.int32)
    w = rng.rand(indptr[-1]).astype(F)
    spk = (rng.rand(n_pre) < 0.2).astype(np.uint8)
    L = ops.build_buckets(dev(torch, indices), n_post, w=w, indptr=dev(torch, indptr))
    got = ops.event_bucket(dev(torch, spk), L).cpu().numpy()
    keep = (indices >= 0) & (indices < n_post)
    ref = event.scatter_csr(spk, indptr, np.where(keep, indices, 0), np.where(keep, w, 0), n_post)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6)
    S = int(L['qexp'].item())
    assert S == event.bucket_qexp(w, indices, n_post)  # W and D over the valid synapses
    assert np.array_equal(got, event.scatter_fixed_point(spk, indptr, indices, w, n_post, S))


def test_bucket_non_finite_weight_falls_back(torch_cuda):
    """A non-finite per-synapse weight cannot be held in fixed point: the sums fall back to
    fp32 and the inf / nan reach exactly the outputs the scatter sends them to."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('bucket non-finite')
    rng = np.random.RandomState(9)
    n_pre, n_post, k = 500, 2000, 20
    idx = rng.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = rng.rand(n_pre, k).astype(F)
    w[3, 4] = np.inf
    w[7, 1] = np.nan
    spk = (rng.rand(n_pre) < 0.5).astype(np.uint8)
    spk[3] = spk[7] = 1
    L = ops.build_buckets(dev(torch, idx), n_post, w=w)
    assert int(L['qexp'].item()) == -1000
    got = ops.event_bucket(dev(torch, spk), L).cpu().numpy()
    ref = event.scatter_fixed(spk, idx, w, n_post)
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(np.isinf(got), np.isinf(ref))
    fin = np.isfinite(ref)
    assert np.allclose(got[fin], ref[fin], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize('p', [0.1, 0.01, 0.001])
def test_bucket_config2_full_size_against_oracle(torch_cuda, p):
    """Config [2] at full size (100k x 100k, K = 1000, per-synapse weights N(0.5, 0.1), spike
    density p): the bucketed path equals the oracle's fixed-point restatement bit for bit
    (with the layout's S equal to the oracle's exponent rule), and is deterministic; the
    fused atomic mat-vec equals the oracle's sequential fp32 sum within the north_star
    tolerance rel 1e-5 / abs 1e-6; both are within their error bounds of the float64 sum;
    homogeneous weights give the sequential scatter's bits on both paths."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('bucket config2 full size vs oracle', p)
    n, k = 100_000, 1000
    rng = np.random.RandomState(7)
    idx = rng.randint(0, n, size=(n, k)).astype(np.int32)
    w = rng.normal(0.5, 0.1, (n, k)).astype(F)
    spk = (np.random.RandomState(1000).rand(n) < p).astype(np.uint8)
    d_idx, d_w, d_spk = dev(torch, idx), dev(torch, w), dev(torch, spk)
    L = ops.build_buckets(d_idx, n, w=d_w)
    got = ops.event_bucket(d_spk, L).cpu().numpy()
    assert np.array_equal(got, ops.event_bucket(d_spk, L).cpu().numpy())  # deterministic
    atomic = ops.event_matvec(d_spk, d_idx, d_w, n).cpu().numpy()
    del L
    S = event.bucket_qexp(w, idx, n)
    indptr = np.arange(n + 1, dtype=np.int64) * k
    say('  gpu done, oracle sums')
    want = event.scatter_fixed_point(spk, indptr, idx.reshape(-1), w, n, S)
    assert np.array_equal(got, want)
    seq = event.scatter_fixed(spk, idx, w, n)
    assert np.allclose(atomic, seq, rtol=1e-5, atol=1e-6)
    act = np.flatnonzero(spk)
    t = idx[act].reshape(-1)
    exact = np.zeros(n)
    np.add.at(exact, t, w[act].reshape(-1).astype(np.float64))
    cnt = np.bincount(t, minlength=n)
    assert np.all(np.abs(got - exact) <= cnt * 2.0 ** -(S + 1) + 2.0 ** -24 * np.abs(exact))
    assert int(cnt.max()) > 0
    Lh = ops.build_buckets(d_idx, n, w=None, w_homo=0.6)
    gh = ops.event_bucket(d_spk, Lh).cpu().numpy()
    hseq = event.scatter_fixed(spk, idx, F(0.6), n)
    assert np.array_equal(gh, hseq)
    assert np.array_equal(ops.event_matvec(d_spk, d_idx, 0.6, n).cpu().numpy(), hseq)


def test_matvec_2000_fixture_on_every_path(torch_cuda):
    """The committed reduced config-[2] digests: the bucketed path gives the fixed-point sums,
    the SELL gather the sequential per-synapse sums, and every path the homogeneous sums."""
    import hashlib
    import json
    import os
    torch = torch_cuda
    from brainstate_amd import ops
    say('matvec 2000 fixture')
    gdir = os.path.join(os.path.dirname(__file__), 'golden')
    sys.path.insert(0, gdir)
    import make_golden
    gold = json.load(open(os.path.join(gdir, 'matvec_2000.json')))
    c = gold['config']
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    spk, idx, w = make_golden.matvec_case(c['p'][0])
    d_idx, d_w = dev(torch, idx), dev(torch, w)
    L = ops.build_buckets(d_idx, c['n_post'], w=d_w)
    Lh = ops.build_buckets(d_idx, c['n_post'], w=None, w_homo=c['w_homo'])
    indptr = np.arange(c['n_pre'] + 1, dtype=np.int64) * c['k']
    sell = ops.build_sell(indptr, idx.reshape(-1), c['n_pre'], c['n_post'], w=w.reshape(-1))
    for case in gold['cases']:
        spk, _, _ = make_golden.matvec_case(case['p'])
        d_spk = dev(torch, spk)
        assert sha(ops.event_bucket(d_spk, L).cpu().numpy()) == case['fixed_point_sha256']
        assert sha(ops.event_bucket(d_spk, Lh).cpu().numpy()) == case['homo_sha256']
        assert sha(ops.event_matvec(d_spk, d_idx, c['w_homo'], c['n_post']).cpu().numpy()) \
            == case['homo_sha256']
        assert sha(ops.event_gather(d_spk, sell).cpu().numpy()) == case['het_sequential_sha256']


def _bucket_ws_header(torch, dev_index=0):
    """R_eff the last bucketed step on the current stream chose (workspace word 0)."""
    from brainstate_amd import ops
    key = ('bucket', dev_index, torch.cuda.current_stream(dev_index).cuda_stream)
    return int(ops._WS_CACHE[key][:4].view(torch.int32).item())


def _expected_row_groups(s, n_pre, nb):
    """The documented rule: R_eff = ceil(active rows of the leading min(n_pre, 16384) rows,
    scaled to n_pre, / 128), within [1, R], R = min(256 // nb, 32, ceil(n_pre / 64))."""
    ns = min(n_pre, 16384)
    act = int(np.count_nonzero(np.asarray(s)[:ns]))
    re = -(-act * n_pre // (ns * 128))
    return max(1, min(_max_row_groups(n_pre, nb), re))


def _max_row_groups(n_pre, nb):
    """R = min(256 // nb, 32, ceil(n_pre / 64)): 32 row groups at most whatever nb (a layout
    of fewer than 8 buckets would otherwise have up to 256 partial rows to add)."""
    return max(1, min(256 // nb, 32, -(-n_pre // 64)))


@pytest.mark.parametrize('n_pre,n_post,k,p,het,accumulate,sdt', [
    (100_000, 100_000, 100, 0.001, True, False, 'u8'),   # R_eff = 1: the step writes out
    (20_000, 100_000, 200, 0.1, True, True, 'u8'),       # R_eff = 16 of 28 partials
    (20_000, 100_000, 200, 0.1, False, False, 'u8'),
    (100_000, 50_000, 20, 0.5, True, False, 'u8'),       # R_eff = R (capped)
    (60_000, 30_000, 20, 0.5, True, False, 'f32'),       # R_eff = R, f32 spikes
    (60_000, 30_000, 20, 0.002, False, True, 'f32'),     # R_eff = 1, f32 spikes
    (3_000, 500_000, 50, 0.01, True, False, 'u8'),       # 41 buckets: 6 sub-ranges each
    (50, 20_000, 30, 0.5, True, True, 'u8'),             # n_pre <= 64: one row group at most
    (2_000, 1_600_000, 40, 0.3, True, True, 'u8'),       # 131 buckets: one row group at most
    (100_000, 6, 4, 0.3, True, False, 'u8'),             # 6 buckets: 32 row groups, not 42
    (100_000, 6, 4, 0.3, False, True, 'u8'),
    (800_000, 1_000_000, 4, 0.05, True, False, 'u8'),   # 82 buckets: 3 groups of 266,667 rows
    (800_000, 1_000_000, 4, 0.05, False, True, 'u8')])
def test_bucket_row_groups_follow_density(torch_cuda, n_pre, n_post, k, p, het, accumulate,
                                          sdt):
    """The step picks its number of row groups from the spikes on the device; whatever it
    picks, the sums are the fixed-point restatement's bit for bit (homogeneous: the
    sequential scatter's), and accumulate adds onto out with the same arithmetic.  Mode
    'dense' on a layout with one row group at most runs as mode 'split' (its one group writes
    out; the fixed-grid kernel only writes partials)."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('bucket row groups', n_pre, n_post, k, p, het, accumulate, sdt)
    rng = np.random.RandomState(n_pre + k)
    idx = rng.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = rng.normal(0.5, 0.1, (n_pre, k)).astype(F) if het else None
    act = rng.rand(n_pre) < p
    s = act.astype(np.uint8) if sdt == 'u8' else np.where(act, rng.rand(n_pre) + 0.5, 0).astype(F)
    L = ops.build_buckets(dev(torch, idx), n_post, w=w, w_homo=0.6)
    base = rng.rand(n_post).astype(F)
    R_est = _expected_row_groups(s, n_pre, L['nb'])
    R_max = _max_row_groups(n_pre, L['nb'])
    gots = {}
    want_hint = max(1, min(R_max, -(-int(np.count_nonzero(s)) // 128)))
    # 'single' last before 'auto': its estimate (from the exact count) steers 'auto': one
    # launch at 1, the fixed grid above half the maximum when its row groups hold at most
    # 8,192 rows, else groups chosen on the device
    short = -(-n_pre // R_max) <= 8192
    auto = 'single' if want_hint == 1 else (
        'dense' if 2 * want_hint > R_max > 1 and short else 'split')
    for mode in ('split', 'dense', 'single', 'auto'):
        out = dev(torch, base.copy())
        gots[mode] = ops.event_bucket(dev(torch, s), L, out=out, accumulate=accumulate,
                                      mode=mode).cpu().numpy()
        ran = auto if mode == 'auto' else mode
        # row groups the step used (single: 1, dense: the maximum) and its estimate
        used = {'single': 1, 'dense': R_max}.get(ran, R_est)
        assert _bucket_ws_header(torch) == used, mode
        if ran == 'dense':   # estimated from row group 0's rows
            assert 1 <= int(L['_hint'][1][0]) <= R_max
        elif ran == 'single':   # from the exact active count
            assert int(L['_hint'][1][0]) == want_hint, mode
        else:
            assert int(L['_hint'][1][0]) == R_est, mode
    got = gots['split']
    for mode in ('single', 'dense', 'auto'):
        assert np.array_equal(gots[mode], got), mode
    indptr = np.arange(n_pre + 1, dtype=np.int64) * k
    if het:
        S = int(L['qexp'].item())
        want = event.scatter_fixed_point(s, indptr, idx.reshape(-1), w, n_post, S)
        if accumulate:
            want = (base + want).astype(F)
    else:
        # homogeneous: counted events, then w added c times from out (or 0) in one chain
        cnt = np.zeros(n_post, np.int64)
        np.add.at(cnt, idx[act].reshape(-1), 1)
        want = (base.copy() if accumulate else np.zeros(n_post, F))
        for c in range(1, int(cnt.max()) + 1):
            want = np.where(cnt >= c, (want + F(0.6)).astype(F), want).astype(F)
    assert np.array_equal(got, want)


@pytest.mark.parametrize('het', [True, False])
def test_bucket_skewed_activity(torch_cuda, het):
    """A silent leading sample (R_eff = 1) followed by 23,616 active rows: one row group lists
    more than 4096 active rows per 16,384-row batch, so the batches split in four and the list
    is flushed many times; the sums stay exact."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('bucket skewed activity', het)
    n_pre, n_post, k = 40_000, 50_000, 64
    rng = np.random.RandomState(77)
    idx = rng.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = rng.normal(0.5, 0.1, (n_pre, k)).astype(F) if het else None
    s = np.zeros(n_pre, np.uint8)
    s[16384:] = 1
    L = ops.build_buckets(dev(torch, idx), n_post, w=w, w_homo=0.6)
    got = ops.event_bucket(dev(torch, s), L).cpu().numpy()
    assert _bucket_ws_header(torch) == 1
    if het:
        indptr = np.arange(n_pre + 1, dtype=np.int64) * k
        want = event.scatter_fixed_point(s, indptr, idx.reshape(-1), w, n_post,
                                         int(L['qexp'].item()))
    else:
        want = event.scatter_fixed(s, idx, F(0.6), n_post)
    assert np.array_equal(got, want)


@pytest.mark.parametrize('sdt,p', [('u8', 0.01), ('u8', 0.3), ('f32', 0.05)])
def test_bucket_unaligned_spike_views(torch_cuda, sdt, p):
    """Spike vectors that do not start on a 16-byte boundary (a row of a [T, n] tensor with
    n % 16 != 0) take the per-row loads and give the same sums."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('bucket unaligned', sdt, p)
    n_pre, n_post, k = 30_001, 20_000, 30
    rng = np.random.RandomState(3)
    idx = rng.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = rng.normal(0.5, 0.1, (n_pre, k)).astype(F)
    s = rng.rand(n_pre) < p
    spk = s.astype(np.uint8) if sdt == 'u8' else np.where(s, rng.rand(n_pre) + 0.5, 0).astype(F)
    buf = dev(torch, np.concatenate([np.zeros(1, spk.dtype), spk]))
    view = buf[1:]
    assert view.data_ptr() % 16 != 0
    L = ops.build_buckets(dev(torch, idx), n_post, w=w)
    got = ops.event_bucket(view, L).cpu().numpy()
    aligned = ops.event_bucket(dev(torch, spk), L).cpu().numpy()
    indptr = np.arange(n_pre + 1, dtype=np.int64) * k
    want = event.scatter_fixed_point(spk, indptr, idx.reshape(-1), w, n_post,
                                     int(L['qexp'].item()))
    assert np.array_equal(got, want) and np.array_equal(aligned, want)


def test_bucket_graph_replays(torch_cuda):
    """The step captured in a HIP graph: each replay re-reads the spike buffer and picks its
    row groups on the device (sparse and dense contents alternate), with eager calls and
    synchronisations between replays; every replay equals the eager result."""
    torch = torch_cuda
    from brainstate_amd import ops
    say('bucket graph replays')
    n_pre, n_post, k = 50_000, 60_000, 100
    rng = np.random.RandomState(21)
    idx = dev(torch, rng.randint(0, n_post, (n_pre, k)).astype(np.int32))
    w = dev(torch, rng.normal(0.5, 0.1, (n_pre, k)).astype(F))
    L = ops.build_buckets(idx, n_post, w=w)
    spks = [dev(torch, (rng.rand(n_pre) < p).astype(np.uint8)) for p in (0.001, 0.2, 0.02)]
    eager = [ops.event_bucket(x, L).cpu().numpy() for x in spks]
    x = torch.zeros(n_pre, dtype=torch.uint8, device='cuda')
    out = torch.empty(n_post, device='cuda')
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        x.copy_(spks[1])
        ops.event_bucket(x, L, out=out)  # workspace of the capture stream allocated here
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        ops.event_bucket(x, L, out=out)
    for rep in range(6):
        j = rep % 3
        x.copy_(spks[j])
        out.fill_(-1.0)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager[j]), rep
        again = ops.event_bucket(spks[(j + 1) % 3], L).cpu().numpy()
        assert np.array_equal(again, eager[(j + 1) % 3])
