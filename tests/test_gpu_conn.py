"""GPU tests of device-side connectivity (bs_conn_fixed_num*, bs_csr_from_selected):
bit-equality with numpy's RandomState stream, which brainstate/nn/_event_fixedprob.py:163-196
draws from, the golden digests, the afferent CSR, and the without-replacement sampler against
its restatement."""
import hashlib
import json
import os
import time

import numpy as np
import pytest

from oracle import conn, rng

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), 'golden')


@pytest.fixture(scope='module')
def bs():
    import torch
    if not torch.cuda.is_available():
        pytest.fail('GPU tests need a ROCm GPU')
    import brainstate_amd
    return brainstate_amd


def say(*a):
    print('[case]', *a, flush=True)


@pytest.mark.parametrize('seed,n_pre,k,n_post', [(1, 300, 80, 4000), (7, 50, 13, 1024),
                                                 (3, 40, 9, 1025), (9, 20, 5, 2),
                                                 (11, 10, 6, 1), (0, 1, 1, 3),
                                                 (2 ** 32 - 1, 64, 7, 2 ** 31 - 1),
                                                 (5, 200_000, 100, 1_000_000)])
def test_indices_equal_numpy_randint(bs, seed, n_pre, k, n_post):
    say('conn randint', seed, n_pre, k, n_post)
    want = np.random.RandomState(seed).randint(0, n_post, size=(n_pre, k)).astype(np.int32)
    idx, sel = bs.ops.conn_fixed_num(seed, n_pre, k, n_post)
    assert sel is None
    assert np.array_equal(idx.cpu().numpy(), want)


@pytest.mark.parametrize('seed,n_pre,k,n_post,ratio', [(3, 500, 20, 800, 0.5),
                                                       (4, 1000, 7, 1, 0.3),
                                                       (6, 333, 0, 10, 0.9),
                                                       (8, 50_000, 100, 100_000, 0.25)])
def test_afferent_selection_and_csr(bs, seed, n_pre, k, n_post, ratio):
    """selected = the same stream's random(n_pre) < ratio after the index draws (:186);
    indptr / indices as :185-196 build them."""
    say('conn afferent', seed, n_pre, k, n_post, ratio)
    r = np.random.RandomState(seed)
    want_idx = r.randint(0, n_post, size=(n_pre, k)) if k else np.zeros((n_pre, 0), np.int64)
    want_sel = r.random(n_pre) < ratio
    idx, sel = bs.ops.conn_fixed_num(seed, n_pre, k, n_post, ratio)
    assert np.array_equal(idx.cpu().numpy(), want_idx.astype(np.int32))
    assert np.array_equal(sel.cpu().numpy(), want_sel)
    indptr, csr = bs.ops.csr_from_selected(idx, sel)
    want_ptr = np.insert(np.arange(1, n_pre + 1) * k - np.cumsum(~want_sel) * k, 0, 0)
    assert np.array_equal(indptr.cpu().numpy(), want_ptr)
    assert np.array_equal(csr.cpu().numpy(), want_idx[want_sel].ravel())


def test_golden_digests_through_fixednumconn(bs):
    """The module path (EventFixedProb with a seed) builds the golden index arrays on the
    device."""
    say('conn golden digests')
    with open(os.path.join(GOLD, 'conn_digests.json')) as f:
        gold = json.load(f)
    for case in gold:
        m = bs.nn.EventFixedProb(case['n_pre'], case['n_post'], case['k'], 0.5, seed=case['seed'])
        idx = m.conn.indices.cpu().numpy()
        assert hashlib.sha256(np.ascontiguousarray(idx).tobytes()).hexdigest() == \
            case['sha256'], case


def test_fixedprob_afferent_module_matches_oracle(bs):
    say('conn afferent module')
    indptr, indices, sel = conn.csr_afferent(300, 200, 12, seed=4, afferent_ratio=0.4)
    m = bs.nn.EventFixedProb(300, 200, 12, 0.5, seed=4, afferent_ratio=0.4)
    assert np.array_equal(m.pre_selected, sel)
    assert np.array_equal(m.conn.indptr.cpu().numpy(), indptr)
    assert np.array_equal(m.conn.indices.cpu().numpy(), indices)


@pytest.mark.parametrize('seed,n_pre,k,n_post', [(123, 40, 30, 40), (2 ** 40 + 5, 30, 64, 1000),
                                                 (7, 8, 1, 1), (9, 16, 300, 350)])
def test_unique_rows_equal_restatement(bs, seed, n_pre, k, n_post):
    say('conn unique', seed, n_pre, k, n_post)
    got = bs.ops.conn_fixed_num_unique(seed, n_pre, k, n_post).cpu().numpy()
    assert np.array_equal(got, rng.unique_rows(seed, n_pre, k, n_post))


def test_unique_rows_large_properties(bs):
    say('conn unique large')
    n_pre, k, n_post = 100_000, 100, 2000
    got = bs.ops.conn_fixed_num_unique(77, n_pre, k, n_post).cpu().numpy()
    assert got.min() >= 0 and got.max() < n_post
    s = np.sort(got, axis=1)
    assert not np.any(s[:, 1:] == s[:, :-1])
    counts = np.bincount(got.ravel(), minlength=n_post)
    exp = got.size / n_post
    chi2 = ((counts - exp) ** 2 / exp).sum()
    assert chi2 < n_post + 8 * np.sqrt(2 * n_post)
    m = bs.nn.EventFixedProb(500, 300, 40, 0.5, seed=3, allow_multi_conn=False)
    rows = np.sort(m.conn.indices.cpu().numpy(), axis=1)
    assert not np.any(rows[:, 1:] == rows[:, :-1])


def test_device_build_time_1m(bs):
    """Config [3]'s connectivity (1M x 100) on the device vs numpy on the host (reported)."""
    import torch
    say('conn 1M timing')
    n = 1_000_000
    bs.ops.conn_fixed_num(100, 1000, 100, n)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    idx, _ = bs.ops.conn_fixed_num(101, 800_000, 100, n)
    torch.cuda.synchronize()
    dev_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    want = np.random.RandomState(101).randint(0, n, size=(800_000, 100)).astype(np.int32)
    host_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    torch.from_numpy(want).cuda()
    torch.cuda.synchronize()
    h2d_s = time.perf_counter() - t0
    print(f'[conn] 8e7 draws: device {dev_s * 1e3:.1f} ms, numpy {host_s * 1e3:.1f} ms + '
          f'H2D {h2d_s * 1e3:.1f} ms', flush=True)
    assert np.array_equal(idx.cpu().numpy(), want)
