"""Pins of the oracle's connectivity and event operators (CPU only)."""
import hashlib
import json
import os

import numpy as np
import pytest

from oracle import conn, event, network

F = np.float32
GOLD = os.path.join(os.path.dirname(__file__), 'golden')


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ---- connectivity: brainstate/nn/_event_fixedprob.py:142-196 ----

def test_conn_num_from_probability():
    assert conn.conn_num_from(0.02, 4000) == 80          # int(n_post * p), :144
    assert conn.conn_num_from(0.2, 30) == 6
    assert conn.conn_num_from(7, 30) == 7


def test_indices_are_numpy_mt19937_stream():
    idx, _ = conn.fixed_num_indices(20, 30, 6, seed=11)
    ref = np.random.RandomState(11).randint(0, 30, size=(20, 6)).astype(np.int32)
    assert idx.dtype == np.int32 and np.array_equal(idx, ref)
    assert idx.min() >= 0 and idx.max() < 30


def test_indices_golden_digests():
    with open(os.path.join(GOLD, 'conn_digests.json')) as f:
        gold = json.load(f)
    for case in gold:
        idx, _ = conn.fixed_num_indices(case['n_pre'], case['n_post'], case['k'], case['seed'])
        assert _sha(idx) == case['sha256'], case


def test_csr_afferent_indptr_closed_form():
    indptr, indices, sel = conn.csr_afferent(50, 40, 5, seed=3, afferent_ratio=0.5)
    assert indptr[0] == 0 and indptr[-1] == indices.size == 5 * sel.sum()
    assert np.array_equal(np.diff(indptr), np.where(sel, 5, 0))
    # the mask is drawn after the indices from the same generator (:183-184)
    rng = np.random.RandomState(3)
    full = rng.randint(0, 40, size=(50, 5))
    assert np.array_equal(sel, rng.random(50) < 0.5)
    assert np.array_equal(indices, full[sel].reshape(-1))


# ---- event mat-vec: brainstate/nn/_event_fixedprob_test.py:247-260 ----

def test_scatter_matches_reference_np_add_at():
    n_in, n_out = 20, 30
    idx, _ = conn.fixed_num_indices(n_in, n_out, conn.conn_num_from(0.2, n_out), seed=11)
    spk = (np.random.RandomState(1).rand(n_in) < 0.3).astype(float)
    out = event.scatter_fixed(spk, idx, 1.5, n_out)
    ref = np.zeros(n_out)
    for i in range(n_in):
        np.add.at(ref, idx[i], 1.5 * float(spk[i]))
    assert np.allclose(out, ref, rtol=1e-4, atol=1e-4)


def test_scatter_brute_force_het_exact_order():
    rng = np.random.RandomState(5)
    n_pre, n_post, k = 37, 23, 9
    idx = rng.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = rng.normal(0.5, 0.1, (n_pre, k)).astype(F)
    spk = rng.rand(n_pre) < 0.4
    out = event.scatter_fixed(spk, idx, w, n_post)
    ref = np.zeros(n_post, F)
    for i in range(n_pre):               # sequential fp32 adds in (i, k) order
        if spk[i]:
            for kk in range(k):
                ref[idx[i, kk]] = F(ref[idx[i, kk]] + w[i, kk])
    assert np.array_equal(out, ref)


def test_scatter_invariant_total_mass():
    rng = np.random.RandomState(6)
    idx = rng.randint(0, 500, (400, 50)).astype(np.int32)
    w = rng.normal(0.5, 0.1, (400, 50)).astype(F)
    spk = rng.rand(400) < 0.1
    out = event.scatter_fixed(spk, idx, w, 500)
    assert np.isclose(out.astype(np.float64).sum(), w[spk].astype(np.float64).sum(), rtol=1e-5)


def test_float_spikes_count_as_events():
    idx = np.array([[0, 1], [1, 2]], np.int32)
    a = event.scatter_fixed(np.array([2.5, 0.0]), idx, 1.0, 3)
    b = event.scatter_fixed(np.array([1, 0], bool), idx, 1.0, 3)
    assert np.array_equal(a, b) and np.array_equal(a, [1, 1, 0])


@pytest.mark.parametrize('het', [False, True])
def test_gather_equals_scatter_bitwise(het):
    rng = np.random.RandomState(7)
    n_pre, n_post, k = 300, 200, 40
    idx = rng.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = rng.normal(0.5, 0.1, (n_pre, k)).astype(F) if het else F(0.6)
    spk = rng.rand(n_pre) < 0.2
    indptr, flat = conn.fixed_to_csr(idx)
    post_ptr, pre_of, syn_of = conn.to_post_major(indptr, flat, n_post)
    w_post = w.reshape(-1)[syn_of] if het else w
    g = event.gather_post_major(spk, post_ptr, pre_of, w_post, n_post)
    s = event.scatter_fixed(spk, idx, w, n_post)
    assert np.array_equal(g, s)


def test_homogeneous_counts_are_repeated_sums():
    t = network.repeated_sum_table(0.6, 10)
    assert t[0] == 0 and t[1] == F(0.6) and t[2] == F(1.2) and t[3] == F(F(1.2) + F(0.6))
    rng = np.random.RandomState(8)
    idx = rng.randint(0, 50, (100, 20)).astype(np.int32)
    spk = rng.rand(100) < 0.5
    counts = np.bincount(idx[spk].reshape(-1), minlength=50)
    assert np.array_equal(event.scatter_fixed(spk, idx, 0.6, 50),
                          network.repeated_sum_table(0.6, counts.max())[counts])


def test_compact_is_flatnonzero():
    spk = np.random.RandomState(9).rand(10000) < 0.01
    idx, c = event.compact(spk)
    assert c == spk.sum() and np.all(np.diff(idx) > 0) and np.array_equal(spk[idx], np.ones(c, bool))
    assert event.compact(np.zeros(0, bool))[1] == 0


# ---- EventLinear: brainstate/nn/_event_linear_test.py ----

@pytest.mark.parametrize('bool_x', [True, False])
@pytest.mark.parametrize('homo_w', [True, False])
def test_event_linear_reference_test1(homo_w, bool_x):          # :26-40
    rng = np.random.RandomState(10)
    x = rng.rand(20) < 0.1
    if not bool_x:
        x = x.astype(F)
    W = F(1.5) if homo_w else rng.uniform(-0.5, 0.5, (20, 40)).astype(F)
    y = event.event_linear(x, W, float_as_event=bool_x, n_out=40)
    expect = (x.sum() * W) * np.ones(40) if homo_w else x.astype(F) @ W
    assert np.allclose(y, expect, rtol=1e-5)


@pytest.mark.parametrize('float_as_event', [True, False])
def test_event_linear_homogeneous_matches_dense(float_as_event):  # :127-162
    spk = np.array([0., 2., 0., 3., 0., 0., 1., 0., 0., 5.], F)
    homo = event.event_linear(spk, F(1.5), float_as_event, n_out=8)
    dense = event.event_linear(spk, np.full((10, 8), 1.5, F), float_as_event)
    assert np.allclose(homo, dense)
    expected = (4 if float_as_event else 11) * 1.5
    assert np.allclose(homo, np.ones(8) * expected)


def test_event_linear_batched_equals_rows():
    rng = np.random.RandomState(11)
    spk = rng.rand(5, 64) < 0.2
    W = rng.normal(0, 0.125, (64, 33)).astype(F)
    out = event.event_linear(spk, W)
    for b in range(5):
        assert np.array_equal(out[b], event.event_linear(spk[b], W))
    assert np.allclose(out, spk.astype(np.float64) @ W.astype(np.float64), atol=1e-5)


@pytest.mark.parametrize('L', [64, 128, 192, 1000, 4096])
def test_event_linear_chunked_order(L):
    """Chunked sums: integer-valued weights make every order exact, so the chunked oracle must
    equal the integer product (a row dropped or counted twice at a chunk boundary fails);
    L >= n_in is the plain ascending sum; real weights stay within fp32 rounding of float64."""
    rng = np.random.RandomState(L)
    n_in = 1000
    spk = rng.rand(6, n_in) < 0.1
    Wi = rng.randint(-8, 9, (n_in, 24)).astype(F)
    assert np.array_equal(event.event_linear(spk, Wi, chunk_rows=L),
                          (spk.astype(np.int64) @ Wi.astype(np.int64)).astype(F))
    x = np.where(spk, rng.rand(6, n_in) * 3, 0).astype(F)
    Wf = rng.normal(0, 0.125, (n_in, 24)).astype(F)
    got = event.event_linear(x, Wf, float_as_event=False, chunk_rows=L)
    assert np.allclose(got, x.astype(np.float64) @ Wf.astype(np.float64), rtol=1e-5, atol=1e-5)
    if L >= n_in:
        assert np.array_equal(got, event.event_linear(x, Wf, float_as_event=False))
    else:  # a different grouping of the same terms: equal up to rounding, not bit for bit
        assert not np.array_equal(event.event_linear(spk, Wf, chunk_rows=L),
                                  event.event_linear(spk, Wf))


# ---- bucketed operator: fixed-point exponent and exact sums ----

def test_bucket_qexp_bounds_every_sum():
    """S = min(30 - e_w - e_d, 100) keeps every output's sum of rounded weights below 2^30 in
    magnitude (D synapses of |w| <= W onto one output: D * W * 2^S < 2^30) and lies within a
    factor 4 of the largest S that does (D * W * 2^S > 2^28 unless capped at 100), so a wrong
    offset or a dropped term fails; rint(w * 2^S) computed in float64 equals its fp32 form
    (ldexp, rint, convert) for every weight, tiny ones included.  The rule is the runner's:
    equal to oracle.network.runner_qexp on the same projection."""
    from oracle import network
    rng = np.random.RandomState(3)
    for _ in range(200):
        n_post = int(rng.randint(1, 50))
        D = int(rng.randint(1, 3000))
        wmax = F(rng.lognormal(0, 8))
        # output 0 receives D synapses, the others fewer
        t = np.concatenate([np.zeros(D, np.int64), rng.randint(0, n_post, D // 2)])
        t[D:][t[D:] == 0] = n_post - 1 if n_post > 1 else -1
        w = (rng.uniform(-1, 1, t.size) * wmax).astype(F)
        w[0] = -wmax
        S = event.bucket_qexp(w, t, n_post)
        Dm = int(np.bincount(t[t >= 0], minlength=n_post).max())
        assert Dm == D
        assert float(wmax) * Dm * 2.0 ** S < 2.0 ** 30
        assert S == 100 or float(wmax) * Dm * 2.0 ** S > 2.0 ** 28
        assert S == network.runner_qexp(t[t >= 0].reshape(1, -1), w[t >= 0].reshape(1, -1),
                                        n_post)
        ws = np.concatenate([w, (rng.uniform(-1, 1, 100) * wmax * F(1e-30)).astype(F)])
        exact = np.rint(ws.astype(np.float64) * 2.0 ** S)
        f32 = np.rint(np.ldexp(ws, S).astype(F)).astype(np.float64)
        assert np.array_equal(exact, f32) and np.abs(exact).max() <= 2.0 ** 30
    t1 = np.zeros(1, np.int64)
    assert event.bucket_qexp(np.zeros(5, F), np.arange(5), 5) == 100     # W = 0: capped
    assert event.bucket_qexp(np.array([1.0, np.inf], F), np.arange(2), 2) == -1000
    assert event.bucket_qexp(np.array([np.nan], F), t1, 1) == -1000
    assert event.bucket_qexp(np.array([0.75], F), t1, 1) == 30          # 0.75 < 2^0, D = 1
    assert event.bucket_qexp(np.array([1.0, 1.0], F), np.zeros(2), 1) == 28   # 1 < 2^1, D = 2
    assert event.bucket_qexp(np.array([1.0, 1.0, 1.0], F), np.zeros(3), 1) == 27  # D = 3 <= 4
    # synapses onto invalid targets enter neither W nor D
    assert event.bucket_qexp(np.array([0.75, 8.0], F), np.array([0, 5]), 1) == 30
    assert event.fixed_point_qexp(F(3e38), 2 ** 31) == -1000           # S < -100


def test_fixed_point_scatter_is_the_rounded_exact_sum():
    """Weights that are multiples of 2^-S are exact, so the result is the exact sum rounded
    once (checked through float64, exact here); any event order gives the same bits; real
    weights stay within fp32 rounding of the float64 sum and of the sequential oracle."""
    rng = np.random.RandomState(11)
    n_pre, n_post, k = 400, 300, 30
    idx = rng.randint(0, n_post, (n_pre, k))
    indptr = np.arange(n_pre + 1) * k
    spk = rng.rand(n_pre) < 0.3
    S = event.bucket_qexp(np.ones(1, F), np.zeros(1), 1)
    wq = (rng.randint(-2**20, 2**20, n_pre * k) * 2.0 ** -18).astype(F)  # multiples of 2^-18
    got = event.scatter_fixed_point(spk, indptr, idx.reshape(-1), wq, n_post, S)
    exact = np.zeros(n_post)
    act = np.repeat(spk, k)
    np.add.at(exact, idx.reshape(-1)[act], wq[act].astype(np.float64))
    assert np.array_equal(got, exact.astype(F))
    perm = rng.permutation(k)  # reorder every row's synapses
    got2 = event.scatter_fixed_point(spk, indptr, idx[:, perm].reshape(-1),
                                     wq.reshape(n_pre, k)[:, perm].reshape(-1), n_post, S)
    assert np.array_equal(got, got2)
    w = rng.normal(0.5, 0.1, n_pre * k).astype(F)
    Sw = event.bucket_qexp(w, idx.reshape(-1), n_post)
    gw = event.scatter_fixed_point(spk, indptr, idx.reshape(-1), w, n_post, Sw)
    ref64 = np.zeros(n_post)
    np.add.at(ref64, idx.reshape(-1)[act], w[act].astype(np.float64))
    cnt = np.bincount(idx.reshape(-1)[act], minlength=n_post)
    # each event's weight rounded to a multiple of 2^-S, then one fp32 rounding of the sum
    assert np.all(np.abs(gw - ref64) <= cnt * 2.0 ** -(Sw + 1) + 2.0 ** -24 * np.abs(ref64))
    seq = event.scatter_csr(spk, indptr, idx.reshape(-1), w, n_post)
    assert np.allclose(gw, seq, rtol=1e-5, atol=1e-6)
    # a scale off by one bit would be caught
    assert not np.allclose(event.scatter_fixed_point(spk, indptr, idx.reshape(-1), w, n_post,
                                                     Sw) * 2, ref64, rtol=1e-3)



# ---- packed EventLinear: per-column fixed point ----

def test_dense_digits_table():
    """Smallest L with 8 L - 2 >= 24 + ceil(log2 n_in), at the boundaries of each L."""
    got = [event.dense_digits(n) for n in (0, 1, 64, 65, 16384, 16385, 65536, 65537, -1)]
    assert got == [4, 4, 4, 5, 5, 6, 6, 0, 0]


def test_dense_fixed_point_dyadic_weights_are_exact():
    """Weights with few significant bits relative to their column maximum are held exactly,
    so every output is the exact sum rounded once (float64 is exact here); the per-column
    scale is exercised by columns 2^40 apart."""
    rng = np.random.RandomState(21)
    n_in, n_out, B = 300, 40, 9
    W = (rng.randint(-2**10, 2**10, (n_in, n_out)) * 2.0 ** -12).astype(F)
    W[:, 5] *= F(2.0 ** -40)
    W[:, 6] *= F(2.0 ** 40)
    W[:, 7] = 0
    spk = (rng.rand(B, n_in) < 0.3).astype(np.uint8) * rng.randint(1, 4, (B, n_in)).astype(np.uint8)
    got = event.event_dense_fixed_point(spk, W)
    exact = ((spk != 0).astype(np.float64) @ W.astype(np.float64)).astype(F)
    assert np.array_equal(got, exact)
    assert np.all(got[:, 7] == 0) and not np.any(np.signbit(got[:, 7]))


def test_dense_fixed_point_ties_to_even_and_bound():
    """q = rint(w 2^S) rounds halves to even: with max|w| = 1 (e = 1) and n_in <= 64 (L = 4,
    D = 30, S = 29), 2^-30 becomes 0, 3 * 2^-30 becomes 2 * 2^-29 and 5 * 2^-30 becomes
    2 * 2^-29 (round half up would give 2^-29, 2 * 2^-29 and 3 * 2^-29).  On random weights each sum stays within 2^-24 max|W[:, j]|
    plus half an ulp of the exact sum, and within the tolerance of the sequential oracle."""
    W = np.zeros((4, 2), F)
    W[:, 0] = [1.0, 2.0 ** -30, 3 * 2.0 ** -30, 5 * 2.0 ** -30]
    W[:, 1] = [0.5, 0.25, -2.0 ** -31, 0.0]
    spk = np.array([[0, 1, 0, 0], [0, 0, 1, 0], [0, 0, 0, 1], [0, 1, 1, 1]], np.uint8)
    got = event.event_dense_fixed_point(spk, W)
    assert got[0, 0] == 0.0 and got[1, 0] == F(2.0 ** -28) and got[2, 0] == F(2.0 ** -28)
    assert got[3, 0] == F(4 * 2.0 ** -29)            # 0 + 2 + 2 units of 2^-29
    assert got[1, 1] == 0.0                          # -2^-31 * 2^30 = -0.5 -> 0 (even)
    rng = np.random.RandomState(5)
    for n_in, n_out, B in [(64, 33, 5), (1000, 50, 7), (20000, 8, 3)]:
        W = rng.normal(0, 0.125, (n_in, n_out)).astype(F)
        W[:, 0] *= F(1e-20)
        spk = rng.rand(B, n_in) < 0.1
        got = event.event_dense_fixed_point(spk, W).astype(np.float64)
        exact = spk.astype(np.float64) @ W.astype(np.float64)
        m = np.abs(W).max(axis=0).astype(np.float64)
        ulp = np.spacing(np.abs(exact).astype(F)).astype(np.float64)
        assert np.all(np.abs(got - exact) <= 2.0 ** -24 * m + 0.5 * ulp + 1e-300)
        seq = event.event_linear(spk, W)
        assert np.allclose(got, seq, rtol=1e-5, atol=1e-6 * m.max())
    assert np.all(np.isnan(event.event_dense_fixed_point(
        np.ones((2, 3), np.uint8), np.array([[1, 2], [np.inf, 0], [0, 1]], F))))

# ---- derivative restatements: pinned by identities, not by retyping the formulas ----

def _conn(seed, n_pre=40, n_post=30, k=5):
    rs = np.random.RandomState(seed)
    idx = rs.randint(0, n_post, (n_pre, k)).astype(np.int32)
    w = rs.randn(n_pre, k)
    x = rs.rand(n_pre) * (rs.rand(n_pre) < 0.4)
    return rs, idx, w, x


@pytest.mark.parametrize('homo', [False, True])
def test_matvec_vjp_adjoint_identity(homo):
    """<g, A(w) v> == <grad_x(g), v> for every v, and <g, A(u) x> == <grad_w(g), u>: a dropped
    term, a wrong index or a transposed operand breaks one of them."""
    rs, idx, w, x = _conn(3)
    if homo:
        w = 1.7
    g = rs.randn(30)
    gx, gw = event.matvec_vjp(x, idx, w, 30, g)
    for _ in range(3):
        v = rs.randn(40)
        assert np.isclose(g @ event.value_matvec(v, idx, w, 30), gx @ v)
        u = rs.randn() if homo else rs.randn(*idx.shape)
        assert np.isclose(g @ event.value_matvec(x, idx, u, 30), np.sum(np.asarray(gw) * u))


def test_matvec_vjp_against_dense_matrix_and_csr():
    rs, idx, w, x = _conn(5)
    A = np.zeros((40, 30))
    np.add.at(A, (np.repeat(np.arange(40), 5), idx.reshape(-1)), w.reshape(-1))
    g = rs.randn(30)
    gx, gw = event.matvec_vjp(x, idx, w, 30, g)
    assert np.allclose(gx, A @ g)
    assert np.allclose(gw, x[:, None] * g[idx])
    # CSR with the same rows gives the same gradients
    indptr = np.arange(41) * 5
    gx2, gw2 = event.matvec_vjp(x, idx.reshape(-1), w.reshape(-1), 30, g, indptr=indptr)
    assert np.allclose(gx2, gx) and np.allclose(gw2.reshape(40, 5), gw)


def test_matvec_jvp_is_bilinear_difference():
    """value_matvec is bilinear in (x, w): f(x+dx, w+dw) - f(x, w) - f(dx, dw) equals the
    tangent exactly (up to float64 rounding)."""
    rs, idx, w, x = _conn(9)
    dx, dw = rs.randn(40), rs.randn(*idx.shape)
    f = lambda a, b: event.value_matvec(a, idx, b, 30)
    t = event.matvec_jvp(x, dx, idx, w, dw, 30)
    assert np.allclose(t, f(x + dx, w + dw) - f(x, w) - f(dx, dw))


def test_dense_vjp_adjoint_identity():
    rs = np.random.RandomState(2)
    x, W, g = rs.randn(3, 7), rs.randn(7, 5), rs.randn(3, 5)
    gx, gW = event.dense_vjp(x, W, g)
    v, U = rs.randn(3, 7), rs.randn(7, 5)
    assert np.isclose(np.sum(g * (v @ W)), np.sum(gx * v))
    assert np.isclose(np.sum(g * (x @ U)), np.sum(gW * U))


def test_matvec_2000_matches_golden():
    """Config [2] at reduced size: the committed digests of the homogeneous, sequential
    per-synapse and fixed-point sums are what the oracle computes."""
    import hashlib
    import json
    import os
    import sys
    gdir = os.path.join(os.path.dirname(__file__), 'golden')
    sys.path.insert(0, gdir)
    import make_golden
    gold = json.load(open(os.path.join(gdir, 'matvec_2000.json')))
    c = gold['config']
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    for case in gold['cases']:
        spk, idx, w = make_golden.matvec_case(case['p'])
        assert int(spk.sum()) == case['active']
        assert sha(event.scatter_fixed(spk, idx, F(c['w_homo']), c['n_post'])) == \
            case['homo_sha256']
        assert sha(event.scatter_fixed(spk, idx, w, c['n_post'])) == case['het_sequential_sha256']
        S = event.bucket_qexp(w, idx, c['n_post'])
        indptr = np.arange(c['n_pre'] + 1, dtype=np.int64) * c['k']
        assert S == case['fixed_point_S']
        assert sha(event.scatter_fixed_point(spk, indptr, idx.reshape(-1), w, c['n_post'], S)) \
            == case['fixed_point_sha256']
