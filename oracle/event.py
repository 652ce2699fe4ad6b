"""Event-driven operators (test infrastructure only).

Semantics restated from the reference's call sites and tests; the arithmetic itself
lives in the un-vendored ``brainevent>=0.0.7`` (pyproject.toml:60), which is absent:

  * ``EventArray(spk) @ FixedPostNumConn((w, idx))`` -- brainstate/nn/_event_fixedprob.py:202-205,
    249-252.  Every nonzero spike is one event; ``out[j] = sum over events (i, k)
    with idx[i, k] == j of w[i, k]`` (scalar w: homogeneous).  Pinned by the
    reference test brainstate/nn/_event_fixedprob_test.py:247-260 (``np.add.at``
    closed form), by brute force on tiny inputs and by scatter == gather.
  * ``EventLinear`` -- brainstate/nn/_event_linear.py:75-102.  Homogeneous weight:
    ``ones(n_out) * (count * w)`` (float_as_event) or ``sum(spk) * w``; otherwise
    the sum of the weight rows selected by nonzero spikes (float_as_event) or
    ``spk @ W``.  Pinned by brainstate/nn/_event_linear_test.py:26-40,127-162.
  * spike compaction has no reference function (brainevent skips zeros inside its
    loops); it is ``np.flatnonzero`` (ascending), pinned as a textbook routine.
  * Derivatives (brainstate/nn/_event_fixedprob_test.py:56-126,
    brainstate/nn/_event_linear_test.py:51-125): the reference's "true gradients" are those
    of the value formulations ``y[j] = sum_{i,k: idx=j} x[i] * w[i,k]`` and ``y = x @ W``
    (x = spike values), with a homogeneous weight broadcast to every synapse.  ``*_vjp``
    and ``*_jvp`` below restate them in float64; they are pinned by the adjoint identity
    <g, A v> = <A^T g, v>, by the exact bilinear expansion of f(x + dx, w + dw), and by the
    dense-matrix formulas (tests/test_oracle_event.py).

Summation order: the oracle adds events to ``out[j]`` in ascending (pre i, k) order
starting from 0.0f.  brainevent's own order is unpinned (no reference vector fixes
it), so fp32 heterogeneous sums from an order-free (atomic) device path are compared
within rtol 1e-5 / atol 1e-6.  Sums of one repeated weight value are order-free in
fp32 (every order performs the same sequence of additions) and compare bit-exactly.
"""
import numpy as np

F = np.float32


def compact(spk):
    """bool/float [n] -> ascending int32 indices of nonzero entries, count."""
    idx = np.flatnonzero(np.asarray(spk) != 0).astype(np.int32)
    return idx, int(idx.size)


def scatter_fixed(spk, idx, w, n_post):
    """Pre-major event mat-vec for fixed-num connectivity ``idx[n_pre, K]``.

    ``w`` is a scalar (homogeneous) or an ``[n_pre, K]`` array.  fp32, events added
    in ascending (i, k) order.
    """
    idx = np.asarray(idx)
    n_pre, k = idx.shape
    indptr = np.arange(n_pre + 1, dtype=np.int64) * k
    return scatter_csr(spk, indptr, idx.reshape(-1),
                       w if np.ndim(w) == 0 else np.asarray(w).reshape(-1), n_post)


def scatter_csr(spk, indptr, indices, w, n_post):
    out = np.zeros(n_post, dtype=F)
    active = np.flatnonzero(np.asarray(spk) != 0)
    homo = np.ndim(w) == 0
    wf = F(w) if homo else np.asarray(w, dtype=F)
    if active.size == 0:
        return out
    # Gather the events in (i, k) order, then accumulate per target in that order.
    starts = np.asarray(indptr, dtype=np.int64)[active]
    ends = np.asarray(indptr, dtype=np.int64)[active + 1]
    lens = ends - starts
    syn = np.concatenate([np.arange(s, e) for s, e in zip(starts, ends)]) if lens.sum() else \
        np.zeros(0, np.int64)
    tgt = np.asarray(indices, dtype=np.int64)[syn]
    vals = np.full(syn.size, wf, dtype=F) if homo else wf[syn]
    _ordered_add(out, tgt, vals)
    return out


def _ordered_add(out, tgt, vals):
    """out[tgt[e]] += vals[e] for e ascending, each add rounded to fp32."""
    if tgt.size == 0:
        return
    order = np.argsort(tgt, kind='stable')
    t = tgt[order]
    v = vals[order]
    bounds = np.flatnonzero(np.diff(t)) + 1
    seg_start = np.concatenate([[0], bounds])
    seg_end = np.concatenate([bounds, [t.size]])
    # Sequential fp32 accumulation per segment, vectorised over segments by position.
    lens = seg_end - seg_start
    acc = np.zeros(seg_start.size, dtype=F)
    for p in range(int(lens.max())):
        m = lens > p
        acc[m] = (acc[m] + v[seg_start[m] + p]).astype(F)
    out[t[seg_start]] = acc   # out is all zeros on entry


def gather_post_major(spk, post_indptr, pre_of, w_post, n_post):
    """Deterministic post-major gather: out[j] = sum over incoming (i) in list order.

    ``w_post`` is a scalar or the weights permuted into post-major order.
    """
    spk = np.asarray(spk) != 0
    homo = np.ndim(w_post) == 0
    out = np.zeros(n_post, dtype=F)
    lens = np.diff(post_indptr)
    act = spk[pre_of]
    vals = np.where(act, F(w_post) if homo else np.asarray(w_post, F), F(0)).astype(F)
    acc = np.zeros(n_post, dtype=F)
    for p in range(int(lens.max()) if lens.size else 0):
        m = lens > p
        pos = post_indptr[:-1][m] + p
        sel = act[pos]
        a = acc[m]
        a[sel] = (a[sel] + vals[pos][sel]).astype(F)
        acc[m] = a
    out[:] = acc
    return out


def event_linear(spk, W, float_as_event=True, n_out=None, chunk_rows=None):
    """brainstate/nn/_event_linear.py:75-102 for spk [..., n_in], W [n_in, n_out] or scalar.

    Heterogeneous W: each output is a sum of fp32 terms; with ``chunk_rows`` = L the inputs
    are cut into chunks of L consecutive rows, each chunk summed in ascending order from 0,
    and the chunk sums added in chunk order (the order the device kernel documents);
    ``chunk_rows=None`` is the plain ascending sum."""
    spk = np.asarray(spk)
    if np.ndim(W) == 0 or np.size(W) == 1:
        w = F(np.asarray(W).reshape(()))
        if float_as_event:
            reduced = np.sum(spk != 0, axis=-1).astype(F)
        else:
            reduced = np.sum(spk.astype(F), axis=-1, dtype=F)
        return (np.ones(spk.shape[:-1] + (n_out,), F) *
                np.asarray(reduced * w, F)[..., None]).astype(F)
    W = np.asarray(W, dtype=F)
    x = spk.reshape(-1, spk.shape[-1])
    n_in = x.shape[1]
    L = n_in if chunk_rows is None else int(chunk_rows)
    out = np.zeros((x.shape[0], W.shape[1]), dtype=F)
    for b in range(x.shape[0]):
        for c, lo in enumerate(range(0, max(n_in, 1), max(L, 1))):
            part = np.zeros(W.shape[1], dtype=F)
            for i in lo + np.flatnonzero(x[b, lo:lo + L] != 0):
                term = W[i] if float_as_event else (F(x[b, i]) * W[i]).astype(F)
                part = (part + term).astype(F)
            out[b] = part if c == 0 else (out[b] + part).astype(F)
    return out.reshape(spk.shape[:-1] + (W.shape[1],))


# ---- destination-bucketed operator: exact fixed-point sums ----

def fixed_point_qexp(wmax, D):
    """The fixed-point exponent rule of the persistent runner and the bucketed operator (csrc
    network.hip k_qexp, event_bucket.hip k_bucket_qexp): with W = ``wmax`` (fp32 max |w|),
    W < 2^e_w (e_w from W's exponent field; -126 for a zero or subnormal W) and the largest
    in-degree D <= 2^e_d, S = min(30 - e_w - e_d, 100).  Every output's sum of
    rint(w * 2^S) then has magnitude < 2^30 + D/2.  -1000 when W is not finite or S < -100."""
    wb = int(np.asarray(wmax, F).reshape(()).view(np.uint32)) & 0x7FFFFFFF
    if wb >= 0x7F800000:
        return -1000
    e_w = (wb >> 23) - 126 if (wb >> 23) else -126
    D = int(D)
    e_d = (D - 1).bit_length() if D > 1 else 0
    S = min(30 - e_w - e_d, 100)
    return -1000 if S < -100 else S


def bucket_qexp(w, targets, n_post):
    """Fixed-point exponent S of the bucketed layout: ``fixed_point_qexp`` over the valid
    synapses (0 <= target < n_post) -- W their largest |w|, D the most of them onto one post.
    ``w`` and ``targets`` are per synapse (same length)."""
    w = np.asarray(w, dtype=F).reshape(-1)
    t = np.asarray(targets).reshape(-1).astype(np.int64)
    ok = (t >= 0) & (t < n_post)
    wv, tv = np.abs(w[ok]), t[ok]
    if wv.size and not np.all(np.isfinite(wv)):
        return -1000
    wmax = wv.max() if wv.size else F(0)
    D = int(np.bincount(tv, minlength=n_post).max()) if tv.size else 0
    return fixed_point_qexp(wmax, D)


def scatter_fixed_point(spk, indptr, indices, w, n_post, S):
    """Event mat-vec with each weight rounded to a multiple of 2^-S (round half to even), the
    rounded weights of the events onto each output summed exactly, the sum rounded once to
    fp32 and scaled by 2^-S.  Out-of-range targets contribute nothing."""
    indptr = np.asarray(indptr, dtype=np.int64)
    indices = np.asarray(indices, dtype=np.int64)
    w = np.asarray(w, dtype=F).reshape(-1)
    acc = np.zeros(n_post, dtype=np.int64)
    for i in np.flatnonzero(np.asarray(spk) != 0):
        lo, hi = indptr[i], indptr[i + 1]
        t = indices[lo:hi]
        keep = (t >= 0) & (t < n_post)
        q = np.rint(np.ldexp(w[lo:hi][keep].astype(np.float64), S)).astype(np.int64)
        np.add.at(acc, t[keep], q)
    return np.ldexp(acc.astype(F), -S).astype(F)



# ---- packed EventLinear: exact fixed-point sums per column ----

def dense_digits(n_in):
    """Signed 8-bit digits L of the packed EventLinear form: the smallest L in 4..6 with
    8 L - 2 >= 24 + ceil(log2 n_in); 0 when n_in > 65536 (not packable)."""
    n_in = int(n_in)
    if n_in < 0 or n_in > 65536:
        return 0
    c = 0
    while (1 << c) < max(n_in, 1):
        c += 1
    for L in (4, 5, 6):
        if 8 * L - 2 >= 24 + c:
            return L
    return 0


def dense_column_shifts(W):
    """S_j = D - e_j with D = 8 L - 2 and max_i |W[i, j]| = f * 2^e_j (f in [0.5, 1)); 0 for a
    column of zeros.  Returns (S int32 [n_out], zero-column mask)."""
    W = np.asarray(W, dtype=F)
    n_in, n_out = W.shape
    D = 8 * dense_digits(n_in) - 2
    m = np.abs(W).max(axis=0) if n_in else np.zeros(n_out, F)
    e = np.frexp(m.astype(np.float64))[1].astype(np.int64)
    zero = m == 0
    return np.where(zero, 0, D - e).astype(np.int32), zero


def _exact_int_matmul(a01, q):
    """a01 (0/1 int) @ q (int64, |q| <= 2^46, n_in <= 65536) exactly, through float64 BLAS on
    24-bit halves: every partial sum stays below 2^53, so each float64 sum is exact."""
    hi = q >> 24
    lo = q - (hi << 24)                       # in [0, 2^24)
    a = a01.astype(np.float64)
    s_hi = (a @ hi.astype(np.float64)).astype(np.int64)
    s_lo = (a @ lo.astype(np.float64)).astype(np.int64)
    return (s_hi << 24) + s_lo


def event_dense_fixed_point(spk, W):
    """Packed EventLinear (event spikes: any nonzero is an event): each weight rounded to a
    multiple of 2^-S_j of its column (round half to even), the rounded weights selected by
    each batch row summed exactly, the sum rounded once to fp32 and scaled by 2^-S_j; a
    column of zeros gives +0.  Any non-finite weight: every output NaN."""
    W = np.asarray(W, dtype=F)
    spk = np.asarray(spk)
    x = spk.reshape(-1, W.shape[0])
    if not np.all(np.isfinite(W)):
        return np.full(spk.shape[:-1] + (W.shape[1],), np.nan, F)
    S, zero = dense_column_shifts(W)
    q = np.rint(np.ldexp(W.astype(np.float64), S[None, :].astype(np.int64))).astype(np.int64)
    tot = _exact_int_matmul((x != 0).astype(np.int8), q)
    out = np.ldexp(tot.astype(F), (-S)[None, :]).astype(F)
    out[:, zero] = F(0.0)
    return out.reshape(spk.shape[:-1] + (W.shape[1],))

# ---- derivatives (float64) ----

def _rows_of(idx, indptr):
    """(row of each synapse, target of each synapse) for fixed-num or CSR connectivity."""
    if indptr is None:
        idx = np.asarray(idx)
        return np.repeat(np.arange(idx.shape[0]), idx.shape[1]), idx.reshape(-1)
    indptr = np.asarray(indptr, np.int64)
    return np.repeat(np.arange(indptr.size - 1), np.diff(indptr)), np.asarray(idx).reshape(-1)


def value_matvec(x, idx, w, n_post, indptr=None):
    """y[j] = sum_{s: tgt[s] = j} x[row[s]] * w[s] in float64 (w scalar: homogeneous)."""
    row, tgt = _rows_of(idx, indptr)
    ws = np.broadcast_to(np.asarray(w, np.float64), tgt.shape) if np.ndim(w) == 0 else \
        np.asarray(w, np.float64).reshape(-1)
    y = np.zeros(n_post, np.float64)
    np.add.at(y, tgt, np.asarray(x, np.float64)[row] * ws)
    return y


def matvec_vjp(x, idx, w, n_post, g, indptr=None):
    """(grad_x [n_pre], grad_w) of <g, value_matvec(x, idx, w)>; grad_w has w's shape (a
    float for a scalar w)."""
    row, tgt = _rows_of(idx, indptr)
    g = np.asarray(g, np.float64)
    x = np.asarray(x, np.float64)
    gt = g[tgt]
    n_pre = x.size
    if np.ndim(w) == 0:
        gx = np.bincount(row, weights=gt * float(w), minlength=n_pre)
        gw = float(np.sum(x[row] * gt))
    else:
        ws = np.asarray(w, np.float64).reshape(-1)
        gx = np.bincount(row, weights=gt * ws, minlength=n_pre)
        gw = (x[row] * gt).reshape(np.shape(w))
    return gx, gw


def matvec_jvp(x, dx, idx, w, dw, n_post, indptr=None):
    """Tangent of value_matvec at (x, w) along (dx, dw): A(w) dx + A(dw) x."""
    t = np.zeros(n_post, np.float64)
    if dx is not None:
        t += value_matvec(dx, idx, w, n_post, indptr)
    if dw is not None:
        t += value_matvec(x, idx, dw, n_post, indptr)
    return t


def dense_vjp(x, W, g):
    """(grad_x, grad_W) of <g, x @ W> for x [B, n_in], W [n_in, n_out], g [B, n_out]."""
    x = np.asarray(x, np.float64)
    W = np.asarray(W, np.float64)
    g = np.asarray(g, np.float64)
    return g @ W.T, x.T @ g
