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


def event_linear(spk, W, float_as_event=True, n_out=None):
    """brainstate/nn/_event_linear.py:75-102 for spk [..., n_in], W [n_in, n_out] or scalar."""
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
    out = np.zeros((x.shape[0], W.shape[1]), dtype=F)
    for b in range(x.shape[0]):
        if float_as_event:
            for i in np.flatnonzero(x[b] != 0):
                out[b] = (out[b] + W[i]).astype(F)
        else:
            for i in np.flatnonzero(x[b] != 0):
                out[b] = (out[b] + F(x[b, i]) * W[i]).astype(F)
    return out.reshape(spk.shape[:-1] + (W.shape[1],))
