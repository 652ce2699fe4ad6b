"""Connectivity construction (test infrastructure only).

Restates brainstate/nn/_event_fixedprob.py:142-196:
  * ``conn_num`` given as a float p is ``int(n_post * p)`` (:142-146);
  * indices are ``RandomState(seed).randint(0, n_post, size=(n_pre, conn_num))``,
    with replacement (:161-168), cast to int32 (``environ.ditype()``, :171);
  * ``afferent_ratio < 1`` keeps pre rows with ``rng.random(n_pre) < ratio`` drawn
    from the same generator after the indices (:183-184) and builds a CSR with
    ``indptr = [0, cumsum(K * selected)]`` (:185-190).

Pinned by: NumPy's legacy MT19937 stream is frozen, so these arrays are the
reference's arrays bit for bit; tests/test_oracle_event.py checks the construction
branches against SHA-256 digests recorded in tests/golden/ and against the
closed-form indptr.

``to_post_major`` (transpose to a per-post incoming list, stable in (pre, k) order)
has no reference counterpart; it is pinned by the scatter == gather identity.
"""
import numpy as np


def conn_num_from(conn_num, n_post):
    """brainstate/nn/_event_fixedprob.py:142-147."""
    if isinstance(conn_num, float):
        assert 0. <= conn_num <= 1.
        conn_num = int(n_post * conn_num)
    assert isinstance(conn_num, int)
    return conn_num


def fixed_num_indices(n_pre, n_post, conn_num, seed):
    """brainstate/nn/_event_fixedprob.py:161-171 (allow_multi_conn=True)."""
    rng = np.random if seed is None else np.random.RandomState(seed)
    idx = rng.randint(0, n_post, size=(n_pre, conn_num))
    return np.asarray(idx, dtype=np.int32), rng


def csr_afferent(n_pre, n_post, conn_num, seed, afferent_ratio):
    """brainstate/nn/_event_fixedprob.py:183-196: returns (indptr, indices, selected)."""
    idx, rng = fixed_num_indices(n_pre, n_post, conn_num, seed)
    selected = rng.random(n_pre) < afferent_ratio
    indices = idx[selected].reshape(-1)
    indptr = (np.arange(1, n_pre + 1) * conn_num - np.cumsum(~selected) * conn_num)
    indptr = np.insert(indptr, 0, 0).astype(np.int32)
    return indptr, indices.astype(np.int32), selected


def fixed_to_csr(idx):
    n_pre, k = idx.shape
    indptr = (np.arange(n_pre + 1, dtype=np.int64) * k).astype(np.int32)
    return indptr, idx.reshape(-1).copy()


def to_post_major(indptr, indices, n_post):
    """Per-post incoming synapse lists in ascending (pre, k) order.

    Returns (post_indptr[n_post+1], pre_of[nnz], syn_of[nnz]) where syn_of is the
    flat index into the pre-major arrays (so a weight vector can be permuted).
    """
    indptr = np.asarray(indptr, dtype=np.int64)
    indices = np.asarray(indices, dtype=np.int64)
    nnz = indices.size
    pre = np.repeat(np.arange(indptr.size - 1, dtype=np.int64), np.diff(indptr))
    order = np.argsort(indices, kind='stable')     # stable keeps (pre, k) order
    counts = np.bincount(indices, minlength=n_post)
    post_indptr = np.zeros(n_post + 1, dtype=np.int64)
    np.cumsum(counts, out=post_indptr[1:])
    assert post_indptr[-1] == nnz
    return post_indptr, pre[order], order
