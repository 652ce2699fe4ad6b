"""Whole E/I network loops (test infrastructure only).

Per-step order of the reference's E/I nets (examples/105_COBA_HH_2007_braincell.py:76-82,
examples/400_CUBA_2005_bpu.py:60-65, docs/tutorials/brain_dynamics/04_building_an_snn.ipynb
cell 11): the spikes of the previous step drive the E projection (pre = neurons
[0, n_exc)) and the I projection (pre = [n_exc, N)), each an event mat-vec onto all N
neurons; then the neurons advance with those inputs (Expon decay + delta input,
COBA current, membrane exp-Euler, spike).  Connectivity per projection is
``EventFixedProb(n_pre, N, conn_num, w, seed)`` (brainstate/nn/_event_fixedprob.py:102-200).

With a synaptic delay of D steps the projections read the neurons' spikes through a
``Delay`` (restated in ``oracle.delay``) updated after every step and read at step D --
what ``N.prefetch_delay('spike', D*dt)`` gives (brainstate/nn/_dynamics.py:222-262,
686-745): step t's inputs come from step t-1-D's spikes, and from no spikes before step 0.
"""
import numpy as np

from . import conn as _conn
from . import delay as _delay
from . import event as _event
from . import neuron as _neuron

F = np.float32


def repeated_sum_table(w, max_count):
    """t[c] = w + w + ... (c times) in fp32, sequentially; order-free for one value."""
    t = np.zeros(max_count + 1, dtype=F)
    s = F(0.0)
    w = F(w)
    for c in range(1, max_count + 1):
        s = F(s + w)
        t[c] = s
    return t


def runner_qexp(idx, w, n_post):
    """Fixed-point exponent S of one projection's per-synapse weights, as the persistent
    runner fixes it: with D = the largest number of the projection's synapses onto one
    neuron (valid targets) and W = max |w| < 2^e_w (e_w from W's exponent field; -126 for a
    zero or subnormal W), D <= 2^e_d, S = min(30 - e_w - e_d, 100).  Every neuron's sum of
    rint(w * 2^S) then has magnitude < 2^30 + D/2 < 2^31."""
    idx = np.asarray(idx)
    w = np.ascontiguousarray(np.broadcast_to(np.asarray(w, F), idx.shape))
    t = idx.reshape(-1)
    t = t[(t >= 0) & (t < n_post)]
    D = int(np.bincount(t, minlength=n_post).max()) if t.size else 0
    wb = int((w.view(np.uint32) & np.uint32(0x7FFFFFFF)).max()) if w.size else 0
    if wb >= 0x7F800000:
        raise ValueError('a per-synapse weight is not finite')
    S = _event.fixed_point_qexp(np.uint32(wb).view(F), D)
    if S == -1000:
        raise ValueError('per-synapse weights too large for the fixed-point input sums')
    return S


def fixed_point_input(spk_pre, idx, w, S, n_post):
    """The runner's input of one projection with per-synapse weights: every weight of an
    event onto j rounded to a multiple of 2^-S (round half to even), the rounded weights
    summed exactly, the sum converted to fp32 once and scaled by 2^-S."""
    act = np.flatnonzero(spk_pre)
    q = np.rint(np.asarray(w, F)[act] * F(2.0 ** S)).astype(np.int64).reshape(-1)
    t = np.asarray(idx)[act].reshape(-1)
    ok = (t >= 0) & (t < n_post)
    acc = np.zeros(n_post, np.int64)
    np.add.at(acc, t[ok], q[ok])
    assert np.abs(acc).max(initial=0) < 2 ** 31
    return (acc.astype(F) * F(2.0 ** -S)).astype(F)


class Projection:
    """One fixed-num projection (pre block of the neuron vector -> all N).

    ``w``: one value (homogeneous; ``het=True`` stores it per synapse) or an array of
    per-synapse weights of the connectivity's shape.  ``fixed=True`` sums per-synapse weights
    as the persistent runner does (``fixed_point_input``); otherwise in the sequential
    (pre, k) order of a plain scatter.  Sums of one repeated value use the repeated-sum table
    either way (order-free)."""

    def __init__(self, pre_lo, pre_hi, n_post, conn_num, w, seed, het=False, fixed=False):
        self.pre_lo, self.pre_hi, self.n_post = pre_lo, pre_hi, n_post
        self.k = _conn.conn_num_from(conn_num, n_post)
        self.idx, _ = _conn.fixed_num_indices(pre_hi - pre_lo, n_post, self.k, seed)
        if np.ndim(w) > 0:
            self.w = np.ascontiguousarray(np.broadcast_to(np.asarray(w, F), self.idx.shape))
            self.w_scalar = self.w.reshape(-1)[0] if self.w.size else F(0)
            self.het = True
        else:
            self.w_scalar = F(w)
            self.het = het
            self.w = np.full(self.idx.shape, F(w), F) if het else F(w)
        self.fixed = fixed
        self.S = runner_qexp(self.idx, self.w, n_post) if (self.het and fixed) else None
        self._table = None

    def __call__(self, spk_pre):
        if self.het and self.fixed:
            return fixed_point_input(spk_pre, self.idx, self.w, self.S, self.n_post)
        if not self.het or np.all(self.w == self.w_scalar):
            # one repeated weight value: counts + repeated-sum table (exact, order-free)
            act = np.flatnonzero(spk_pre)
            counts = np.bincount(self.idx[act].reshape(-1), minlength=self.n_post)
            mc = int(counts.max()) if counts.size else 0
            if self._table is None or self._table.size <= mc:
                self._table = repeated_sum_table(self.w_scalar, max(mc, 64))
            return self._table[counts]
        return _event.scatter_fixed(spk_pre, self.idx, self.w, self.n_post)


def _spike_delay(N, delay_steps, delay_state):
    """Spike history read at step D (None for D = 0: the previous step's spikes)."""
    if not delay_steps:
        return None
    d = _delay.Delay((N,), np.bool_)
    d.register_entry('spike', None)
    d.max_length = int(delay_steps) + 1
    d.init_state()
    if delay_state is not None:
        d.history[...] = delay_state[0]
        d.write_ptr = int(delay_state[1])
    return d


def run_coba_lif(V0, proj_e, proj_i, p, n_exc, steps, record_raster=True, init=None,
                 delay_steps=0, delay_state=None):
    """COBA LIFRef network.  Returns dict(raster [T,N] bool, counts [T], final state)."""
    N = V0.size
    hist = _spike_delay(N, delay_steps, delay_state)
    if init is None:
        V = np.asarray(V0, F).copy()
        ge = np.zeros(N, F)
        gi = np.zeros(N, F)
        ref = np.zeros(N, np.int32)
        spk = np.zeros(N, bool)
    else:
        V, ge, gi, ref, spk = [np.array(a) for a in init]
    raster = np.zeros((steps, N), bool) if record_raster else None
    counts = np.zeros(steps, np.int64)
    for t in range(steps):
        src = spk if hist is None else hist.retrieve_at_step(delay_steps)
        in_e = proj_e(src[:n_exc])
        in_i = proj_i(src[n_exc:])
        V, ge, gi, ref, spk = _neuron.coba_lif_step(V, ge, gi, ref, in_e, in_i, p, spk)
        if hist is not None:
            hist.update(spk)
        if record_raster:
            raster[t] = spk
        counts[t] = spk.sum()
    return dict(raster=raster, counts=counts, V=V, ge=ge, gi=gi, ref=ref, spk=spk,
                delay_state=None if hist is None else (hist.history.copy(), hist.write_ptr))


def run_coba_hh(V0, proj_e, proj_i, p, n_exc, steps, record_raster=True, init=None,
                delay_steps=0, delay_state=None):
    """COBA Hodgkin-Huxley network (exp-Euler gates)."""
    N = V0.size
    hist = _spike_delay(N, delay_steps, delay_state)
    if init is None:
        V = np.asarray(V0, F).copy()
        m, h, n = _neuron.hh_init(V)
        ge = np.zeros(N, F)
        gi = np.zeros(N, F)
        spk = np.zeros(N, bool)
    else:
        V, m, h, n, ge, gi, spk = [np.array(a) for a in init]
    raster = np.zeros((steps, N), bool) if record_raster else None
    counts = np.zeros(steps, np.int64)
    for t in range(steps):
        src = spk if hist is None else hist.retrieve_at_step(delay_steps)
        in_e = proj_e(src[:n_exc])
        in_i = proj_i(src[n_exc:])
        V, m, h, n, ge, gi, spk = _neuron.hh_step(V, m, h, n, ge, gi, in_e, in_i, p)
        if hist is not None:
            hist.update(spk)
        if record_raster:
            raster[t] = spk
        counts[t] = spk.sum()
    return dict(raster=raster, counts=counts, V=V, m=m, h=h, n=n, ge=ge, gi=gi, spk=spk,
                delay_state=None if hist is None else (hist.history.copy(), hist.write_ptr))


def spike_hash(spk):
    """Order-free 32-bit digest of a spike set: sum over spiking i of mix32(i) mod 2^32."""
    i = np.flatnonzero(spk).astype(np.uint64)
    return int(np.sum(mix32(i), dtype=np.uint64) & np.uint64(0xFFFFFFFF))


def mix32(i):
    """32-bit integer hash (Murmur3 finaliser) on uint64 arrays, result < 2^32."""
    M = np.uint64(0xFFFFFFFF)
    x = np.asarray(i, np.uint64) & M
    x = (x ^ (x >> np.uint64(16))) & M
    x = (x * np.uint64(0x85EBCA6B)) & M
    x = (x ^ (x >> np.uint64(13))) & M
    x = (x * np.uint64(0xC2B2AE35)) & M
    x = (x ^ (x >> np.uint64(16))) & M
    return x
