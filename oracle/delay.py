"""Ring-buffer delay (test infrastructure only).

Restates the semantics of brainstate's ``Delay`` (brainstate/nn/_delay.py:399-957), which the
device ``Delay`` and the runner's synaptic delay are checked against:

* ``delay_steps(time, dt)`` -- ``ceil(time / dt)`` evaluated in float32 (``_get_delay``,
  :351-360: ``jnp.ceil`` of the ratio; with x64 off a Python-float ratio is rounded to float32
  first, so 1.1 / 0.1 = 11.000000000000002 gives 11, not 12);
* ``max_length`` = ceil(time/dt) + 1, grown by every registration to max(step) + 1
  (:546-551, :678-686); ``max_time`` only grows (:678);
* ``update`` writes ``history[write_ptr // every] = x`` (every call, or only when
  ``write_ptr % every == 0`` with ``update_every``), then advances
  ``write_ptr = (write_ptr + 1) % (max_length * every)`` (:909-956);
* ``retrieve_at_step(d, *idx)`` reads ``history[((write_ptr - 1) // every - d) % max_length]``
  (floor division and floor modulo, :772-790), then indexes with ``idx``;
* ``retrieve_at_time`` (:798-907): ``fts = (t_now - t_delay) / slot_dt`` in float32;
  'linear' blends the floor / ceil steps as ``a * (1 - t) + b * t``; 'nearest' rounds half to
  even; the other registered methods (:163-338) are evaluated at the float ring index
  ``(write_ptr - 1) // every - fts`` from 2-4 neighbouring slots.

Pinned by the reference's own expectations (brainstate/nn/_delay_test.py:62-85, 126-182,
275-302, 444-522, 618-653, 676-705, 748-830) and the notebook's worked values
(docs/tutorials/brain_dynamics/02_synaptic_delays.ipynb cells 11, 17, 27), restated in
tests/test_oracle_delay.py.
"""
import math

import numpy as np

F = np.float32

ALIASES = {'linear_interp': 'linear', 'round': 'nearest'}
METHODS = ('nearest', 'round', 'linear', 'linear_interp', 'cubic', 'hermite', 'polynomial2',
           'polynomial3')


def delay_steps(time, dt):
    """ceil(time / dt) as the reference evaluates it (float32 ratio)."""
    if time is None:
        return 0
    if np.ndim(time) == 0 and not isinstance(time, np.ndarray):
        ratio = F(float(time) / float(dt))
    else:
        ratio = np.asarray(time, F) / F(dt)
    r = np.ceil(ratio).astype(np.int32)
    return int(r) if np.ndim(r) == 0 else r


def tap_weights(method, t):
    """(offsets relative to floor(idx), weights) of a registered interpolation method, with the
    weights computed in float32 as the reference's formulas (:193-338) spell them."""
    t = F(t)
    one, half = F(1.0), F(0.5)
    t2, t3 = t * t, t * t * t
    if method == 'cubic':      # Catmull-Rom, :210-214
        w = [-half * t3 + t2 - half * t, F(1.5) * t3 - F(2.5) * t2 + one,
             F(-1.5) * t3 + F(2.0) * t2 + half * t, half * t3 - half * t2]
        return (-1, 0, 1, 2), w
    if method == 'hermite':    # :246-249 with m0 = (v1 - v_m1)/2, m1 = (v2 - v0)/2 expanded
        h00 = F(2) * t3 - F(3) * t2 + one
        h10 = t3 - F(2) * t2 + t
        h01 = F(-2) * t3 + F(3) * t2
        h11 = t3 - t2
        return (-1, 0, 1, 2), [-half * h10, h00 - half * h11, h01 + half * h10, half * h11]
    if method == 'polynomial2':  # :287-290
        return (-1, 0, 1), [half * t * (t - one), (one - t) * (one + t), half * t * (t + one)]
    if method == 'polynomial3':  # :321-324
        return (-1, 0, 1, 2), [-t * (t - one) * (t - F(2)) / F(6),
                               (t + one) * (t - one) * (t - F(2)) / F(2),
                               -t * (t + one) * (t - F(2)) / F(2),
                               t * (t + one) * (t - one) / F(6)]
    if method == 'linear':       # :180-190
        return (0, 1), [one - t, t]
    raise ValueError(method)


class Delay:
    """Dense history ``[max_length, *shape]`` with the reference's write pointer."""

    def __init__(self, shape, dtype=F, time=None, init=None, dt=0.1, update_every=None,
                 interpolation='linear'):
        self.shape, self.dtype, self.dt = tuple(shape), dtype, float(dt)
        self.interpolation = ALIASES.get(interpolation, interpolation)
        self.update_every = update_every
        self.every = 1 if update_every is None else int(update_every / self.dt)
        self.slot_dt = self.dt if update_every is None else float(update_every)
        self.max_time = 0.0 if time is None else float(time)
        self.max_length = delay_steps(time, self.slot_dt) + 1
        self.init = init
        self.entries = {}
        self.history = None
        self.write_ptr = 0

    def register_entry(self, name, time, *idx):
        if name in self.entries:
            raise KeyError(name)
        if time is None:
            self.entries[name] = None
            return None
        steps = delay_steps(time, self.slot_dt)
        self.max_time = max(self.max_time, float(np.max(time)))
        if self.max_length <= int(np.max(steps)) + 1:
            self.max_length = int(np.max(steps)) + 1
        self.entries[name] = (steps,) + tuple(idx)
        return self.entries[name]

    def init_state(self, batch_size=None):
        shape = (self.max_length,) + ((batch_size,) if batch_size is not None else ()) + self.shape
        if self.init is None:
            self.history = np.zeros(shape, self.dtype)
        elif callable(self.init):
            self.history = np.asarray(self.init(shape, self.dtype), self.dtype)
        else:
            self.history = np.broadcast_to(np.asarray(self.init, self.dtype), shape).copy()
        self.write_ptr = 0

    def update(self, x):
        if self.write_ptr % self.every == 0:
            self.history[self.write_ptr // self.every] = x
        self.write_ptr = (self.write_ptr + 1) % (self.max_length * self.every)

    def current_slot(self):
        return (self.write_ptr - 1) // self.every

    def retrieve_at_step(self, d, *idx):
        slot = np.mod(self.current_slot() - np.asarray(d, np.int64), self.max_length)
        return self.history[(slot,) + tuple(idx)]

    def at(self, name):
        info = self.entries[name]
        return self.retrieve_at_step(*((0,) if info is None else info))

    def retrieve_at_time(self, t_delay, t_now, *idx):
        fts = (F(t_now) - F(t_delay)) / F(self.slot_dt)
        m = self.interpolation
        if m == 'linear':
            lo, hi = int(np.floor(fts)), int(np.ceil(fts))
            t = fts - np.floor(fts)
            a = self.retrieve_at_step(lo, *idx)
            b = self.retrieve_at_step(hi, *idx)
            return a * (F(1) - t) + b * t
        if m == 'nearest':
            return self.retrieve_at_step(int(np.round(fts)), *idx)
        fidx = F(self.current_slot()) - fts
        i0 = int(math.floor(float(fidx)))
        offs, w = tap_weights(m, fidx - F(i0))
        out = None
        for o, wq in zip(offs, w):
            v = wq * self.history[((i0 + o) % self.max_length,) + tuple(idx)]
            out = v if out is None else out + v
        return out
