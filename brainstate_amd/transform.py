"""Loop drivers and gradients mirroring brainstate.transform.for_loop / jit / grad.

The reference traces the step function once and runs it as an XLA While loop
(brainstate/transform/_loop_collect_return.py:487-572).  Here each step launches the HIP
kernels directly; ``for_loop`` records the step function without running it
(brainstate_amd/_trace.py) and, when every step is the E/I network step, runs the loop in the
persistent runner.
"""
import numpy as np
import torch

from . import _trace


def _stack(outs):
    if not outs:
        return outs
    first = outs[0]
    if torch.is_tensor(first):
        return torch.stack(outs)
    if isinstance(first, (tuple, list)):
        return type(first)(_stack([o[i] for o in outs]) for i in range(len(first)))
    if isinstance(first, dict):
        return {k: _stack([o[k] for o in outs]) for k in first}
    if first is None:
        return None
    return outs


def _prealloc(o, length):
    """Stacked buffers [length, ...] for step outputs shaped like ``o`` (tensors that take no
    part in autodiff, in tuples, lists and dicts, None allowed), or None for anything else."""
    if torch.is_tensor(o):
        if o.requires_grad:
            return None
        return torch.empty((length,) + tuple(o.shape), dtype=o.dtype, device=o.device)
    if o is None:
        return _NONE
    if isinstance(o, (tuple, list)):
        parts = [_prealloc(x, length) for x in o]
        return None if any(b is None for b in parts) else type(o)(parts)
    if isinstance(o, dict):
        parts = {k: _prealloc(v, length) for k, v in o.items()}
        return None if any(b is None for b in parts.values()) else parts
    return None


_NONE = object()   # a None output leaf inside the preallocated structure


def _put(buf, i, o):
    """Copy step i's outputs into row i of the buffers; False (nothing guaranteed written)
    when ``o`` differs from the first step's outputs in structure, shape, dtype or device."""
    if buf is _NONE:
        return o is None
    if torch.is_tensor(buf):
        if not (torch.is_tensor(o) and o.shape == buf.shape[1:] and o.dtype == buf.dtype
                and o.device == buf.device and not o.requires_grad):
            return False
        buf[i].copy_(o)
        return True
    if isinstance(buf, (tuple, list)):
        return (isinstance(o, (tuple, list)) and len(o) == len(buf)
                and all(_put(b, i, x) for b, x in zip(buf, o)))
    return (isinstance(o, dict) and o.keys() == buf.keys()
            and all(_put(buf[k], i, o[k]) for k in buf))


def _take(buf, i):
    """Step i's outputs as views into the buffers."""
    if buf is _NONE:
        return None
    if torch.is_tensor(buf):
        return buf[i]
    if isinstance(buf, (tuple, list)):
        return type(buf)(_take(b, i) for b in buf)
    return {k: _take(b, i) for k, b in buf.items()}


def _finish(buf):
    """The preallocated buffers as for_loop's result (None leaves back to None)."""
    if buf is _NONE:
        return None
    if torch.is_tensor(buf):
        return buf
    if isinstance(buf, (tuple, list)):
        return type(buf)(_finish(b) for b in buf)
    return {k: _finish(b) for k, b in buf.items()}


fuse_loops = True   # False: for_loop always steps eagerly
last_loop = None    # how the last for_loop ran: 'fused' (persistent runner) or 'eager'


class ProgressBar:
    """Progress of a ``for_loop`` (brainstate/transform/_progress_bar.py:265-453): the same
    arguments and checks.  ``freq`` steps per update (default: every 5 % of the steps, or
    every step up to 20), or ``count`` updates in all; ``desc`` a string or a
    ``(format_string, fn)`` pair, ``fn`` mapping ``{'i': step}`` to the format's fields.
    Drawn with tqdm when it is importable, else as a line on stderr per update.  A loop
    that runs in the persistent runner advances the bar once for the steps of its launch."""

    def __init__(self, freq=None, count=None, desc=None, **kwargs):
        if isinstance(freq, int) and freq <= 0:
            raise ValueError(f'Print rate (freq) should be > 0, but got {freq}.')
        if freq is not None and count is not None:
            raise ValueError('Cannot specify both count and freq.')
        if desc is not None and not isinstance(desc, str):
            if not isinstance(desc, (tuple, list)):
                raise TypeError(f'desc must be a string or a (format_string, callable) '
                                f'tuple/list, but got {type(desc).__name__}.')
            if len(desc) != 2:
                raise ValueError(f'desc tuple/list must have exactly two elements '
                                 f'(format_string, callable), but got {len(desc)}.')
            if not isinstance(desc[0], str):
                raise TypeError(f'The first element of a desc tuple must be a format '
                                f'string, but got {type(desc[0]).__name__}.')
            if not callable(desc[1]):
                raise TypeError(f'The second element of a desc tuple must be callable, '
                                f'but got {type(desc[1]).__name__}.')
        self.print_freq = freq
        self.print_count = count
        self.desc = desc
        self.kwargs = {k: v for k, v in kwargs.items()
                       if k not in ('total', 'mininterval', 'maxinterval', 'miniters')}

    def init(self, n):
        """The bar of an n-step loop: steps per update as the reference resolves them."""
        freq, count = self.print_freq, self.print_count
        if count is not None:
            freq = n // count
            if freq == 0:
                raise ValueError(f'Count {count} is too large for n {n}.')
        elif freq is None:
            freq = int(n / 20) if n > 20 else 1
        elif freq > n:
            raise ValueError(f'Print rate should be less than the number of steps {n}, '
                             f'got {freq}')
        return _Bar(n, freq, self.desc, self.kwargs)


class _Bar:
    """One loop's bar: ``step(i)`` after step i, ``advance(k, i)`` after k steps ending at i,
    ``close()`` at the end (which also draws the steps past the last whole ``freq``)."""

    def __init__(self, n, freq, desc, kwargs):
        self.n, self.freq, self.desc, self.done, self.shown = n, freq, desc, 0, 0
        try:
            from tqdm.auto import tqdm
            self.bar = tqdm(total=n, **kwargs)
        except ImportError:
            self.bar = None
        self._describe(0)

    def _describe(self, i):
        if self.desc is None:
            msg = f'Running for {self.n:,} iterations'
        elif isinstance(self.desc, str):
            msg = self.desc
        else:
            msg = self.desc[0].format(**self.desc[1]({'i': i}))
        if self.bar is not None:
            self.bar.set_description(msg, refresh=False)
        self.msg = msg

    def _show(self, i):
        k = self.done - self.shown
        if k <= 0:
            return
        self._describe(i)
        if self.bar is not None:
            self.bar.update(k)
        else:
            import sys
            print(f'{self.msg}: {self.done}/{self.n}', file=sys.stderr)
        self.shown = self.done

    def step(self, i):
        self.advance(1, i)

    def advance(self, k, i):
        self.done += k
        if self.done - self.shown >= self.freq:
            self._show(i)

    def close(self):
        self._show(self.n - 1)
        if self.bar is not None:
            self.bar.close()


def _ei_structure(tr, calls, out):
    """The E/I step the persistent runner runs, read off one recorded step (``_trace``):
    ``(neuron, proj_e, proj_i, n_exc, inp, raster_dtype)`` when the step made exactly the two
    projection calls onto one LIFRef / HH population, each given a spike vector of that
    population (E: its first n_exc neurons, I: the rest; the population's spike State read
    outside the modules, sliced, compared with 0 or converted), then called the population
    with one input, and returned the population's spikes (the call's result or its spike
    State, as a spike vector) or nothing; else None.  ``inp`` is a number, a tensor or array
    of the population's state shape (one input per neuron), or a ``StepArg`` (the loop's
    per-step argument itself); ``raster_dtype`` the dtype of the stacked output (None: no
    output)."""
    from .nn._event import FixedPostNumConn
    from .nn._neurons import HH, AlignPostProj, LIFRef
    if len(calls) != 3:
        return None
    (pa, aa, ka), (pb, ab, kb), (neuron, an, kn) = calls
    if not isinstance(neuron, (LIFRef, HH)) or ka or kb or kn or len(an) > 1:
        return None
    if getattr(neuron, 'has_param_arrays', lambda: False)():   # the runner's are scalars
        return None
    if neuron.before_updates or neuron.after_updates:   # e.g. a delay recording the neuron
        return None
    chans = getattr(neuron, '_channels', [])
    if len(chans) != 2 or {id(pa), id(pb)} != {id(c) for c in chans}:
        return None
    proj_e, proj_i = chans
    if not (isinstance(proj_e, AlignPostProj) and isinstance(proj_i, AlignPostProj)):
        return None
    conns = [getattr(p.comm, 'conn', None) for p in chans]
    if not all(isinstance(c, FixedPostNumConn) for c in conns):
        return None
    n, n_exc = neuron.num, conns[0].shape[0]
    if conns[0].shape != (n_exc, n) or conns[1].shape != (n - n_exc, n):
        return None
    spike = neuron.spike
    shape = tuple(spike._value.shape)
    given = {id(pa): aa, id(pb): ab}
    for proj, lo, hi in ((proj_e, 0, n_exc), (proj_i, n_exc, n)):
        args = given[id(proj)]
        if len(args) != 1 or not torch.is_tensor(args[0]):
            return None
        m = tr.marks.get(id(args[0]))
        if m is None or m.state is not spike or (m.lo, m.hi) != (lo, hi) or \
                tuple(args[0].shape) != shape[:-1] + (hi - lo,):
            return None
    # the step's output: the population's call or its full spike vector, or nothing
    if out is None:
        raster_dtype = None
    elif isinstance(out, _trace.DryOut):
        if out.index != 2:
            return None
        raster_dtype = spike._value.dtype   # the neuron returns its spike State's value
    elif torch.is_tensor(out) and id(out) in tr.marks:
        m = tr.marks[id(out)]
        if m.state is not spike or (m.lo, m.hi) != (0, n) or tuple(out.shape) != shape:
            return None
        raster_dtype = out.dtype
    else:
        return None
    inp = an[0] if an else 0.0
    if isinstance(inp, _trace.StepArg):
        return neuron, proj_e, proj_i, n_exc, inp, raster_dtype
    inp = _input_value(inp, neuron)
    if inp is None:
        return None
    return neuron, proj_e, proj_i, n_exc, inp, raster_dtype


def _input_value(inp, neuron):
    """A neuron input as the runner takes it: a float, or an fp32 device tensor of the
    population's state shape; None when it is neither (or depends on marked state)."""
    if isinstance(inp, np.ndarray):
        inp = torch.as_tensor(inp)
    if torch.is_tensor(inp):
        tr = _trace.active()
        if tr is not None and id(inp) in tr.marks:
            return None
        if inp.numel() == 1:
            return float(inp.reshape(()).item())
        if not torch.is_floating_point(inp) and inp.dtype not in (torch.int32, torch.int64):
            return None
        shape = tuple(neuron.V._value.shape)
        try:   # one input per neuron: must broadcast to the population's state shape
            if tuple(torch.broadcast_shapes(tuple(inp.shape), shape)) != shape:
                return None
        except RuntimeError:
            return None
        return inp
    if isinstance(inp, (bool, np.bool_)) or not isinstance(inp, (int, float, np.floating,
                                                                  np.integer)):
        return None
    return float(inp)


def _same_input(a, b):
    if torch.is_tensor(a) or torch.is_tensor(b):
        if not (torch.is_tensor(a) and torch.is_tensor(b)):
            return False
        if a is b:
            return True
        return a.shape == b.shape and a.device == b.device and bool(torch.equal(a, b))
    return a == b


_MAX_INPUT_BYTES = 1 << 30   # per-step input arrays a recorded loop may hold


def _schedule(xs, j, length, neuron):
    """Per-step inputs when the step passes its j-th argument straight to the population:
    [(first step, steps, input)] with equal consecutive inputs merged; None when an input is
    not one the runner takes."""
    x = xs[j]
    if torch.is_tensor(x) or isinstance(x, np.ndarray):
        t = torch.as_tensor(x)
        if t.shape[0] < length:
            return None
        t = t[:length]
        if t.dim() == 1 or int(np.prod(tuple(t.shape[1:]))) == 1:   # one number per step
            if not (torch.is_floating_point(t) or t.dtype in (torch.int32, torch.int64)):
                return None
            v = t.reshape(length).detach().cpu().to(torch.float64).numpy()
            cut = np.flatnonzero(v[1:] != v[:-1]) + 1
            starts = np.concatenate([[0], cut]).astype(np.int64)
            ends = np.concatenate([cut, [length]]).astype(np.int64)
            return [(int(a), int(b - a), float(v[a])) for a, b in zip(starts, ends)]
        vals = [_input_value(t[i], neuron) for i in range(length)]
    else:
        vals = [_input_value(x[i], neuron) for i in range(length)]
    return _merge(vals)


def _merge(vals):
    segs = []
    for i, v in enumerate(vals):
        if v is None:
            return None
        if segs and _same_input(segs[-1][2], v):
            segs[-1][1] += 1
        else:
            segs.append([i, 1, v])
    return [tuple(s) for s in segs]


def _record(f, xs, length):
    """The recording passes of ``for_loop(f, *xs)`` (brainstate_amd/_trace.py): returns
    ``(neuron, proj_e, proj_i, n_exc, segments, raster_dtype)`` when every step is the E/I
    step the runner implements -- segments [(first step, steps, input)] of equal inputs --
    else None.  No network kernel runs; random states are restored unless the per-step
    recording drew numbers that the runner then uses (those of the eager steps)."""
    tr = _trace.Trace()
    with _trace.rng_guard() as rng:
        try:
            calls, out = tr.run(f, _trace.step_args(len(xs)))
            st = _ei_structure(tr, calls, out)
            if st is None:
                return None
            if rng.changed():   # draws inside the step: record each step's own
                rng.restore()
                raise _trace.Dependent()
            neuron, pe, pi, n_exc, inp, rd = st
            if isinstance(inp, _trace.StepArg):
                segs = _schedule(xs, inp.index, length, neuron)
            else:
                segs = [(0, length, inp)]
            return None if segs is None else (neuron, pe, pi, n_exc, segs, rd)
        except _trace.NotFusable:
            return None
        except _trace.Dependent:
            pass
        except Exception:   # the step cannot be recorded; eager stepping shows why
            return None
        # the step uses its arguments: record every step with its own
        first, vals, held = None, [], 0
        try:
            for i in range(length):
                calls, out = tr.run(f, [x[i] for x in xs])
                st = _ei_structure(tr, calls, out)
                if st is None or isinstance(st[4], _trace.StepArg):
                    rng.restore()
                    return None
                if first is None:
                    first = st
                elif any(a is not b for a, b in zip(first[:4], st[:4])) or first[5] != st[5]:
                    rng.restore()
                    return None
                v = st[4]
                if torch.is_tensor(v) and not (vals and vals[-1] is v):
                    held += v.numel() * v.element_size()
                    if held > _MAX_INPUT_BYTES:
                        rng.restore()
                        return None
                vals.append(v)
        except (_trace.NotFusable, _trace.Dependent):
            rng.restore()
            return None
        except Exception:
            rng.restore()
            return None
        segs = _merge(vals)
        if segs is None:
            rng.restore()
            return None
        neuron, pe, pi, n_exc, _, rd = first
        return neuron, pe, pi, n_exc, segs, rd


def _fuse_key(neuron, pe, pi, n_exc, inp):
    """What a runner built by ``fuse`` depends on besides the state it reloads: the modules,
    the connectivity and weight objects (tensors with their version counters; a numpy array
    changed in place is not seen), the population's shape and model, and the input kind."""
    from .nn._fuse import _scalar_input
    parts = [neuron, pe, pi, int(n_exc), type(neuron), tuple(neuron.V.value.shape),
             _scalar_input(inp) is None]
    for proj in (pe, pi):
        conn = getattr(proj.comm, 'conn', None)
        idx = getattr(conn, 'indices', None)
        w = proj.comm.weight.value
        parts += [idx, getattr(idx, '_version', None), w,
                  w._version if torch.is_tensor(w) else None,
                  None if torch.is_tensor(w) or np.ndim(w) else float(w)]
    return parts


def _same_key(a, b):
    if a is None or b is None or len(a) != len(b):
        return False
    for x, y in zip(a, b):
        if isinstance(x, (int, float, bool, tuple, type(None))) and not torch.is_tensor(x):
            if x != y:
                return False
        elif x is not y:
            return False
    return True


def _scalar_of(v):
    """A recorded input as one float (a number, or a one-element array or tensor), or None."""
    if torch.is_tensor(v) or isinstance(v, np.ndarray):
        return float(v.reshape(-1)[0]) if int(np.prod(tuple(v.shape))) == 1 else None
    try:
        return float(v)
    except (TypeError, ValueError):
        return None


def _runner_for(neuron, pe, pi, n_exc, inp):
    """The persistent runner of this net: the one the last loop on it built, reloaded with
    the modules' current state, while connectivity, weights and input kind are unchanged
    (its set-up -- layout, in-degrees, inbox capacities, workspace -- takes ~15-30 ms at 1M
    neurons, more than 2,000 of its steps), else a new one (kept for the next loop)."""
    from .nn._fuse import fuse
    key = _fuse_key(neuron, pe, pi, n_exc, inp)
    cached = getattr(neuron, '_fused_runner', None)
    if cached is not None and _same_key(cached[0], key):
        try:
            cached[1].reload(inp)
            return cached[1]
        except (NotImplementedError, ValueError):
            pass
    if cached is not None:   # its workspace goes before the new one is allocated (the
        cached[1].ws = None  # runner and its closures form a cycle that waits for the gc)
    neuron._fused_runner = None
    r = fuse(neuron, pe, pi, n_exc, inp)
    neuron._fused_runner = (key, r)
    return r


def _fused_loop(f, xs, length):
    """for_loop through the persistent runner: the steps are recorded first (``_record``);
    when every one is the E/I step the runner implements, the runner advances all of them
    from the modules' state -- one launch with the per-step inputs when they are numbers,
    else one per run of equal inputs -- and writes the final
    state back.  Returns the stacked output (a tensor, or a list of None), or None when the
    loop must run eagerly."""
    plan = _record(f, xs, length)
    if plan is None:
        return None
    neuron, proj_e, proj_i, n_exc, segs, rdtype = plan
    first = next((v for _, _, v in segs if torch.is_tensor(v)), segs[0][2])
    try:
        r = _runner_for(neuron, proj_e, proj_i, n_exc, first)
    except NotImplementedError:   # a state the runner cannot start from
        return None
    T = length
    res = raster = None
    direct = False
    if rdtype is not None:
        # the stacked result [T, *spike shape] in the output's dtype; a bool or uint8 result
        # in the runner's neuron order is the raster itself (the runner writes it in place)
        shape = tuple(neuron.spike.value.shape)
        res = torch.empty((T,) + shape, dtype=rdtype, device=r.device)
        perm = np.asarray(r.replica_index).reshape(-1)
        ident = getattr(r, 'replica_identity', False) or np.array_equal(perm,
                                                                         np.arange(perm.size))
        direct = ident and rdtype in (torch.bool, torch.uint8)
        raster = (res.view(torch.uint8).view(T, -1) if direct else
                  torch.empty(T, r.n, dtype=torch.uint8, device=r.device))
    scalars = [_scalar_of(v) for _, _, v in segs]
    if len(segs) > 1 and r.I_ext is None and all(x is not None for x in scalars):
        # inputs that change between steps: every step's value in one array, one launch
        per_step = np.empty(T, np.float32)
        for (t0, steps, _), x in zip(segs, scalars):
            per_step[t0:t0 + steps] = x
        r.run(T, raster=raster, inputs=torch.from_numpy(per_step).to(r.device))
    else:
        for t0, steps, v in segs:
            r.set_input(v)
            r.run(steps, raster=None if raster is None else raster[t0:t0 + steps])
    r.check()
    r.write_back()
    if rdtype is None:
        return [None] * length
    if not direct:
        src = raster if ident else raster[:, torch.as_tensor(perm, device=raster.device)]
        res.view(T, -1).copy_(src)
    return res


def for_loop(f, *xs, length=None, reverse=False, unroll=1, pbar=None):
    """Call ``f(*x_t)`` for t along the leading axis of ``xs`` and stack the outputs
    (brainstate/transform/_loop_collect_return.py:487-572).

    The reference traces ``f`` once and runs the whole loop as one compiled scan
    (:254,268).  Here ``f`` is first recorded without running its modules
    (brainstate_amd/_trace.py): once with placeholders for the per-step arguments, and, when
    the step uses them, once per step with the concrete values.  When every step is the E/I
    network step the persistent runner implements (the two event projections of one LIFRef
    or HH population fed its spikes, then the population called with one input -- the
    update of examples/105_COBA_HH_2007_braincell.py and of the SNN tutorial), the runner
    advances all steps (one launch, with the per-step inputs when they are numbers; one per
    run of equal per-neuron input arrays), and the state is written back at
    the end.  Anything else -- other modules, State assignments outside modules, state used
    for anything but the projections' spike vectors, inputs the runner does not take --
    runs eagerly step by step.  Python side effects of ``f`` happen in the recording pass
    (once, or once per step) and again per step when the loop then runs eagerly.  The runner
    stays on the population for the next loop on the same connectivity, weights and input
    kind, which reloads it from the modules' state instead of building a new one (its
    workspace, ~1.6 GB at 1e8 synapses, stays allocated until then)."""
    global last_loop
    if length is None:
        if not xs:
            raise ValueError('for_loop needs xs or length')
        length = len(xs[0])
    if isinstance(pbar, int) and not isinstance(pbar, bool):
        pbar = ProgressBar(freq=pbar)   # an int is the update frequency, as in the reference
    bar = pbar.init(length) if pbar is not None else None
    last_loop = 'eager'
    try:
        if fuse_loops and not reverse and length >= 3:
            stacked = _fused_loop(f, xs, length)
            if stacked is not None:
                if bar is not None:
                    bar.advance(length, length - 1)
                last_loop = 'fused'
                return stacked if torch.is_tensor(stacked) else _stack(stacked)
        # Each step's outputs are copied into buffers allocated for all steps after the first
        # (a snapshot, so an output that is a state tensor the next step updates in place
        # keeps this step's value; no list of per-step tensors for the allocator to grow
        # under, and no second copy to stack them); outputs of other kinds are kept as they
        # come and stacked at the end.
        order = range(length - 1, -1, -1) if reverse else range(length)
        buf, outs = None, [None] * length
        for n_done, i in enumerate(order):
            o = f(*[x[i] for x in xs])
            if n_done == 0:
                buf = _prealloc(o, length)
            if buf is not None and not _put(buf, i, o):
                # outputs unlike the first step's: the steps so far as views, then a list
                for j in order[:n_done]:
                    outs[j] = _take(buf, j)
                buf = None
            if buf is None:
                outs[i] = o
            if bar is not None:
                bar.step(i)
        return _finish(buf) if buf is not None else _stack(outs)
    finally:
        if bar is not None:
            bar.close()


def jit(fn=None, **kwargs):
    """Kernels are compiled ahead of time; ``jit`` returns the function unchanged."""
    if fn is None:
        return lambda f: f
    return fn


def _as_leaf(v):
    t = torch.as_tensor(v)
    if not torch.is_floating_point(t):
        raise TypeError(f'grad requires real floating-point inputs, got {t.dtype}')
    return t.detach().requires_grad_(True)


def grad(fun=None, grad_states=None, argnums=None, has_aux=False, return_value=False, **kwargs):
    """Gradient of a scalar-valued ``fun`` (brainstate/transform/_grad_grad.py:49-140), on
    torch autograd.  Return conventions follow the reference:

    * ``grad_states`` None: ``arg_grads`` (argnums defaults to 0);
    * ``grad_states`` given, ``argnums`` None: ``var_grads`` (same structure as grad_states);
    * both given: ``(var_grads, arg_grads)``;
    each followed by ``loss_value`` if ``return_value`` and ``aux`` if ``has_aux``.
    ``arg_grads`` is one tensor for an int ``argnums`` and a tuple for a sequence.
    Integer or bool arguments raise TypeError, as in JAX.
    """
    if fun is None:
        return lambda f: grad(f, grad_states, argnums, has_aux, return_value, **kwargs)
    if grad_states is None and argnums is None:
        argnums = 0
    nums = None if argnums is None else ((argnums,) if isinstance(argnums, int) else tuple(argnums))
    if isinstance(grad_states, dict):
        skeys, slist = list(grad_states.keys()), list(grad_states.values())
    elif grad_states is None:
        skeys, slist = None, []
    elif isinstance(grad_states, (list, tuple)):
        skeys, slist = None, list(grad_states)
    else:
        skeys, slist = None, [grad_states]

    def g(*args):
        args = list(args)
        for i in nums or ():
            args[i] = _as_leaf(args[i])
        old = [st.value for st in slist]
        leaves = []
        for st in slist:
            leaf = _as_leaf(st.value)
            st.restore_value(leaf)
            leaves.append(leaf)
        try:
            out = fun(*args)
        finally:
            for st, v in zip(slist, old):
                st.restore_value(v)
        value, aux = (out[0], out[1]) if has_aux else (out, None)
        targets = [args[i] for i in nums or ()] + leaves
        gr = torch.autograd.grad(value, targets, allow_unused=True)
        gr = [torch.zeros_like(t) if x is None else x for x, t in zip(gr, targets)]
        arg_g = gr[:len(nums or ())]
        var_g = gr[len(nums or ()):]
        if nums is not None:
            arg_g = arg_g[0] if isinstance(argnums, int) else tuple(arg_g)
        if grad_states is not None:
            if skeys is not None:
                var_g = dict(zip(skeys, var_g))
            elif not isinstance(grad_states, (list, tuple)):
                var_g = var_g[0]
            else:
                var_g = type(grad_states)(var_g)
        if grad_states is None:
            res = arg_g
        elif nums is None:
            res = var_g
        else:
            res = (var_g, arg_g)
        extra = ((value.detach(),) if return_value else ()) + ((aux,) if has_aux else ())
        return (res,) + extra if extra else res

    return g
