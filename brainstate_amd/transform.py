"""Loop drivers and gradients mirroring brainstate.transform.for_loop / jit / grad.

The reference traces the step function once and runs it as an XLA While loop
(brainstate/transform/_loop_collect_return.py:487-572).  Here each step launches the HIP
kernels directly; ``for_loop`` recognises the E/I network step from the module calls of its
first two steps and runs the rest of the loop in the persistent runner (one launch).
"""
import numpy as np
import torch


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


def _ei_step(log, spk_before=None):
    """The E/I step the persistent runner runs, read off the module calls one step made:
    ``(neuron, proj_e, proj_i, n_exc, inp)`` when they were exactly the two projections onto
    one LIFRef / HH population, each given spikes of the population's shape (E: its first
    n_exc neurons, I: the rest) -- equal to ``spk_before``, its spikes before the step, when
    given -- then that population with one constant input (a scalar, or an array of the
    population's state shape, one input per neuron); else None."""
    from .nn._event import FixedPostNumConn
    from .nn._neurons import HH, AlignPostProj, LIFRef
    if len(log) != 3:
        return None
    (pa, aa, ka), (pb, ab, kb), (neuron, an, kn) = log
    if not isinstance(neuron, (LIFRef, HH)) or ka or kb or kn or len(an) > 1:
        return None
    if getattr(neuron, 'has_param_arrays', lambda: False)():   # the runner's are scalars
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
    shape = tuple(neuron.spike.value.shape)
    given = {id(pa): aa, id(pb): ab}
    for proj, lo, hi in ((proj_e, 0, n_exc), (proj_i, n_exc, n)):
        args = given[id(proj)]
        if len(args) != 1 or not torch.is_tensor(args[0]) or \
                tuple(args[0].shape) != shape[:-1] + (hi - lo,):
            return None
        if spk_before is not None and not torch.equal(args[0] != 0, spk_before[..., lo:hi] != 0):
            return None
    inp = an[0] if an else 0.0
    if isinstance(inp, np.ndarray):
        inp = torch.as_tensor(inp)
    if torch.is_tensor(inp):
        if inp.numel() != 1:
            if not torch.is_floating_point(inp) and inp.dtype not in (torch.int32, torch.int64):
                return None
            shape = tuple(neuron.V.value.shape)
            try:   # one input per neuron: must broadcast to the population's state shape
                if tuple(torch.broadcast_shapes(tuple(inp.shape), shape)) != shape:
                    return None
            except RuntimeError:
                return None
            return neuron, proj_e, proj_i, n_exc, inp.detach().to(torch.float32).clone()
        inp = inp.item()
    if not isinstance(inp, (int, float, np.floating, np.integer)):
        return None
    return neuron, proj_e, proj_i, n_exc, float(inp)


def _same_input(a, b):
    if torch.is_tensor(a) or torch.is_tensor(b):
        return (torch.is_tensor(a) and torch.is_tensor(b) and a.shape == b.shape and
                a.device == b.device and torch.equal(a, b))
    return a == b


def _fused_loop(f, xs, length):
    """for_loop through the persistent runner.  Steps 0 and 1 run eagerly while their module
    calls are recorded; when both are the same E/I step (``_ei_step``; step 1 checked against
    the population's spikes before it), with the same constant input and with the
    population's spikes (or nothing) as the step's output, the runner advances the other
    steps in one launch from the state the eager steps left -- pending spikes included -- and
    writes the final state back.  Returns (outputs of the eager steps, the stacked output of
    all steps or None when the loop must go on eagerly)."""
    from .nn import _event, _module
    from .nn._fuse import fuse
    outs, steps = [], []
    for i in range(2):
        before = steps[0][0].spike.value.clone() if steps else None
        _event.defer_layouts = True
        try:
            with _module.record_calls() as log:
                out = f(*[x[i] for x in xs])
        finally:
            _event.defer_layouts = False
        outs.append(out)
        step = _ei_step(log, before)
        if step is None:
            return outs, None
        spk = step[0].spike.value
        if out is not None and not (torch.is_tensor(out) and out.shape == spk.shape and
                                    torch.equal(out != 0, spk != 0)):
            return outs, None
        steps.append(step)
    if any(a is not b for a, b in zip(steps[0][:3], steps[1][:3])) or \
            steps[0][3] != steps[1][3] or not _same_input(steps[0][4], steps[1][4]):
        return outs, None
    neuron, proj_e, proj_i, n_exc, inp = steps[1]
    r = fuse(neuron, proj_e, proj_i, n_exc, inp)
    T = length - 2
    want = outs[0] is not None
    res = raster = None
    direct = False
    if want:
        # the stacked result: the eager steps' outputs, then the runner's raster (every neuron
        # of every step as 0/1) in their order and dtype.  A bool or uint8 result in the
        # runner's neuron order is the raster itself: the runner writes rows 2.. in place
        # (a separate raster and its conversion took 18 ms for 10,000 steps of 1M neurons)
        res = torch.empty((length,) + tuple(outs[0].shape), dtype=outs[0].dtype,
                          device=outs[0].device)
        perm = np.asarray(r.replica_index).reshape(-1)
        ident = getattr(r, 'replica_identity', False) or np.array_equal(perm,
                                                                         np.arange(perm.size))
        direct = ident and res.dtype in (torch.bool, torch.uint8) and res.device == r.device
        raster = (res[2:].view(torch.uint8).view(T, -1) if direct else
                  torch.empty(T, r.n, dtype=torch.uint8, device=r.device))
    r.run(T, raster=raster)
    r.check()
    r.write_back()
    if not want:
        return outs, [None] * length
    res[0].copy_(outs[0])
    res[1].copy_(outs[1])
    if not direct:
        if ident:
            res[2:].view(T, -1).copy_(raster)
        else:
            res[2:].view(T, -1).copy_(raster[:, torch.as_tensor(perm, device=raster.device)])
    return outs, res


def for_loop(f, *xs, length=None, reverse=False, unroll=1, pbar=None):
    """Call ``f(*x_t)`` for t along the leading axis of ``xs`` and stack the outputs
    (brainstate/transform/_loop_collect_return.py:487-572).

    The reference traces ``f`` once and runs the whole loop as one compiled scan.  Here a
    step function that is the E/I network step (the two event projections of one LIFRef or
    HH population fed its spikes, then the population with a constant input -- the update
    of examples/105_COBA_HH_2007_braincell.py and of the SNN tutorial) is recognised from the
    module calls of its first two steps, which run eagerly, and every later step runs in
    the persistent runner, one launch; the state is written back at the end.  Any other step
    function runs eagerly step by step."""
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
            done, stacked = _fused_loop(f, xs, length)
            if bar is not None:
                bar.advance(len(done) if stacked is None else length, length - 1)
            if stacked is not None:
                last_loop = 'fused'
                return stacked if torch.is_tensor(stacked) else _stack(stacked)
            outs = done
            for i in range(len(done), length):
                outs.append(f(*[x[i] for x in xs]))
                if bar is not None:
                    bar.step(i)
            return _stack(outs)
        order = range(length - 1, -1, -1) if reverse else range(length)
        outs = []
        for i in order:
            outs.append(f(*[x[i] for x in xs]))
            if bar is not None:
                bar.step(i)
        if reverse:
            outs = outs[::-1]
        return _stack(outs)
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
