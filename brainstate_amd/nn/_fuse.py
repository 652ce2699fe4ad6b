"""Hand a module-built E/I network to the persistent whole-loop runner.

``fuse(neuron, proj_e, proj_i, n_exc, inp)`` takes the pieces of the reference's E/I net
(examples/105_COBA_HH_2007_braincell.py:54-82: ``N``, ``E`` fed by ``spk[:n_exc]``, ``I`` fed
by ``spk[n_exc:]``) and returns an ``EINetRunner`` that advances the same network many steps
per launch, with the constant external input ``inp`` the script passes as ``N(inp)`` (a
scalar, or an array broadcast to the population's state shape: one input per neuron).
Spikes of the last step that the neurons hold (a loop stepped eagerly so far) become the
runner's first inputs (synaptic delay 0).  ``delay`` (ms) is the synaptic delay of a net whose
projections read
``N.prefetch_delay('spike', delay)()`` instead of the previous step's spikes; it becomes
ceil(delay / dt) steps as brainstate's Delay computes them.  A net initialised with
``init_all_states(..., batch_size=B)`` ([B, n] states, the replicas sharing connectivity)
becomes one runner over the block-diagonal union of the B replicas.  ``runner.write_back()``
copies the state back into the modules; ``runner.set_input(x)`` changes the external input
of the next run (``for_loop`` with an input that changes between runs of steps).
"""
import numpy as np
import torch

from .. import environ
from ..runner import EINetRunner
from ._delay import _get_delay, _leaves
from ._event import FixedPostNumConn
from ._neurons import HH, LIFRef


def _proj_arrays(proj, n_pre, n):
    conn = getattr(proj.comm, 'conn', None)
    if not isinstance(conn, FixedPostNumConn):
        raise NotImplementedError('fuse() needs fixed-num (EventFixedProb) projections')
    if conn.shape != (n_pre, n):
        raise ValueError(f'projection shape {conn.shape} does not match ({n_pre}, {n})')
    # device tensors stay on the device (no round trip through the host for one replica)
    idx = conn.indices
    w = proj.comm.weight.value
    if torch.is_tensor(w):
        w = w.detach()
        return idx, (float(w.reshape(())) if w.numel() == 1 else
                     w.to(torch.float32).expand(idx.shape))
    w = np.asarray(w, np.float32)
    return idx, (float(w.reshape(())) if w.size == 1 else
                 torch.as_tensor(np.broadcast_to(w, idx.shape).copy(), device=idx.device))


def _union_perm(B, n, n_exc):
    """Runner index of neuron j of replica b ([B, n]): the runner takes excitatory neurons
    first, so the union of B replicas lists every replica's E neurons, then every I neuron."""
    j = np.arange(n, dtype=np.int64)[None, :]
    b = np.arange(B, dtype=np.int64)[:, None]
    return np.where(j < n_exc, b * n_exc + j, B * n_exc + b * (n - n_exc) + (j - n_exc))


def _check_start(neuron, proj_e, proj_i, delay):
    """Raise unless the runner can start from the modules' current state; returns whether
    the neurons hold spikes of their last step (pending inputs of the first step)."""
    if len(neuron._channels) != 2 or neuron._channels[0] is not proj_e or \
            neuron._channels[1] is not proj_i:
        raise ValueError('proj_e and proj_i must be the two projections onto neuron, in order')
    if proj_e.syn.delta is not None or proj_i.syn.delta is not None:
        raise NotImplementedError('fuse() starts between steps (a synapse holds an input of a '
                                  'step in progress)')
    pending = bool(neuron.spike.value.any())
    if pending and delay is not None:
        raise NotImplementedError('fuse() with a synaptic delay starts from a state without '
                                  'pending spikes')
    for hook in neuron.after_updates.values():   # spike histories of prefetch_delay readers
        hist = getattr(hook, 'history', None)
        if hist is not None and any(bool(h.any()) for h in _leaves(hist.value)):
            raise NotImplementedError('fuse() starts from a state without pending spikes '
                                      '(a delay history holds spikes)')
    if getattr(neuron, 'has_param_arrays', lambda: False)():
        raise NotImplementedError('fuse(): the runner takes scalar neuron parameters; a '
                                  'population with per-neuron parameters steps eagerly')
    return pending


def _scalar_input(inp):
    """The input as one number, or None when it is an array of more than one value."""
    if (torch.is_tensor(inp) or isinstance(inp, np.ndarray)) and np.prod(tuple(inp.shape)) != 1:
        return None
    return float(inp.reshape(()).item() if torch.is_tensor(inp) else np.reshape(inp, ()))


def fuse(neuron, proj_e, proj_i, n_exc, inp=0.0, delay=None):
    pending = _check_start(neuron, proj_e, proj_i, delay)
    n = neuron.num
    Vs = neuron.V.value
    B = int(Vs.shape[0]) if Vs.dim() == 2 else 1   # init_all_states(batch_size=B)
    idx_e, w_e = _proj_arrays(proj_e, n_exc, n)
    idx_i, w_i = _proj_arrays(proj_i, n - n_exc, n)
    dev = idx_e.device
    if isinstance(w_e, float) != isinstance(w_i, float):   # one heterogeneous -> both per synapse
        w_e = torch.full(idx_e.shape, w_e, device=dev) if isinstance(w_e, float) else w_e
        w_i = torch.full(idx_i.shape, w_i, device=dev) if isinstance(w_i, float) else w_i
    # one replica: the runner's order is the net's (no permutation to build or apply)
    perm = _union_perm(B, n, n_exc) if B > 1 else np.arange(n, dtype=np.int64)[None, :]
    if B > 1:   # block-diagonal union of the replicas, one runner
        pm = torch.as_tensor(perm, device=dev)
        idx_e = torch.cat([pm[b][idx_e.long()] for b in range(B)]).to(torch.int32)
        idx_i = torch.cat([pm[b][idx_i.long()] for b in range(B)]).to(torch.int32)
        if not isinstance(w_e, float):
            w_e, w_i = w_e.repeat(B, 1), w_i.repeat(B, 1)
    pt = torch.as_tensor(perm.reshape(-1), device=Vs.device) if B > 1 else None

    def to_runner(x):
        if pt is None:
            return x.reshape(-1).clone()
        out = torch.empty(B * n, dtype=x.dtype, device=x.device)
        out[pt] = x.reshape(-1)
        return out

    def from_runner(x):
        return (x if pt is None else x[pt]).reshape(Vs.shape).clone()

    V0 = to_runner(Vs)
    if isinstance(neuron, HH):
        model = 'hh'
    elif isinstance(neuron, LIFRef):
        model = 'lif'
    else:
        raise NotImplementedError(type(neuron).__name__)
    delay_steps = _get_delay(delay, environ.get_dt())[1]
    I0 = _scalar_input(inp)
    if I0 is None:
        I0, I_arr = 0.0, to_runner(torch.broadcast_to(
            torch.as_tensor(inp, dtype=torch.float32, device=Vs.device), Vs.shape))
    else:
        I_arr = None
    r = EINetRunner(model, B * n, B * n_exc, idx_e, idx_i, w_e, w_i, neuron.params(I0),
                    V0, delay_steps=delay_steps, I_ext=I_arr)
    def load_state():
        # carry the current state over (the runner initialised HH gates at steady state)
        r.state['ge'].copy_(to_runner(proj_e.syn.g.value))
        r.state['gi'].copy_(to_runner(proj_i.syn.g.value))
        if model == 'lif':
            r.state['ref'].copy_(to_runner(neuron.ref.value))
        else:
            r.state['m'].copy_(to_runner(neuron.m.value))
            r.state['h'].copy_(to_runner(neuron.h.value))
            r.state['n'].copy_(to_runner(neuron.n.value))

    load_state()

    def write_back():
        neuron.V.value = from_runner(r.state['V'])
        proj_e.syn.g.value = from_runner(r.state['ge'])
        proj_i.syn.g.value = from_runner(r.state['gi'])
        neuron.spike.value = from_runner(r.spk).view(torch.bool)
        if model == 'lif':
            neuron.ref.value = from_runner(r.state['ref'])
        else:
            neuron.m.value = from_runner(r.state['m'])
            neuron.h.value = from_runner(r.state['h'])
            neuron.n.value = from_runner(r.state['n'])

    def set_input(v):
        """The external input of the next run: a number, or (a runner built with one input
        per neuron) an array broadcast to the population's state shape."""
        if I_arr is None:
            if (torch.is_tensor(v) or isinstance(v, np.ndarray)) and np.prod(tuple(v.shape)) != 1:
                raise ValueError('set_input: this runner takes one number per run (it was '
                                 'built with a scalar input)')
            r.params.I_ext = float(v.reshape(()).item() if torch.is_tensor(v) else
                                   np.reshape(v, ()))
        else:
            r.I_ext.copy_(to_runner(torch.broadcast_to(
                torch.as_tensor(v, dtype=torch.float32, device=Vs.device), Vs.shape)))

    if pending:   # the spikes of the last step drive the runner's first step
        r.seed(to_runner(neuron.spike.value.to(torch.uint8)), 1)

    def reload(v):
        """Start the next run from the modules' current state (a runner kept across
        loops on the same connectivity and weights): neuron parameters, input, state, and
        the current spikes as the inputs of the first step -- published as the events of
        the step after the last one this runner ran, so no count word of an earlier run can
        be taken for one of this run.  Synaptic delay 0 only."""
        if delay_steps:
            raise NotImplementedError('reload(): a runner with a synaptic delay is rebuilt')
        _check_start(neuron, proj_e, proj_i, None)
        if (_scalar_input(v) is None) != (I_arr is not None):
            raise ValueError('reload(): the input kind (one number or one per neuron) changed')
        r.params = neuron.params(0.0 if I_arr is not None else _scalar_input(v))
        if I_arr is not None:
            set_input(v)
        r.state['V'].copy_(to_runner(neuron.V.value))
        load_state()
        r.seed(to_runner(neuron.spike.value.to(torch.uint8)), r.t + 1)
        r.dt = environ.get_dt()

    r.write_back = write_back
    r.set_input = set_input
    r.reload = reload
    r.replica_index = perm   # runner neuron of (replica b, neuron j), for rasters
    r.replica_identity = B == 1   # replica_index is the identity
    r.dt = environ.get_dt()
    return r
