"""Build + ctypes binding of the C restatement oracle/c/coba_cpu.c (test infrastructure only).

Output: oracle/_build/libbsoracle.so (git-ignored).  Used by tests/ as a second checker
and by bench.py's ``cpu_baseline`` leg as the timed multi-core CPU baseline.
"""
import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, 'c', 'coba_cpu.c')
OUTDIR = os.path.join(HERE, '_build')
LIB = os.path.join(OUTDIR, 'libbsoracle.so')


def build(verbose=False):
    os.makedirs(OUTDIR, exist_ok=True)
    cmd = ['gcc', '-O3', '-march=x86-64-v2', '-fopenmp', '-ffp-contract=off', '-fno-fast-math',
           '-fPIC', '-shared', SRC, '-o', LIB + '.tmp', '-lm']
    if verbose:
        print(' '.join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(LIB + '.tmp', LIB)
    return LIB


class _LifParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_float) for n in ('V_rest', 'V_th', 'V_reset', 'inv_tau', 'R', 'I_ext',
                                                'E_e', 'E_i', 'dt', 'decay_e', 'decay_i')] + \
               [('ref_steps', ctypes.c_int32), ('cuba', ctypes.c_int32),
                ('scale_e', ctypes.c_float), ('scale_i', ctypes.c_float),
                ('soft_reset', ctypes.c_int32), ('deferred_reset', ctypes.c_int32)]


class _HhParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_float) for n in ('ENa', 'gNa', 'EK', 'gK', 'EL', 'gL', 'inv_C',
                                                'V_th', 'I_ext', 'E_e', 'E_i', 'dt', 'decay_e',
                                                'decay_i')]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        L.bso_coba_lif_run.restype = ctypes.c_longlong
        L.bso_coba_hh_run.restype = ctypes.c_longlong
        L.bso_max_threads.restype = ctypes.c_int
        L.bso_net_qexp.restype = ctypes.c_int
        _lib = L
    return _lib


def lif_params(p):
    """From an oracle.neuron.LIFParams."""
    return _LifParams(p.V_rest, p.V_th, p.V_reset, p.inv_tau, p.R, p.I_ext, p.E_e, p.E_i, p.dt,
                      p.de, p.di, int(p.ref_steps), int(bool(getattr(p, 'cuba', False))),
                      float(getattr(p, 'scale_e', 1.0)), float(getattr(p, 'scale_i', 1.0)),
                      int(bool(getattr(p, 'soft_reset', False))),
                      int(bool(getattr(p, 'deferred_reset', False))))


def hh_params(p):
    """From an oracle.neuron.HHParams."""
    return _HhParams(p.ENa, p.gNa, p.EK, p.gK, p.EL, p.gL, p.inv_C, p.V_th, p.I_ext, p.E_e,
                     p.E_i, p.dt, p.de, p.di)


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def net_qexp(idx_e, w_e, idx_i, w_i, n):
    """Fixed-point exponents (S_e, S_i) of per-synapse weights, as the runner fixes them."""
    import numpy as np
    q = np.zeros(2, np.int32)
    idx_e = np.ascontiguousarray(idx_e, np.int32)
    idx_i = np.ascontiguousarray(idx_i, np.int32)
    w_e = np.ascontiguousarray(np.broadcast_to(np.asarray(w_e, np.float32), idx_e.shape))
    w_i = np.ascontiguousarray(np.broadcast_to(np.asarray(w_i, np.float32), idx_i.shape))
    rc = lib().bso_net_qexp(ctypes.c_int(n), ctypes.c_int(idx_e.shape[0]),
                            ctypes.c_int(idx_e.shape[1]), ctypes.c_int(idx_i.shape[1]),
                            _ptr(idx_e), _ptr(w_e), _ptr(idx_i), _ptr(w_i), _ptr(q))
    if rc:
        raise ValueError('a per-synapse weight is not finite (or too large)')
    return int(q[0]), int(q[1])


def _common(state, idx_e, idx_i, w_e, w_i, delay):
    import numpy as np
    het = np.ndim(w_e) > 0
    n = state['V'].size
    for key in ('in_e', 'in_i'):
        if state[key].size != (delay + 1) * n or state[key].itemsize != 4:
            raise ValueError(f'{key} must hold (delay + 1) * n = {(delay + 1) * n} 4-byte values')
    qexp = None
    if het:
        if 'qexp' not in state:
            state['qexp'] = np.array(net_qexp(idx_e, w_e, idx_i, w_i, n), np.int32)
        qexp = state['qexp']
    t0 = int(state.get('t', 0))
    ctf = ctypes.c_float
    args = [ctypes.c_int(n), None, ctypes.c_int(idx_e.shape[1]), ctypes.c_int(idx_i.shape[1]),
            _ptr(idx_e), _ptr(w_e) if het else None, ctf(0.0 if het else float(w_e)),
            _ptr(idx_i), _ptr(w_i) if het else None, ctf(0.0 if het else float(w_i))]
    return args, qexp, t0


def coba_lif_run(state, idx_e, idx_i, w_e, w_i, p, n_exc, steps, nthreads=0, counts=None,
                 hashes=None, delay=0):
    """Advance ``state`` (dict of numpy arrays V, ge, gi, ref, spk, in_e, in_i) in place.

    With ``delay`` D > 0, in_e / in_i are rings of D+1 input slots ([(D+1) * n]) and
    ``state['t']`` (absolute index of the next step, default 0) is advanced.  With
    per-synapse weights the rings hold int32 fixed-point sums (start them at zero) and
    ``state['qexp']`` caches the exponents.  ``state['I_ext']`` (optional, float32 [n]) is each
    neuron's external input in place of ``p.I_ext``."""
    args, qexp, t0 = _common(state, idx_e, idx_i, w_e, w_i, delay)
    args[1] = ctypes.c_int(n_exc)
    state['t'] = t0 + int(steps)
    return lib().bso_coba_lif_run(
        *args, ctypes.byref(lif_params(p)),
        _ptr(state['V']), _ptr(state['ge']), _ptr(state['gi']), _ptr(state['ref']),
        _ptr(state['spk']), _ptr(state['in_e']), _ptr(state['in_i']), ctypes.c_int(steps),
        _ptr(counts), _ptr(hashes), ctypes.c_int(nthreads), ctypes.c_int(delay),
        ctypes.c_longlong(t0), _ptr(qexp), _ptr(_input(state)))


def _input(state):
    import numpy as np
    x = state.get('I_ext')
    return None if x is None else np.ascontiguousarray(x, np.float32)


def coba_hh_run(state, idx_e, idx_i, w_e, w_i, p, n_exc, steps, nthreads=0, counts=None,
                hashes=None, delay=0):
    """HH network (state: V, m, h, n, ge, gi, spk, in_e, in_i), as coba_lif_run."""
    args, qexp, t0 = _common(state, idx_e, idx_i, w_e, w_i, delay)
    args[1] = ctypes.c_int(n_exc)
    state['t'] = t0 + int(steps)
    return lib().bso_coba_hh_run(
        *args, ctypes.byref(hh_params(p)),
        _ptr(state['V']), _ptr(state['m']), _ptr(state['h']), _ptr(state['n']),
        _ptr(state['ge']), _ptr(state['gi']), _ptr(state['spk']), _ptr(state['in_e']),
        _ptr(state['in_i']), ctypes.c_int(steps), _ptr(counts), _ptr(hashes),
        ctypes.c_int(nthreads), ctypes.c_int(delay), ctypes.c_longlong(t0), _ptr(qexp),
        _ptr(_input(state)))


def hh_init(V):
    """Steady-state gates (m, h, n) at V."""
    import numpy as np
    V = np.ascontiguousarray(V, np.float32)
    m, h, n = (np.empty_like(V) for _ in range(3))
    lib().bso_hh_init(ctypes.c_int(V.size), _ptr(V), _ptr(m), _ptr(h), _ptr(n))
    return m, h, n


def lif_state(V0, delay=0):
    """Fresh LIF state for coba_lif_run (rings zero; they are reinterpreted as int32 sums
    with per-synapse weights)."""
    import numpy as np
    F = np.float32
    n = V0.size
    return dict(V=np.array(V0, F), ge=np.zeros(n, F), gi=np.zeros(n, F),
                ref=np.zeros(n, np.int32), spk=np.zeros(n, np.uint8),
                in_e=np.zeros((delay + 1) * n, F), in_i=np.zeros((delay + 1) * n, F))


def hh_state(V0, delay=0):
    """Fresh HH state for coba_hh_run, gates at steady state."""
    import numpy as np
    F = np.float32
    n = V0.size
    V = np.array(V0, F)
    m, h, ng = hh_init(V)
    return dict(V=V, m=m, h=h, n=ng, ge=np.zeros(n, F), gi=np.zeros(n, F),
                spk=np.zeros(n, np.uint8), in_e=np.zeros((delay + 1) * n, F),
                in_i=np.zeros((delay + 1) * n, F))
