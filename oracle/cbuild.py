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
               [('ref_steps', ctypes.c_int32)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        L.bso_coba_lif_run.restype = ctypes.c_longlong
        L.bso_max_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def lif_params(p):
    """From an oracle.neuron.LIFParams."""
    return _LifParams(p.V_rest, p.V_th, p.V_reset, p.inv_tau, p.R, p.I_ext, p.E_e, p.E_i, p.dt,
                      p.de, p.di, int(p.ref_steps))


def coba_lif_run(state, idx_e, idx_i, w_e, w_i, p, n_exc, steps, nthreads=0, counts=None,
                 hashes=None, delay=0):
    """Advance ``state`` (dict of numpy arrays V, ge, gi, ref, spk, in_e, in_i) in place.

    With ``delay`` D > 0, in_e / in_i are rings of D+1 input slots ([(D+1) * n]) and
    ``state['t']`` (absolute index of the next step, default 0) is advanced."""
    import numpy as np
    P = ctypes.c_void_p
    f = lambda a: a.ctypes.data_as(P) if a is not None else None
    het = np.ndim(w_e) > 0
    n = state['V'].size
    for key in ('in_e', 'in_i'):
        if state[key].size != (delay + 1) * n:
            raise ValueError(f'{key} must hold (delay + 1) * n = {(delay + 1) * n} floats')
    t0 = int(state.get('t', 0))
    state['t'] = t0 + int(steps)
    return lib().bso_coba_lif_run(
        ctypes.c_int(n), ctypes.c_int(n_exc), ctypes.c_int(idx_e.shape[1]),
        ctypes.c_int(idx_i.shape[1]), f(idx_e), f(w_e) if het else None,
        ctypes.c_float(0.0 if het else float(w_e)), f(idx_i), f(w_i) if het else None,
        ctypes.c_float(0.0 if het else float(w_i)), ctypes.byref(lif_params(p)),
        f(state['V']), f(state['ge']), f(state['gi']), f(state['ref']), f(state['spk']),
        f(state['in_e']), f(state['in_i']), ctypes.c_int(steps), f(counts), f(hashes),
        ctypes.c_int(nthreads), ctypes.c_int(delay), ctypes.c_longlong(t0))
