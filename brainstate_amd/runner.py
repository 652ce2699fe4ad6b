"""Device-resident E/I network runner over the persistent C-ABI loop (bs_coba_*_run).

Holds connectivity, neuron state and the ring of event inboxes in HBM and
advances the network ``steps`` at a time in one launch.  This is the compiled form of
``brainstate.transform.for_loop(net.update, times)`` for the E/I nets of
examples/105_COBA_HH_2007_braincell.py:54-91 and examples/400_CUBA_2005_bpu.py:36-66.
"""
import ctypes

import numpy as np
import torch

from . import _native as N
from . import ops


def _ndim(x):
    return x.dim() if torch.is_tensor(x) else np.ndim(x)


def _dev_array(x, dtype, shape, dev, like=None):
    """``x`` as a contiguous ``dtype`` tensor on ``dev`` of ``shape`` (or broadcast to the
    shape of ``like``); a tensor already in that form is returned as it is."""
    if torch.is_tensor(x):
        t = x.to(device=dev, dtype=dtype)
    else:
        np_dtype = np.int32 if dtype == torch.int32 else np.float32
        t = torch.from_numpy(np.ascontiguousarray(np.asarray(x, np_dtype))).to(dev)
    t = t.expand(like.shape) if like is not None else t.reshape(shape)
    return t.contiguous()


class EINetRunner:
    """E/I network: neurons [0, n_exc) project with (idx_e, w_e), [n_exc, n) with (idx_i, w_i).

    ``model`` is 'lif' (Expon + COBA + LIFRef) or 'hh' (Expon + COBA + Hodgkin-Huxley).
    ``w_e``/``w_i`` are scalars (homogeneous) or [n_pre, K] arrays (heterogeneous).
    A step's input sums are exact integer sums, whatever the order in which events arrive:
    event counts turned into w added c times (homogeneous), or per-synapse weights rounded
    to multiples of 2^-S with one exponent S per projection (the largest that keeps every
    sum inside int32), summed exactly, then rounded once to fp32.
    ``delay_steps`` D: step t's synaptic inputs come from the spikes of step t-1-D (the
    reference's ``N.prefetch_delay('spike', D*dt)``; no spikes before the first step).
    ``I_ext`` (optional, [n]): each neuron's constant external input, in place of
    ``params.I_ext``.
    """

    def __init__(self, model, n, n_exc, idx_e, idx_i, w_e, w_i, params, V0, device='cuda',
                 blocks_per_cu=0, delay_steps=0, I_ext=None):
        N.require_gpu()
        self.delay_steps = int(delay_steps)
        self.model = model
        self.n, self.n_exc = int(n), int(n_exc)
        self.device = torch.device(device)
        dev = self.device
        # connectivity: numpy arrays are uploaded; tensors already on the device are used as
        # they are (a net built on the device is not copied through the host)
        self.idx_e = _dev_array(idx_e, torch.int32, (self.n_exc, -1), dev)
        self.idx_i = _dev_array(idx_i, torch.int32, (self.n - self.n_exc, -1), dev)
        for name, idx in (('idx_e', self.idx_e), ('idx_i', self.idx_i)):
            if idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= self.n):
                raise ValueError(f'{name}: target index out of range [0, {self.n})')
        self.k_e, self.k_i = self.idx_e.shape[1], self.idx_i.shape[1]
        het = _ndim(w_e) > 0 or _ndim(w_i) > 0
        if het:
            self.w_e = _dev_array(w_e, torch.float32, None, dev, like=self.idx_e)
            self.w_i = _dev_array(w_i, torch.float32, None, dev, like=self.idx_i)
            if not bool(torch.isfinite(self.w_e).all() & torch.isfinite(self.w_i).all()):
                raise ValueError('per-synapse weights must be finite')
            self.w_e_homo = self.w_i_homo = 0.0
        else:
            self.w_e = self.w_i = None
            self.w_e_homo, self.w_i_homo = (float(np.float32(float(w))) for w in (w_e, w_i))
        self.params = params
        self.I_ext = None if I_ext is None else _dev_array(I_ext, torch.float32, (self.n,), dev)
        f32 = dict(dtype=torch.float32, device=dev)
        self.spk = torch.zeros(self.n, dtype=torch.uint8, device=dev)
        self.t = 0   # absolute index of the next step
        V0 = (V0.to(device=dev, dtype=torch.float32).reshape(-1) if torch.is_tensor(V0) else
              torch.as_tensor(np.asarray(V0, np.float32)).to(dev))
        if model == 'lif':
            self.state = dict(V=V0.clone(), ge=torch.zeros(self.n, **f32),
                              gi=torch.zeros(self.n, **f32),
                              ref=torch.zeros(self.n, dtype=torch.int32, device=dev))
        elif model == 'hh':
            self.state = dict(V=V0.clone(), m=torch.empty(self.n, **f32),
                              h=torch.empty(self.n, **f32), n=torch.empty(self.n, **f32),
                              ge=torch.zeros(self.n, **f32), gi=torch.zeros(self.n, **f32))
            ops.hh_init(self.state['V'], self.state['m'], self.state['h'], self.state['n'])
        else:
            raise ValueError(f'unknown model {model!r}')
        self._net = N.Net(self.n, self.n_exc, self.k_e, self.k_i,
                          self.idx_e.data_ptr(), None if self.w_e is None else self.w_e.data_ptr(),
                          self.w_e_homo,
                          self.idx_i.data_ptr(), None if self.w_i is None else self.w_i.data_ptr(),
                          self.w_i_homo, self.spk.data_ptr(), int(blocks_per_cu),
                          self.delay_steps,
                          None if self.I_ext is None else self.I_ext.data_ptr())
        nbytes = int(N.lib().bs_net_workspace_size(ctypes.byref(self._net)))
        if nbytes == 0:
            N.check(N.BS_ERR_INVALID, 'bs_net_workspace_size')
        self.ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        N.check(N.lib().bs_net_prepare(ctypes.byref(self._net), N.ptr(self.ws),
                                       N.stream_handle(dev)), 'bs_net_prepare')

    def seed(self, spk, t0=1):
        """Take ``spk`` ([n], nonzero = spike) as the spikes of step t0 - 1, so that the next
        run starts at step t0 >= 1 with their inputs (synaptic delay 0)."""
        spk = torch.as_tensor(spk, device=self.device).reshape(-1)
        if spk.numel() != self.n:
            raise ValueError(f'seed: {spk.numel()} spikes for {self.n} neurons')
        spk = (spk != 0).to(torch.uint8).contiguous()
        N.check(N.lib().bs_net_seed_spikes(ctypes.byref(self._net), N.ptr(spk), int(t0),
                                           N.ptr(self.ws), N.stream_handle(self.device)),
                'bs_net_seed_spikes')
        self.spk.copy_(spk)
        self.t = int(t0)

    @property
    def grid_blocks(self):
        return int(N.lib().bs_net_grid_blocks(ctypes.byref(self._net)))

    def run(self, steps, counts=None, hashes=None, raster=None, inputs=None):
        """Advance ``steps`` steps in one launch.  Optional int32/uint32 [steps] outputs and a
        uint8 [steps, n] raster are filled on the device.  ``inputs`` (optional, [steps]):
        each step's external input in place of ``params.I_ext`` (bs_coba_*_run_inputs)."""
        s = self.state
        stream = N.stream_handle(self.device)
        steps = int(steps)
        tail = (N.ptr(counts), N.ptr(hashes), N.ptr(raster), N.ptr(self.ws), stream)
        if inputs is not None:
            inputs = torch.as_tensor(inputs, dtype=torch.float32,
                                     device=self.device).reshape(-1).contiguous()
            if inputs.numel() != steps:
                raise ValueError(f'run: {inputs.numel()} inputs for {steps} steps')
        if self.model == 'lif':
            st = N.LifState(s['V'].data_ptr(), s['ge'].data_ptr(), s['gi'].data_ptr(),
                            s['ref'].data_ptr())
            if inputs is None:
                rc = N.lib().bs_coba_lif_run(ctypes.byref(self._net), ctypes.byref(st),
                                             ctypes.byref(self.params), self.t, steps, *tail)
            else:
                rc = N.lib().bs_coba_lif_run_inputs(ctypes.byref(self._net), ctypes.byref(st),
                                                    ctypes.byref(self.params), N.ptr(inputs),
                                                    self.t, steps, *tail)
            N.check(rc, 'bs_coba_lif_run')
        else:
            st = N.HhState(s['V'].data_ptr(), s['m'].data_ptr(), s['h'].data_ptr(),
                           s['n'].data_ptr(), s['ge'].data_ptr(), s['gi'].data_ptr())
            if inputs is None:
                rc = N.lib().bs_coba_hh_run(ctypes.byref(self._net), ctypes.byref(st),
                                            ctypes.byref(self.params), self.t, steps, *tail)
            else:
                rc = N.lib().bs_coba_hh_run_inputs(ctypes.byref(self._net), ctypes.byref(st),
                                                   ctypes.byref(self.params), N.ptr(inputs),
                                                   self.t, steps, *tail)
            N.check(rc, 'bs_coba_hh_run')
        self.t += steps

    def check(self):
        """Synchronise and raise if a run's wait hit its spin limit or the per-synapse weights
        could not be given a fixed-point exponent (a weight is not finite)."""
        rc = N.lib().bs_net_error(N.ptr(self.ws), N.stream_handle(self.device))
        if rc != 0:
            raise N.NativeError(f'runner error {rc}: '
                                + N.lib().bs_last_error().decode(errors='replace'))
