"""Event-driven connectivity layers with brainstate's constructor signatures.

* ``FixedNumConn`` / ``EventFixedNumConn`` / ``EventFixedProb`` --
  brainstate/nn/_event_fixedprob.py:65-255.  Same arguments, validation and connectivity
  stream (numpy MT19937 ``randint`` with replacement, :161-171); ``update(spk)`` runs the
  fused HIP spike-vector event mat-vec (C ABI ``bs_event_matvec_f32``: per-workgroup
  compaction of the spike vector, then the pre-major scatter of the active rows) instead of
  brainevent's kernel.
* ``EventLinear`` -- brainstate/nn/_event_linear.py:32-102, on ``bs_event_dense_f32``.

Tensors live on the GPU; there is no CPU path.
"""
import numpy as np
import torch

from .. import _native as N
from .. import ops
from .._state import FakeState, ParamState
from . import init
from ._module import Module

__all__ = ['FixedNumConn', 'EventFixedNumConn', 'EventFixedProb', 'EventLinear']


def _device():
    N.require_gpu()
    return torch.device('cuda', torch.cuda.current_device())


def _to_dev(a, dtype):
    if torch.is_tensor(a):
        return a.to(device=_device(), dtype=dtype).contiguous()
    return torch.as_tensor(np.ascontiguousarray(np.asarray(a)), dtype=dtype, device=_device())


class FixedPostNumConn:
    """Fixed-num (pre-major) connectivity: ``indices [n_pre, K]`` int32, weight scalar or
    ``[n_pre, K]``; the object brainevent.FixedPostNumConn stands for at
    brainstate/nn/_event_fixedprob.py:176-181."""

    def __init__(self, data, shape):
        w, indices = data
        self.indices = indices
        self.data = w
        self.shape = tuple(shape)

    def with_data(self, w):
        return FixedPostNumConn((w, self.indices), self.shape)

    def matvec_events(self, spk):
        n_pre, n_post = self.shape
        w = self.data
        if torch.is_tensor(w) and w.numel() > 1:
            w = w.expand(self.indices.shape) if w.shape != self.indices.shape else w
        return ops.event_matvec(spk, self.indices, w, n_post)


class CSR:
    """CSR connectivity of the afferent-ratio branch (brainstate/nn/_event_fixedprob.py:183-196)."""

    def __init__(self, data, shape):
        w, indices, indptr = data
        self.data, self.indices, self.indptr = w, indices, indptr
        self.shape = tuple(shape)

    def with_data(self, w):
        return CSR((w, self.indices, self.indptr), self.shape)

    def matvec_events(self, spk):
        n_pre, n_post = self.shape
        w = self.data
        if torch.is_tensor(w) and w.numel() > 1 and w.shape != self.indices.shape:
            w = w.expand(self.indices.shape)
        return ops.event_matvec(spk, self.indices, w, n_post, indptr=self.indptr)


def _weight_for_kernel(w):
    """Scalar (homogeneous) stays a float; arrays become fp32 device tensors."""
    if init._is_scalar(w):
        return float(w)
    t = _to_dev(w, torch.float32)
    return float(t.reshape(()).item()) if t.numel() == 1 else t


class FixedNumConn(Module):
    """brainstate/nn/_event_fixedprob.py:65-209 (same constructor and checks)."""
    __module__ = 'brainstate_amd.nn'

    def __init__(self, in_size, out_size, conn_num, conn_weight, efferent_target='post',
                 afferent_ratio=1., allow_multi_conn=True, seed=None, name=None,
                 conn_init='vmap', param_type=ParamState):
        super().__init__(name=name)
        self.in_size = init.to_size(in_size)
        self.out_size = init.to_size(out_size)
        self.efferent_target = efferent_target
        assert efferent_target in ('pre', 'post'), \
            'The target of the connection must be either "pre" or "post".'
        if efferent_target == 'pre':
            raise NotImplementedError(
                "efferent_target='pre' is not currently supported by FixedNumConn: "
                "the generated connection indices do not match the layout expected by "
                "the underlying brainevent sparse connection, which can raise a shape "
                "error or abort the process. Use efferent_target='post' instead.")
        assert 0. <= afferent_ratio <= 1., 'Afferent ratio must be in [0, 1].'
        if isinstance(conn_num, float):
            assert 0. <= conn_num <= 1., 'Connection probability must be in [0, 1].'
            conn_num = int(self.out_size[-1] * conn_num)
        assert isinstance(conn_num, int), 'Connection number must be an integer.'
        self.conn_num = conn_num
        self.seed = seed
        self.allow_multi_conn = allow_multi_conn
        if self.conn_num >= 1:
            n_post = self.out_size[-1]
            n_pre = self.in_size[-1]
            rng = np.random if seed is None else np.random.RandomState(seed)
            if allow_multi_conn:
                indices = rng.randint(0, n_post, size=(n_pre, self.conn_num))
            else:
                # brainstate draws these with its JAX RNG (init_indices_without_replace,
                # :39-62); that stream is not reproducible here, so numpy's is used.
                if self.conn_num > n_post:
                    raise ValueError('conn_num exceeds n_post without replacement')
                indices = np.stack([rng.choice(n_post, size=self.conn_num, replace=False)
                                    for _ in range(n_pre)]) if n_pre else \
                    np.zeros((0, self.conn_num), np.int64)
            indices = np.asarray(indices, dtype=np.int32)
            if afferent_ratio == 1.:
                w = init.param(conn_weight, (n_pre, self.conn_num), allow_none=False)
                self.weight = param_type(w)
                self.conn = FixedPostNumConn((w, _to_dev(indices, torch.int32)),
                                             shape=(n_pre, n_post))
            else:
                self.pre_selected = rng.random(n_pre) < afferent_ratio
                indices = indices[self.pre_selected].flatten()
                w = init.param(conn_weight, (indices.size,), allow_none=False)
                self.weight = param_type(w)
                indptr = (np.arange(1, n_pre + 1) * self.conn_num -
                          np.cumsum(~self.pre_selected) * self.conn_num)
                indptr = np.insert(indptr, 0, 0).astype(np.int32)
                self.conn = CSR((w, _to_dev(indices, torch.int32), _to_dev(indptr, torch.int32)),
                                shape=(n_pre, n_post))
        else:
            self.weight = FakeState(init.param(conn_weight, (), allow_none=False))

    def _matvec(self, x):
        if self.conn_num < 1:
            lead = tuple(x.shape[:-1]) if torch.is_tensor(x) else ()
            return torch.zeros(lead + (self.out_size[-1],), dtype=torch.float32,
                               device=_device())
        conn = self.conn.with_data(_weight_for_kernel(self.weight.value))
        x = x if torch.is_tensor(x) else _to_dev(x, torch.float32)
        if x.device.type != 'cuda':
            x = x.to(_device())
        if x.dim() == 1:
            return conn.matvec_events(x)
        flat = x.reshape(-1, x.shape[-1])
        out = torch.stack([conn.matvec_events(row) for row in flat])
        return out.reshape(tuple(x.shape[:-1]) + (self.out_size[-1],))

    def update(self, x):
        if torch.is_tensor(x) and x.dtype != torch.bool and x.dtype != torch.uint8:
            raise NotImplementedError(
                'FixedNumConn on non-event (value) inputs is a value-weighted sparse mat-vec, '
                'outside the event path; wrap spikes with EventFixedNumConn or pass bool spikes')
        return self._matvec(x)


class EventFixedNumConn(FixedNumConn):
    """brainstate/nn/_event_fixedprob.py:212-252: every nonzero entry of ``spk`` is one event."""
    __module__ = 'brainstate_amd.nn'

    def update(self, spk):
        return self._matvec(spk)


EventFixedProb = EventFixedNumConn


class EventLinear(Module):
    """brainstate/nn/_event_linear.py:32-102."""
    __module__ = 'brainstate_amd.nn'

    def __init__(self, in_size, out_size, weight, float_as_event=True, block_size=64,
                 name=None, param_type=ParamState):
        super().__init__(name=name)
        self.in_size = init.to_size(in_size)
        self.out_size = init.to_size(out_size)
        self.float_as_event = float_as_event
        self.block_size = block_size
        w = init.param(weight, (self.in_size[-1], self.out_size[-1]), allow_none=False)
        self.weight = param_type(w)

    def update(self, spk):
        w = self.weight.value
        x = spk if torch.is_tensor(spk) else _to_dev(spk, torch.float32)
        if x.device.type != 'cuda':
            x = x.to(_device())
        n_w = 1 if init._is_scalar(w) else int(np.prod(w.shape))
        if n_w == 1:
            # homogeneous shortcut, :77-97 (reference-owned arithmetic on the reduction)
            wv = float(np.asarray(w.cpu() if torch.is_tensor(w) else w).reshape(()))
            if self.float_as_event:
                reduced = (x != 0).sum(-1).to(torch.float32)
            else:
                reduced = x.to(torch.float32).sum(-1)
            return torch.ones(tuple(x.shape[:-1]) + (self.out_size[-1],), device=x.device) * \
                (reduced * np.float32(wv)).unsqueeze(-1)
        W = _to_dev(w, torch.float32)
        W = W.expand(self.in_size[-1], self.out_size[-1]).contiguous()
        if x.dtype not in (torch.bool, torch.uint8, torch.float32):
            x = x.to(torch.float32)
        return ops.event_dense(x, W, float_as_event=self.float_as_event)
