"""Event-driven connectivity layers with brainstate's constructor signatures.

* ``FixedNumConn`` / ``EventFixedNumConn`` / ``EventFixedProb`` --
  brainstate/nn/_event_fixedprob.py:65-255.  Same arguments, validation and connectivity
  stream (numpy MT19937 ``randint`` with replacement, :161-171); ``update(spk)`` runs the
  fused HIP spike-vector event mat-vec (C ABI ``bs_event_matvec_f32``: per-workgroup
  compaction of the spike vector, then the pre-major scatter of the active rows) instead of
  brainevent's kernel.
  With ``event_kernel='bucket'`` (or ``'auto'`` with per-synapse weights, or with a
  homogeneous weight onto more than 16,384 neurons whose rows average at least 4 synapses
  per destination bucket), the event path of inference runs the
  destination-bucketed operator instead (``bs_event_bucket_f32``: no global or fp32 atomics,
  exact fixed-point sums with the persistent runner's exponent, deterministic) on a layout
  built on first use and rebuilt when the weight value changes.
* ``EventLinear`` -- brainstate/nn/_event_linear.py:32-102, on ``bs_event_dense_f32``.

Both are differentiable (torch autograd, reverse and forward mode) with the gradients the
reference tests pin (brainstate/nn/_event_fixedprob_test.py:56-126,
brainstate/nn/_event_linear_test.py:51-125): those of the value formulation
``sum_i x[i] * w[i, :]`` / ``x @ W`` with the spike values x, on the HIP reverse-mode kernels
(``bs_event_matvec_vjp_f32``, ``bs_event_dense_vjp_f32``) and tangents built from
``bs_value_matvec_f32`` / ``bs_event_dense_f32``.

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


def _kw(w):
    """Weight argument for the kernels: a float for one (homogeneous) value, else the tensor."""
    if not torch.is_tensor(w):
        return float(w)
    return float(w.reshape(())) if w.numel() == 1 else w


def _het(w):
    """True for per-synapse weights (a tensor of more than one value)."""
    return torch.is_tensor(w) and w.numel() > 1


def _grad_weight(w, like):
    """The weight as a tensor for the autograd Functions (a Python scalar becomes a 0-d
    fp32 tensor on the device of ``like``)."""
    if torch.is_tensor(w):
        return w
    return torch.tensor(float(w), dtype=torch.float32, device=like.device)


class _EventMatvecFn(torch.autograd.Function):
    """out = mat-vec of spk with weights w over (indices, indptr): every nonzero spike is one
    event (value=False) or weighs by its value (value=True).  Differentiable in the spike
    values and the weights, with the derivatives of the value formulation in both modes.
    ``spk`` may carry leading batch dimensions ([..., n_pre] -> [..., n_post])."""

    @staticmethod
    def forward(spk, w, indices, indptr, n_post, value=False):
        if value:
            return ops.value_matvec(spk, indices, _kw(w), n_post, indptr=indptr)
        return ops.event_matvec(spk, indices, _kw(w), n_post, indptr=indptr)

    @staticmethod
    def setup_context(ctx, inputs, output):
        spk, w, indices, indptr, n_post, _ = inputs
        ctx.save_for_backward(spk, w, indices, indptr)
        ctx.save_for_forward(spk, w, indices, indptr)
        ctx.n_post = n_post

    @staticmethod
    def backward(ctx, g):
        spk, w, indices, indptr = ctx.saved_tensors
        need_s, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        n_pre = spk.shape[-1] if spk.dim() else 1
        rows = spk.reshape(-1, n_pre)
        grows = g.reshape(-1, ctx.n_post)
        if rows.shape[0] == 1:
            gs, gw = ops.event_matvec_vjp(rows[0], indices, _kw(w), ctx.n_post,
                                          grows[0].contiguous(), indptr=indptr,
                                          need_spk=need_s, need_w=need_w)
        else:   # every batch row in one launch; weight gradients summed in row order
            gs, gw = ops.event_matvec_vjp_batch(rows, indices, _kw(w), ctx.n_post, grows,
                                                indptr=indptr, need_spk=need_s, need_w=need_w)
        gs = gs.reshape(spk.shape).to(spk.dtype) if need_s else None
        if gw is not None:
            gw = gw.reshape(w.shape)
        return gs, gw, None, None, None, None

    @staticmethod
    def jvp(ctx, dspk, dw, *_):
        spk, w, indices, indptr = ctx.saved_tensors
        lead = tuple(spk.shape[:-1])
        t = torch.zeros(lead + (ctx.n_post,), dtype=torch.float32, device=indices.device)
        if dspk is not None:
            ops.value_matvec(dspk.reshape(spk.shape), indices, _kw(w), ctx.n_post,
                             indptr=indptr, out=t, accumulate=True)
        if dw is not None:
            ops.value_matvec(spk.to(torch.float32), indices, _kw(dw), ctx.n_post,
                             indptr=indptr, out=t, accumulate=True)
        return t


def _no_autodiff(*ts):
    """True when no operand takes part in reverse or forward mode autodiff (including the
    wrapped tensors of torch.func transforms)."""
    from torch.autograd import forward_ad
    for t in ts:
        if torch.is_tensor(t):
            if t.requires_grad and torch.is_grad_enabled():
                return False
            if forward_ad.unpack_dual(t).tangent is not None:
                return False
            if torch._C._functorch.is_functorch_wrapped_tensor(t):
                return False
    return True


_BUCKET_AUTO_POSTS = 16384   # 'auto', homogeneous weight: bucketed above this many outputs
_BUCKET_AUTO_SEG = 4         # ... and with at least this many synapses per row and bucket


def _wants_grad(*ts):
    """Route through the autograd Functions only when autodiff may record this call: grad
    mode on and an operand that requires grad, carries a forward-mode tangent or is wrapped
    by a torch.func transform.  Otherwise the kernels are called directly (no Function
    dispatch: its argument binding cost ~40 us of host time per call)."""
    return torch.is_grad_enabled() and not _no_autodiff(*ts)


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

    def matvec_events(self, spk, value=False):
        n_pre, n_post = self.shape
        w = self.data
        if torch.is_tensor(w) and w.numel() > 1:
            w = w.expand(self.indices.shape) if w.shape != self.indices.shape else w
        if _wants_grad(spk, w):
            return _EventMatvecFn.apply(spk, _grad_weight(w, spk), self.indices, None, n_post,
                                        value)
        wk = _kw(w) if torch.is_tensor(w) else w
        if value:
            return ops.value_matvec(spk, self.indices, wk, n_post)
        return ops.event_matvec(spk, self.indices, wk, n_post)


class CSR:
    """CSR connectivity of the afferent-ratio branch (brainstate/nn/_event_fixedprob.py:183-196)."""

    def __init__(self, data, shape):
        w, indices, indptr = data
        self.data, self.indices, self.indptr = w, indices, indptr
        self.shape = tuple(shape)

    def with_data(self, w):
        return CSR((w, self.indices, self.indptr), self.shape)

    def matvec_events(self, spk, value=False):
        n_pre, n_post = self.shape
        w = self.data
        if torch.is_tensor(w) and w.numel() > 1 and w.shape != self.indices.shape:
            w = w.expand(self.indices.shape)
        if _wants_grad(spk, w):
            return _EventMatvecFn.apply(spk, _grad_weight(w, spk), self.indices, self.indptr,
                                        n_post, value)
        wk = _kw(w) if torch.is_tensor(w) else w
        if value:
            return ops.value_matvec(spk, self.indices, wk, n_post, indptr=self.indptr)
        return ops.event_matvec(spk, self.indices, wk, n_post, indptr=self.indptr)


def _weight_for_kernel(w):
    """fp32 device tensor of the weight, or a Python float for a scalar weight that is not a
    tensor (no host-to-device copy and no read-back per call); a tensor that requires grad
    keeps its autograd graph."""
    if torch.is_tensor(w):
        return _to_dev(w, torch.float32)
    if init._is_scalar(w):
        return float(w)   # one homogeneous value: passed to the kernels as a float
    return _to_dev(w, torch.float32)


def _module_weight(mod, v):
    """``_weight_for_kernel(v)`` for the weight State value ``v`` of module ``mod``; the device
    copy of a numpy weight is kept on the module while the State holds the same array object
    (an eager step would otherwise copy every synapse's weight to the device: 400 MB per step
    for 1M neurons x 100 synapses).  A numpy array changed in place is not seen (it carries
    no version): assign a new array, or a tensor."""
    if isinstance(v, np.ndarray) and not init._is_scalar(v):
        c = getattr(mod, '_wdev', None)
        if c is None or c[0] is not v:
            c = (v, _to_dev(v, torch.float32))
            mod._wdev = c
        return c[1]
    return _weight_for_kernel(v)


class FixedNumConn(Module):
    """brainstate/nn/_event_fixedprob.py:65-209 (same constructor and checks)."""
    __module__ = 'brainstate_amd.nn'

    def __init__(self, in_size, out_size, conn_num, conn_weight, efferent_target='post',
                 afferent_ratio=1., allow_multi_conn=True, seed=None, name=None,
                 conn_init='vmap', param_type=ParamState, event_kernel='auto'):
        super().__init__(name=name)
        if event_kernel not in ('auto', 'atomic', 'bucket'):
            raise ValueError(f"event_kernel must be 'auto', 'atomic' or 'bucket', not {event_kernel!r}")
        self.event_kernel = event_kernel
        self._bucket = None       # (key of the weight value, layout)
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
        if self.conn_num >= 1 and seed is not None:
            self._build_on_device(n_pre=self.in_size[-1], n_post=self.out_size[-1],
                                  conn_weight=conn_weight, afferent_ratio=afferent_ratio,
                                  param_type=param_type)
        elif self.conn_num >= 1:
            n_post = self.out_size[-1]
            n_pre = self.in_size[-1]
            rng = np.random  # seed=None: the global numpy stream, as the reference (:163)
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

    def _build_on_device(self, n_pre, n_post, conn_weight, afferent_ratio, param_type):
        """Index draws on the device (bs_conn_fixed_num*): with replacement they equal
        RandomState(seed).randint(0, n_post, (n_pre, K)) bit for bit (:163-168), and the
        afferent selection is the same stream's next random(n_pre) < afferent_ratio (:186).
        Without replacement (the reference's JAX draws, :39-62) the rows come from Philox."""
        k, seed = self.conn_num, int(self.seed)
        ratio = None if afferent_ratio == 1. else float(afferent_ratio)
        if self.allow_multi_conn:
            indices, sel = ops.conn_fixed_num(seed, n_pre, k, n_post, ratio)
        else:
            if k > n_post:
                raise ValueError('conn_num exceeds n_post without replacement')
            indices = ops.conn_fixed_num_unique(seed, n_pre, k, n_post)
            sel = None if ratio is None else ops.conn_fixed_num(seed, n_pre, 0, n_post, ratio)[1]
        if ratio is None:
            w = init.param(conn_weight, (n_pre, k), allow_none=False)
            self.weight = param_type(w)
            self.conn = FixedPostNumConn((w, indices), shape=(n_pre, n_post))
        else:
            self.pre_selected = sel.cpu().numpy()
            indptr, csr_indices = ops.csr_from_selected(indices, sel)
            w = init.param(conn_weight, (csr_indices.numel(),), allow_none=False)
            self.weight = param_type(w)
            self.conn = CSR((w, csr_indices, indptr), shape=(n_pre, n_post))

    def _matvec(self, x, value=False):
        if self.conn_num < 1:
            lead = tuple(x.shape[:-1]) if torch.is_tensor(x) else ()
            return torch.zeros(lead + (self.out_size[-1],), dtype=torch.float32,
                               device=_device())
        w = _module_weight(self, self.weight.value)
        x = x if torch.is_tensor(x) else _to_dev(x, torch.float32)
        if x.device.type != 'cuda':
            x = x.to(_device())
        if not value and self._bucketed(w) and _no_autodiff(x, w):
            L = self._bucket_layout(w)
            if x.dim() == 1:
                return ops.event_bucket(x, L)
            # [..., n_pre] spikes: each row through the bucketed operator (the same sums as a
            # replica inside the union runner)
            rows = x.reshape(-1, x.shape[-1])
            out = torch.empty(rows.shape[0], self.out_size[-1], dtype=torch.float32,
                              device=x.device)
            for b in range(rows.shape[0]):
                ops.event_bucket(rows[b], L, out=out[b])
            return out.reshape(tuple(x.shape[:-1]) + (self.out_size[-1],))
        conn = self.conn.with_data(w)
        return conn.matvec_events(x, value)   # [..., n_pre] -> [..., n_post], one launch

    def _bucketed(self, w):
        """'auto': per-synapse weights always take the bucketed operator -- its exact
        fixed-point sums are those the persistent runner adds (same exponent rule), so an
        eager step equals the fused one bit for bit and does not depend on the order of the
        device's atomics -- and a homogeneous weight above 16,384 outputs when a row's
        synapses average at least 4 per bucket (elsewhere the atomic kernel, which adds equal
        addends, whose sums do not depend on their order: both give the same bits).  Measured
        (us per call at p = 0.0005 / 0.01 / 0.1): 800k x 1M, K = 100 (82 buckets, 1.2 synapses
        per bucket) bucketed 31 / 64 / 425, atomic 14 / 46 / 393; 100k x 100k, K = 100 (9
        buckets, 11 per bucket) bucketed 11 / 15 / 21, atomic 13 / 14 / 57; 400k x 400k, K =
        300 (33 buckets, 9 per bucket) 21 / 26 / 108 against 13 / 65 / 581."""
        if self.event_kernel == 'bucket':
            return True
        if self.event_kernel != 'auto':
            return False
        if _het(w):
            return True
        n_post = self.out_size[-1]
        if n_post <= _BUCKET_AUTO_POSTS:
            return False
        if getattr(self, '_plan', None) is None or self._plan[0] != n_post:
            self._plan = (n_post, ops.bucket_plan(n_post)[0])
        return self.conn_num >= _BUCKET_AUTO_SEG * self._plan[1]

    def _bucket_layout(self, w):
        """Destination-bucketed layout of the current connectivity and weight; rebuilt when the
        weight State is assigned a new value (another object, or another scalar value) or its
        tensor is modified in place (version counter).  The cache holds the weight object it
        was built from, so a freed weight's identity cannot be recycled by a new one; a numpy
        weight changed in place is not seen (it carries no version)."""
        v = self.weight.value
        key = (v._version if torch.is_tensor(v) else None,
               float(v) if init._is_scalar(v) else None)
        if self._bucket is None or self._bucket[0] is not v or self._bucket[1] != key:
            homo = not _het(w)
            conn = self.conn
            indptr = getattr(conn, 'indptr', None)
            wt = None
            if not homo:
                wt = w.detach()
                if indptr is None and wt.shape != conn.indices.shape:
                    wt = wt.expand(conn.indices.shape)
            layout = ops.build_buckets(conn.indices, self.out_size[-1], w=wt,
                                       w_homo=_kw(w) if homo else 0.0,
                                       indptr=indptr)
            self._bucket = (v, key, layout)
        return self._bucket[2]

    def update(self, x):
        """``x @ conn`` (:202-209): bool spikes are events; any other dtype is a
        value-weighted sparse mat-vec (sum_i x[i] * w[i, :])."""
        value = not (torch.is_tensor(x) and x.dtype in (torch.bool, torch.uint8)) and not (
            isinstance(x, np.ndarray) and x.dtype == np.bool_)
        return self._matvec(x, value)


class EventFixedNumConn(FixedNumConn):
    """brainstate/nn/_event_fixedprob.py:212-252: every nonzero entry of ``spk`` is one event."""
    __module__ = 'brainstate_amd.nn'

    def update(self, spk):
        return self._matvec(spk)


EventFixedProb = EventFixedNumConn


class _EventDenseFn(torch.autograd.Function):
    """out = spk @ W (rows of W selected by the nonzero spikes when float_as_event, else
    weighted by the spike values); derivatives of spk_values @ W in both modes."""

    @staticmethod
    def forward(spk, W, float_as_event):
        return ops.event_dense(spk, W, float_as_event=float_as_event)

    @staticmethod
    def setup_context(ctx, inputs, output):
        spk, W, fae = inputs
        ctx.save_for_backward(spk, W)
        ctx.save_for_forward(spk, W)
        ctx.fae = fae

    @staticmethod
    def backward(ctx, g):
        spk, W = ctx.saved_tensors
        gs, gw = ops.event_dense_vjp(spk, W, g, need_spk=ctx.needs_input_grad[0],
                                     need_w=ctx.needs_input_grad[1])
        if gs is not None:
            gs = gs.reshape(spk.shape).to(spk.dtype)
        return gs, gw, None

    @staticmethod
    def jvp(ctx, dspk, dW, _):
        spk, W = ctx.saved_tensors
        t = None
        if dspk is not None:
            t = ops.event_dense(dspk.to(torch.float32), W, float_as_event=False)
        if dW is not None:
            u = ops.event_dense(spk, dW.contiguous(), float_as_event=ctx.fae)
            t = u if t is None else t + u
        return t


class _HomoLinearFn(torch.autograd.Function):
    """EventLinear's homogeneous shortcut (brainstate/nn/_event_linear.py:77-97): every output
    is (count of nonzero spikes, or their sum) * w.  Derivatives of x @ (ones * w), as the
    reference pins them (brainstate/nn/_event_linear_test.py:51-125)."""

    @staticmethod
    def forward(x, w, n_out, float_as_event):
        red = (x != 0).sum(-1).to(torch.float32) if float_as_event else x.to(torch.float32).sum(-1)
        return torch.ones(tuple(x.shape[:-1]) + (n_out,), device=x.device) * \
            (red * w.reshape(()).to(torch.float32)).unsqueeze(-1)

    @staticmethod
    def setup_context(ctx, inputs, output):
        x, w, n_out, fae = inputs
        ctx.save_for_backward(x, w)
        ctx.save_for_forward(x, w)
        ctx.n_out, ctx.fae = n_out, fae

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        gsum = g.sum(-1)
        gx = gw = None
        if ctx.needs_input_grad[0]:
            gx = (gsum.unsqueeze(-1) * w.reshape(())).expand(x.shape).to(x.dtype)
        if ctx.needs_input_grad[1]:
            gw = (gsum * x.to(torch.float32).sum(-1)).sum().reshape(w.shape).to(w.dtype)
        return gx, gw, None, None

    @staticmethod
    def jvp(ctx, dx, dw, *_):
        x, w = ctx.saved_tensors
        red = (x != 0).sum(-1).to(torch.float32) if ctx.fae else x.to(torch.float32).sum(-1)
        t = torch.zeros(tuple(x.shape[:-1]), dtype=torch.float32, device=x.device)
        if dx is not None:
            t = t + dx.to(torch.float32).sum(-1) * w.reshape(())
        if dw is not None:
            t = t + red * dw.reshape(())
        return t.unsqueeze(-1).expand(tuple(x.shape[:-1]) + (ctx.n_out,)).contiguous()


class EventLinear(Module):
    """brainstate/nn/_event_linear.py:32-102.

    ``event_kernel`` picks the kernel of the heterogeneous event product: ``'packed'`` (and
    ``'auto'``, for event inputs, i.e. ``float_as_event=True``, and up to 65536 inputs) packs
    the weight once per value (ops.pack_dense; repacked when the weight State is assigned or
    modified in place) and runs the matrix-core form, exact in fixed point per column;
    ``'stream'`` streams W through the fp32 event kernel in its documented chunk order (also
    used for value inputs, for weights holding inf or NaN, and whenever autodiff records the
    spikes or the weight).  Packing reads W twice and
    writes ~1.25x its size, so the packed form pays from the second call with one weight.
    Accuracy of the packed form: |out - exact| <= 2^-24 * max|W[:, j]| + half an ulp of the
    output, in column j -- within abs 1e-6 + rel 1e-5 of the exact sum whenever the columns'
    largest |w| is at most 16 (a 4096 x 4096 W ~ N(0, 1/64) has max |w| ~ 0.6); an fp32 sum in
    any order has errors of the same size, ulps of its partial sums, on larger weights."""
    __module__ = 'brainstate_amd.nn'

    def __init__(self, in_size, out_size, weight, float_as_event=True, block_size=64,
                 name=None, param_type=ParamState, event_kernel='auto'):
        super().__init__(name=name)
        if event_kernel not in ('auto', 'packed', 'stream'):
            raise ValueError(f'event_kernel must be auto, packed or stream, got {event_kernel!r}')
        self.in_size = init.to_size(in_size)
        self.out_size = init.to_size(out_size)
        self.float_as_event = float_as_event
        self.block_size = block_size
        self.event_kernel = event_kernel
        w = init.param(weight, (self.in_size[-1], self.out_size[-1]), allow_none=False)
        self.weight = param_type(w)
        self._packed = None

    def _packed_weight(self, W):
        """ops.pack_dense of the current weight; None when the packed form does not apply.
        A torch weight is packed once per value (cached on the tensor object, its storage and
        its version counter, which in-place changes bump); a numpy weight, which carries no
        version, is packed on every call."""
        if self.event_kernel == 'stream' or not self.float_as_event:
            return None
        if ops.dense_digits(W.shape[0]) == 0:
            return None
        v = self.weight.value
        if not torch.is_tensor(v):
            P = ops.pack_dense(W.detach())
            return P if P['finite'] else None
        # the cache holds the weight tensor it packed, so a freed weight's identity and
        # storage cannot be recycled by a new tensor while the packed form is kept
        key = (v.data_ptr(), v._version)
        if self._packed is None or self._packed[0] is not v or self._packed[1] != key:
            self._packed = (v, key, ops.pack_dense(W.detach()))
        P = self._packed[2]
        return P if P['finite'] else None

    def update(self, spk):
        w = self.weight.value
        x = spk if torch.is_tensor(spk) else _to_dev(spk, torch.float32)
        if x.device.type != 'cuda':
            x = x.to(_device())
        n_w = 1 if init._is_scalar(w) else int(np.prod(w.shape))
        if n_w == 1:
            # homogeneous shortcut, :77-97 (reference-owned arithmetic on the reduction)
            wt = _grad_weight(_weight_for_kernel(w), x).reshape(())
            return _HomoLinearFn.apply(x, wt, self.out_size[-1], self.float_as_event)
        W = _module_weight(self, w)
        W = W.expand(self.in_size[-1], self.out_size[-1]).contiguous()
        if x.dtype not in (torch.bool, torch.uint8, torch.float32):
            x = x.to(torch.float32)
        if _no_autodiff(x, W):
            P = self._packed_weight(W)
            if P is not None:
                return ops.event_dense_packed(x, P)
        if _wants_grad(x, W):
            return _EventDenseFn.apply(x, W, self.float_as_event)
        return ops.event_dense(x, W, float_as_event=self.float_as_event)
