"""``brainstate.nn.exp_euler_step`` (brainstate/nn/_exp_euler.py:33-276) on the device.

One exponential-Euler step of ``dx/dt = f(x, *args)`` (optionally ``+ g(x, *args) dW``):

    J = vector-Jacobian product of f at x with ones    (the reference's ``vector_grad``,
                                                          the diagonal of df/dx for an
                                                          elementwise f)
    x' = x + (dt * exprel(dt * J)) * f(x)                 (one fused multiply-add)
    x' += g(x) * sqrt(dt) * N(0, 1)                        (when a diffusion g is given)

The drift and J come from torch autograd on the caller's function (its own arithmetic, in the
state's dtype); the update itself runs in the HIP kernel ``bs_exp_euler_f32`` /
``bs_exp_euler_f64``, with the exprel the fused neuron updates use.  float16 / bfloat16
states are stepped in float32 and rounded back.  The diffusion noise is torch's normal
generator on the device (the reference draws from brainstate.random: that stream is not
reproduced).  Units (brainunit) are not modelled.
"""
import math

import numpy as np
import torch

from .. import _native as N
from .. import environ

__all__ = ['exp_euler_step']

_FLOATS = (torch.float16, torch.bfloat16, torch.float32, torch.float64)


def _on_device(x):
    """The state as a device tensor: tensors keep their dtype; Python and numpy floats take
    the default float dtype (float32 unless the precision is 64), as jnp.asarray does."""
    dev = torch.device('cuda', torch.cuda.current_device())
    if torch.is_tensor(x):
        return x.to(dev)
    t = torch.as_tensor(x)
    if torch.is_floating_point(t):
        t = t.to(torch.float64 if np.dtype(environ.dftype()) == np.float64 else torch.float32)
    return t.to(dev)


def _drift_and_vjp(fn, x, rest, kwargs):
    """(f(x, *rest), ones^T df/dx) with x's shape and dtype."""
    xg = x.detach().clone().requires_grad_(True)
    with torch.enable_grad():
        y = fn(xg, *rest, **kwargs)
        # a drift built without x (a constant) may live on the host: bring it to x's device
        y = (y if torch.is_tensor(y) else torch.as_tensor(y)).to(device=x.device, dtype=x.dtype)
        jac = None
        if y.requires_grad:
            jac, = torch.autograd.grad(y, xg, grad_outputs=torch.ones_like(y),
                                       allow_unused=True)
    drift = torch.broadcast_to(y.detach(), x.shape)
    jac = torch.zeros_like(x) if jac is None else jac.detach()
    return drift, jac


def _check_operands(ts, n):
    """Every operand the kernel reads or writes is a contiguous tensor of n elements on the
    first one's device, and that device is a GPU (a host pointer must never reach a kernel)."""
    dev = ts[0].device
    if dev.type != 'cuda':
        raise ValueError(f'exp_euler_step: operands must be on a GPU, got {dev}')
    for t in ts:
        if t.device != dev or t.numel() != n or not t.is_contiguous():
            raise ValueError(f'exp_euler_step: operand on {t.device} with {t.numel()} '
                             f'elements (contiguous: {t.is_contiguous()}), expected {n} on {dev}')


def _step(x, drift, jac, dt):
    """x + dt * exprel(dt * jac) * drift on the device (HIP kernel)."""
    work = torch.float64 if x.dtype == torch.float64 else torch.float32
    xs, fs, js = (t.to(device=x.device, dtype=work).contiguous() for t in (x, drift, jac))
    out = torch.empty_like(xs)
    n = xs.numel()
    _check_operands((xs, fs, js, out), n)
    stream = N.stream_handle(xs.device)
    if work == torch.float64:
        rc = N.lib().bs_exp_euler_f64(n, N.ptr(xs), N.ptr(fs), N.ptr(js), float(dt), N.ptr(out),
                                      stream)
    else:
        rc = N.lib().bs_exp_euler_f32(n, N.ptr(xs), N.ptr(fs), N.ptr(js), float(dt), N.ptr(out),
                                      stream)
    N.check(rc, 'bs_exp_euler')
    return out.to(x.dtype)


def exp_euler_step(fn, *args, **kwargs):
    """``exp_euler_step(f, x, *args)`` or ``exp_euler_step(f, g, x, *args)``: the state after
    one step of dt (``environ.get_dt()``); ``args`` and ``kwargs`` go to f (and g)."""
    assert callable(fn), 'The drift function should be callable.'
    assert len(args) > 0, 'The input arguments should not be empty.'
    diffusion = None
    if callable(args[0]):
        diffusion, args = args[0], args[1:]
        assert len(args) > 0, 'State variable is required after diffusion function.'
    N.require_gpu()
    x = _on_device(args[0])
    if x.dtype not in _FLOATS:
        raise ValueError(f'State variable dtype must be float16, bfloat16, float32, or float64 '
                         f'for Exponential Euler method, but got {x.dtype}.')
    dt = environ.get_dt()
    drift, jac = _drift_and_vjp(fn, x, args[1:], kwargs)
    x_next = _step(x, drift, jac, dt)
    if diffusion is not None:
        g = diffusion(x, *args[1:], **kwargs)
        g = (g if torch.is_tensor(g) else torch.as_tensor(g)).to(device=x.device, dtype=x.dtype)
        noise = torch.randn(x.shape, device=x.device, dtype=x.dtype)
        x_next = x_next + g * math.sqrt(float(dt)) * noise
    return x_next
