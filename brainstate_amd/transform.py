"""Loop drivers and gradients mirroring brainstate.transform.for_loop / jit / grad.

The reference traces the step function once and runs it as an XLA While loop
(brainstate/transform/_loop_collect_return.py:487-572).  Here each step launches the HIP
kernels directly (no tracing); a network that fits the persistent runner runs whole loops
in one launch via ``brainstate_amd.nn.fuse``.
"""
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


def for_loop(f, *xs, length=None, reverse=False, unroll=1, pbar=None):
    """Call ``f(*x_t)`` for t along the leading axis of ``xs`` and stack the outputs
    (brainstate/transform/_loop_collect_return.py:487-572)."""
    if length is None:
        if not xs:
            raise ValueError('for_loop needs xs or length')
        length = len(xs[0])
    order = range(length - 1, -1, -1) if reverse else range(length)
    outs = [f(*[x[i] for x in xs]) for i in order]
    if reverse:
        outs = outs[::-1]
    return _stack(outs)


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
