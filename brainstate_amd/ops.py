"""Operator-level Python API over the C ABI (torch device tensors in, device tensors out).

These are the building blocks the brainstate-compatible layers call; each maps onto one
C entry point of include/brainstate_amd.h and raises ``NativeError`` on failure.
"""
import ctypes

import numpy as np
import torch

from . import _native as N

_WS_CACHE = {}


def _spk_dtype(spk):
    if spk.dtype in (torch.bool, torch.uint8, torch.int8):
        return N.BS_SPK_U8
    if spk.dtype == torch.float32:
        return N.BS_SPK_F32
    raise TypeError(f'spike tensor dtype {spk.dtype} not supported (bool/uint8/float32)')


def _spk_view(spk):
    spk = spk.contiguous()
    if spk.dtype == torch.bool:
        spk = spk.view(torch.uint8)
    return spk


def compact_workspace(n, device):
    """Zero-filled workspace for bs_spike_compact, cached per (device, stream, size)."""
    nbytes = int(N.lib().bs_spike_compact_workspace_size(int(n)))
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = _WS_CACHE.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 4096), dtype=torch.uint8, device=device)
        _WS_CACHE[key] = ws
    return ws


def spike_compact(spk):
    """Ascending indices of nonzero spikes -> (idx int32 [n] (first count valid), count int32 [1])."""
    N.require_gpu()
    spk = _spk_view(spk)
    n = spk.numel()
    dev = spk.device
    idx = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    cnt = torch.empty(1, dtype=torch.int32, device=dev)
    ws = compact_workspace(n, dev)
    N.check(N.lib().bs_spike_compact(N.ptr(spk), _spk_dtype(spk), n, N.ptr(idx), N.ptr(cnt),
                                     N.ptr(ws), N.stream_handle(dev)), 'bs_spike_compact')
    return idx, cnt


def event_scatter(active, n_active, indices, w, n_post, k=None, indptr=None, out=None,
                  accumulate=False):
    """Pre-major event mat-vec over active rows (fixed-num if indptr is None)."""
    dev = indices.device
    n_pre = (indices.shape[0] if indptr is None else indptr.numel() - 1)
    if indptr is None:
        k = indices.shape[1] if indices.dim() == 2 else int(k)
    homo = not torch.is_tensor(w) or w.numel() == 1
    w_homo = float(w) if homo else 0.0
    if out is None:
        out = torch.empty(n_post, dtype=torch.float32, device=dev)
        accumulate = False
    N.check(N.lib().bs_event_scatter_f32(
        N.ptr(active), N.ptr(n_active), int(n_pre), N.ptr(indptr), N.ptr(indices.contiguous()),
        int(k or 0), None if homo else N.ptr(w.contiguous()), w_homo, int(n_post), N.ptr(out),
        1 if accumulate else 0, N.stream_handle(dev)), 'bs_event_scatter_f32')
    return out


def _batch_of(x):
    """(leading shape, batch rows, row length) of a [..., n] operand."""
    lead = tuple(x.shape[:-1])
    return lead, int(np.prod(lead)) if lead else 1, int(x.shape[-1]) if x.dim() else 1


def event_matvec(spk, indices, w, n_post, k=None, indptr=None, out=None, accumulate=False):
    """Event mat-vec straight from the spike vector (one fused compaction + scatter launch);
    ``spk`` [..., n_pre] with leading batch dimensions gives [..., n_post] in one launch."""
    spk = _spk_view(spk)
    dev = indices.device
    lead, batch, n_pre = _batch_of(spk)
    k = _rows(n_pre, indices, k, indptr)
    homo = not torch.is_tensor(w) or w.numel() == 1
    w_homo = float(w) if homo else 0.0
    if out is None:
        out = torch.empty(lead + (n_post,), dtype=torch.float32, device=dev)
        accumulate = False
    args = (N.ptr(indptr), N.ptr(indices.contiguous()), k,
            None if homo else N.ptr(w.contiguous()), w_homo, int(n_post), N.ptr(out),
            1 if accumulate else 0, N.stream_handle(dev))
    if spk.dim() <= 1:
        N.check(N.lib().bs_event_matvec_f32(N.ptr(spk), _spk_dtype(spk), n_pre, *args),
                'bs_event_matvec_f32')
    else:
        for b0 in range(0, batch, 65535):
            nb = min(65535, batch - b0)
            rows = spk.reshape(batch, n_pre)[b0:b0 + nb]
            dst = out.reshape(batch, n_post)[b0:b0 + nb]
            N.check(N.lib().bs_event_matvec_batch_f32(
                N.ptr(rows), _spk_dtype(spk), nb, n_pre, *args[:6], N.ptr(dst), *args[7:]),
                'bs_event_matvec_batch_f32')
    return out


def _rows(n_pre, indices, k, indptr):
    if indptr is None:
        k = indices.shape[1] if indices.dim() == 2 else int(k)
        if indices.shape[0] != n_pre:
            raise ValueError(f'vector of {n_pre} for {indices.shape[0]} pre rows')
    elif indptr.numel() - 1 != n_pre:
        raise ValueError(f'vector of {n_pre} for {indptr.numel() - 1} pre rows')
    return int(k or 0)


def value_matvec(x, indices, w, n_post, k=None, indptr=None, out=None, accumulate=False):
    """Value-weighted sparse mat-vec: out[j] = sum_{i,k: idx[i,k]=j} x[i] * w[i,k] (fp32 x);
    leading batch dimensions of ``x`` are rows of one batched launch."""
    x = x.to(torch.float32).contiguous()
    dev = indices.device
    lead, batch, n_pre = _batch_of(x)
    k = _rows(n_pre, indices, k, indptr)
    homo = not torch.is_tensor(w) or w.numel() == 1
    if out is None:
        out = torch.empty(lead + (n_post,), dtype=torch.float32, device=dev)
        accumulate = False
    wp, wh = (None, float(w)) if homo else (N.ptr(w.contiguous()), 0.0)
    if x.dim() <= 1:
        N.check(N.lib().bs_value_matvec_f32(
            N.ptr(x), n_pre, N.ptr(indptr), N.ptr(indices.contiguous()), k, wp, wh, int(n_post),
            N.ptr(out), 1 if accumulate else 0, N.stream_handle(dev)), 'bs_value_matvec_f32')
    else:
        for b0 in range(0, batch, 65535):
            nb = min(65535, batch - b0)
            N.check(N.lib().bs_value_matvec_batch_f32(
                N.ptr(x.reshape(batch, n_pre)[b0:b0 + nb]), nb, n_pre, N.ptr(indptr),
                N.ptr(indices.contiguous()), k, wp, wh, int(n_post),
                N.ptr(out.reshape(batch, n_post)[b0:b0 + nb]), 1 if accumulate else 0,
                N.stream_handle(dev)), 'bs_value_matvec_batch_f32')
    return out


def event_matvec_vjp(spk, indices, w, n_post, grad_out, k=None, indptr=None, need_spk=True,
                     need_w=True):
    """Reverse mode of event_matvec: (grad_spk [n_pre] or None, grad_w or None); grad_w has
    the shape of the per-synapse weights, or is a 0-d tensor for a homogeneous weight."""
    spk = _spk_view(spk)
    dev = indices.device
    n_pre = spk.numel()
    k = _rows(n_pre, indices, k, indptr)
    homo = not torch.is_tensor(w) or w.numel() == 1
    g = grad_out.to(torch.float32).contiguous()
    gs = torch.empty(n_pre, dtype=torch.float32, device=dev) if need_spk else None
    gw = None
    if need_w:
        gw = torch.empty((), dtype=torch.float32, device=dev) if homo else \
            torch.empty(w.shape, dtype=torch.float32, device=dev)
    N.check(N.lib().bs_event_matvec_vjp_f32(
        N.ptr(spk), _spk_dtype(spk), int(n_pre), N.ptr(indptr), N.ptr(indices.contiguous()), k,
        None if homo else N.ptr(w.contiguous()), float(w) if homo else 0.0, int(n_post),
        N.ptr(g), N.ptr(gs), N.ptr(gw), N.stream_handle(dev)), 'bs_event_matvec_vjp_f32')
    return gs, gw


def event_matvec_vjp_batch(spk, indices, w, n_post, grad_out, k=None, indptr=None,
                           need_spk=True, need_w=True):
    """event_matvec_vjp for spk [B, n_pre] and grad_out [B, n_post] in one launch: grad_spk
    [B, n_pre] (row b as event_matvec_vjp gives it) and grad_w summed over the rows in row
    order (bs_event_matvec_vjp_batch_f32)."""
    spk = _spk_view(spk)
    dev = indices.device
    B, n_pre = int(spk.shape[0]), int(spk.shape[1])
    k = _rows(n_pre, indices, k, indptr)
    homo = not torch.is_tensor(w) or w.numel() == 1
    g = grad_out.to(torch.float32).reshape(B, n_post).contiguous()
    gs = torch.empty(B, n_pre, dtype=torch.float32, device=dev) if need_spk else None
    gw = None
    if need_w:
        gw = torch.empty((), dtype=torch.float32, device=dev) if homo else \
            torch.empty(w.shape, dtype=torch.float32, device=dev)
    N.check(N.lib().bs_event_matvec_vjp_batch_f32(
        N.ptr(spk), _spk_dtype(spk), B, n_pre, N.ptr(indptr), N.ptr(indices.contiguous()), k,
        None if homo else N.ptr(w.contiguous()), float(w) if homo else 0.0, int(n_post),
        N.ptr(g), N.ptr(gs), N.ptr(gw), N.stream_handle(dev)), 'bs_event_matvec_vjp_batch_f32')
    return gs, gw


def event_dense_vjp(spk, W, grad_out, need_spk=True, need_w=True):
    """Reverse mode of event_dense: (grad_spk [B, n_in] or None, grad_W [n_in, n_out] or None),
    the gradients of spk_values @ W."""
    squeeze = spk.dim() == 1
    s2 = _spk_view(spk.reshape(1, -1) if squeeze else spk)
    B, n_in = s2.shape
    n_out = W.shape[1]
    g = grad_out.reshape(B, n_out).to(torch.float32).contiguous()
    gs = torch.empty(B, n_in, dtype=torch.float32, device=W.device) if need_spk else None
    gw = torch.empty(n_in, n_out, dtype=torch.float32, device=W.device) if need_w else None
    N.check(N.lib().bs_event_dense_vjp_f32(
        N.ptr(s2), _spk_dtype(s2), B, n_in, N.ptr(W.contiguous()), n_out, N.ptr(g), N.ptr(gs),
        N.ptr(gw), N.stream_handle(W.device)), 'bs_event_dense_vjp_f32')
    if gs is not None and squeeze:
        gs = gs[0]
    return gs, gw


def spike_pack(spk, bits=None):
    """Spikes -> bitmap int32 [(n + 31) // 32] (bit i % 32 of word i // 32)."""
    spk = _spk_view(spk)
    n = spk.numel()
    if bits is None:
        bits = torch.empty(max((n + 31) // 32, 1), dtype=torch.int32, device=spk.device)
    N.check(N.lib().bs_spike_pack(N.ptr(spk), _spk_dtype(spk), n, N.ptr(bits),
                                  N.stream_handle(spk.device)), 'bs_spike_pack')
    return bits


def event_gather(spk, sell, out=None, bits=None):
    """Post-major deterministic gather; ``sell`` from :func:`build_sell`."""
    spk = _spk_view(spk)
    dev = spk.device
    n_post = sell['n_post']
    if out is None:
        out = torch.empty(n_post, dtype=torch.float32, device=dev)
    bits = spike_pack(spk, bits)
    w = sell.get('w')
    N.check(N.lib().bs_event_gather_f32(
        N.ptr(bits), int(sell['n_pre']), N.ptr(sell['slice_ptr']), N.ptr(sell['pre']), N.ptr(w),
        float(sell.get('w_homo', 0.0)), int(n_post), N.ptr(out), N.stream_handle(dev)),
        'bs_event_gather_f32')
    return out


def build_sell(indptr, indices, n_pre, n_post, w=None, w_homo=0.0, device='cuda'):
    """Host-side SELL-64x4 post-major layout from a pre-major CSR (numpy arrays).

    Incoming synapses of each post are kept in ascending (pre, k) order (a stable sort on
    the target index), so the gather reproduces a sequential pre-major scatter.  Column c of
    lane l in slice s sits at ``slice_ptr[s] + (c // 4) * 256 + l * 4 + c % 4``: a lane's four
    consecutive columns form one 16-byte word (layout contract of ``bs_event_gather_f32``).
    """
    indptr = np.asarray(indptr, dtype=np.int64)
    indices = np.asarray(indices, dtype=np.int64)
    nnz = indices.size
    if nnz and (indices.min() < 0 or indices.max() >= n_post):
        raise ValueError('connectivity index out of range [0, n_post)')
    pre = np.repeat(np.arange(n_pre, dtype=np.int32), np.diff(indptr))
    order = np.argsort(indices, kind='stable')
    tgt_sorted = indices[order]
    counts = np.bincount(indices, minlength=n_post).astype(np.int64)
    n_slices = (n_post + 63) // 64
    pad_counts = np.zeros(n_slices * 64, np.int64)
    pad_counts[:n_post] = counts
    width = (pad_counts.reshape(n_slices, 64).max(axis=1) + 3) // 4 * 4
    slice_ptr = np.zeros(n_slices + 1, np.int64)
    np.cumsum(width * 64, out=slice_ptr[1:])
    total = int(slice_ptr[-1])
    sell_pre = np.full(total, -1, np.int32)
    sell_w = np.zeros(total, np.float32) if w is not None else None
    post_start = np.zeros(n_post + 1, np.int64)
    np.cumsum(counts, out=post_start[1:])
    # rank of each synapse within its post's list
    rank = np.arange(nnz, dtype=np.int64) - post_start[tgt_sorted]
    s = tgt_sorted // 64
    lane = tgt_sorted - s * 64
    pos = slice_ptr[s] + (rank // 4) * 256 + lane * 4 + rank % 4
    sell_pre[pos] = pre[order]
    if w is not None:
        sell_w[pos] = np.asarray(w, np.float32).reshape(-1)[order]
    t = lambda a: torch.from_numpy(a).to(device)
    return dict(n_pre=n_pre, n_post=n_post, slice_ptr=t(slice_ptr), pre=t(sell_pre),
                w=None if sell_w is None else t(sell_w), w_homo=float(w_homo),
                padded=total, nnz=nnz)


def bucket_plan(n_post):
    """(nb, P): the destination buckets and the posts per bucket that ``build_buckets`` lays
    ``n_post`` outputs out in (``bs_bucket_plan``)."""
    P = ctypes.c_int32(0)
    nb = int(N.lib().bs_bucket_plan(int(n_post), ctypes.byref(P)))
    if nb < 0:
        N.check(N.BS_ERR_INVALID, 'bs_bucket_plan')
    return nb, P.value


def build_buckets(indices, n_post, w=None, w_homo=0.0, indptr=None, k=None):
    """Destination-bucketed layout of a fixed-num ([n_pre, k] indices) or CSR connectivity, built
    on the device (layout contract of ``bs_bucket_build``); ``w`` per synapse or None."""
    N.require_gpu()
    dev = indices.device
    idx = indices.contiguous().to(torch.int32)
    if indptr is None:
        if idx.dim() == 2:
            n_pre, k = idx.shape
        else:
            k = int(k)
            n_pre = idx.numel() // k if k > 0 else 0
        ip = None
    else:
        ip = indptr.contiguous().to(device=dev, dtype=torch.int32)
        n_pre = ip.numel() - 1
        k = 0
    nnz = idx.numel()
    nb, P = bucket_plan(n_post)
    seg = torch.empty(max(n_pre * (nb + 1), 1), dtype=torch.int32, device=dev)
    lidx = torch.empty(max(nnz, 1), dtype=torch.int16, device=dev)
    lw = qexp = scratch = None
    if w is not None:
        wt = torch.as_tensor(w, dtype=torch.float32, device=dev).contiguous().reshape(-1)
        lw = torch.empty(max(nnz, 1), dtype=torch.float32, device=dev)
        qexp = torch.zeros(1, dtype=torch.int32, device=dev)
        scratch = torch.empty(int(n_post) + 1, dtype=torch.int32, device=dev)  # W, in-degrees
    opt = lambda t: N.ptr(t) if t is not None else None
    N.check(N.lib().bs_bucket_build(int(n_pre), opt(ip), N.ptr(idx), int(k),
                                    N.ptr(wt) if w is not None else None, int(n_post), nb,
                                    P, N.ptr(seg), N.ptr(lidx), opt(lw), opt(qexp),
                                    opt(scratch), N.stream_handle(dev)), 'bs_bucket_build')
    return dict(n_pre=int(n_pre), n_post=int(n_post), nb=nb, P=P, seg=seg, lidx=lidx,
                w=lw, qexp=qexp, w_homo=float(w_homo))


def _bucket_call_args(L):
    """The layout's fixed arguments of bs_event_bucket_f32 and its workspace size, computed
    once per layout (the tensors they point into live in the layout dict)."""
    opt = lambda t: N.ptr(t) if t is not None else None
    nbytes = int(N.lib().bs_event_bucket_workspace_size(L['n_pre'], L['n_post'], L['nb']))
    rmax = (nbytes - 256) // (4 * L['n_post']) if nbytes > 0 else 1   # row groups at most
    return ((L['n_pre'], L['n_post'], L['nb'], L['P'], N.ptr(L['seg']), N.ptr(L['lidx']),
             opt(L['w']), opt(L['qexp']), L['w_homo']), nbytes,
            (L['seg'], L['lidx'], L['w'], L['qexp']), rmax)


def _bucket_hint(L):
    """The layout's density hint: an int32 in pinned host memory that each step's kernel
    overwrites with its estimate of the row groups the spikes need (0: no step yet)."""
    h = L.get('_hint')
    if h is None:
        t = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        h = L['_hint'] = (t, t.numpy(), ctypes.c_void_p(t.data_ptr()))
    return h


_BUCKET_MODES = {'split': 0, 'single': 1, 'dense': 2}
_DENSE_MAX_ROWS = 8192   # spike rows per row group, at most, for the fixed-grid mode


def bucket_auto_mode(layout):
    """The mode ('single', 'split' or 'dense') that ``event_bucket(mode='auto')`` takes next
    on this layout, from the estimate the previous step left (none yet: 'split').

    One launch when the estimate is one row group; the row groups fixed at their maximum
    when it is more than half of that (on the 100k x 100k, K = 1000 mat-vec the fixed grid took 19.9 us at p = 0.03,
    estimate 23 of 28, where row groups chosen on the device took 23.2 us, and 21.1 against
    17.7 us at p = 0.01, estimate 9); else row groups chosen on the device.  The fixed grid
    also needs short row groups: each of its workgroups sweeps its rows 4,096 at a time, one
    memory round trip and two barriers per sweep, so with few row groups of many rows (a wide
    output: 82 buckets of 1M posts leave 3 row groups of 266,667 rows for 800k spike rows)
    it took 129 - 595 us where row groups chosen on the device took 31 - 425 us (p = 0.0005 -
    0.1); at most 8,192 rows per group."""
    h = int(_bucket_hint(layout)[1][0])
    cached = layout.get('_call')
    rmax = cached[3] if cached is not None else _bucket_call_args(layout)[3]
    if h == 1:
        return 'single'
    short = -(-layout['n_pre'] // max(rmax, 1)) <= _DENSE_MAX_ROWS
    return 'dense' if 2 * h > rmax > 1 and short else 'split'


def event_bucket(spk, layout, out=None, accumulate=False, mode='auto'):
    """``EventArray(spk) @ conn`` on a destination-bucketed layout (``build_buckets``).

    mode 'auto' follows the previous step's estimate of the row groups the spikes need: one
    launch with no partial sums when it was one ('single'), the row groups fixed at their
    maximum when it was more than half of that ('dense'), else row groups chosen on the
    device ('split').  The
    estimate is read without a synchronisation, so it may lag a step or two; every mode gives
    the same bits."""
    spk = _spk_view(spk)
    L = layout
    dev = L['seg'].device
    cached = L.get('_call')
    if cached is None or any(a is not b for a, b in
                             zip(cached[2], (L['seg'], L['lidx'], L['w'], L['qexp']))):
        cached = L['_call'] = _bucket_call_args(L)
    fixed, nbytes = cached[0], cached[1]
    hint = _bucket_hint(L)
    if mode == 'auto':
        m = _BUCKET_MODES[bucket_auto_mode(L)]
    elif mode in _BUCKET_MODES:
        m = _BUCKET_MODES[mode]
    else:
        raise ValueError(f"event_bucket: mode must be 'auto', 'single', 'split' or 'dense', "
                         f"got {mode!r}")
    if out is None:
        out = torch.empty(L['n_post'], dtype=torch.float32, device=dev)
    sh = torch.cuda.current_stream(dev).cuda_stream
    key = ('bucket', dev.index, sh)
    ws = _WS_CACHE.get(key)
    if nbytes > 0 and (ws is None or ws.numel() < nbytes):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _WS_CACHE[key] = ws
    N.check(N.lib().bs_event_bucket_f32(
        N.ptr(spk), _spk_dtype(spk), *fixed, N.ptr(out), 1 if accumulate else 0,
        N.ptr(ws) if nbytes > 0 else None, nbytes, m, hint[2], ctypes.c_void_p(sh)),
        'bs_event_bucket_f32')
    return out


def event_dense(spk, W, float_as_event=True, out=None):
    """spk [B, n_in] (or [n_in]) x W [n_in, n_out] -> [B, n_out]."""
    squeeze = spk.dim() == 1
    s2 = _spk_view(spk.reshape(1, -1) if squeeze else spk)
    B, n_in = s2.shape
    n_out = W.shape[1]
    if out is None:
        out = torch.empty(B, n_out, dtype=torch.float32, device=W.device)
    nbytes = int(N.lib().bs_event_dense_workspace_size(B, n_in, n_out))
    ws = None
    if nbytes > 0:
        # ticket counters lead the workspace: zero on entry, left zero by every call; the
        # bytes after them hold partial sums, so bytes past the previous call's counters
        # are zeroed before a call that needs more counters
        tick = int(N.lib().bs_event_dense_ticket_bytes(B, n_in, n_out))
        key = ('dense', W.device.index, torch.cuda.current_stream(W.device).cuda_stream)
        ws, zero = _WS_CACHE.get(key, (None, 0))
        if ws is None or ws.numel() < nbytes:
            ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=W.device)
            zero = ws.numel()
        if tick > zero:
            ws[zero:tick].zero_()
        _WS_CACHE[key] = (ws, tick)
    N.check(N.lib().bs_event_dense_f32(N.ptr(s2), _spk_dtype(s2), B, n_in, N.ptr(W.contiguous()),
                                       n_out, 1 if float_as_event else 0, N.ptr(out),
                                       N.ptr(ws) if ws is not None else None, nbytes,
                                       N.stream_handle(W.device)), 'bs_event_dense_f32')
    return out[0] if squeeze else out



def dense_digits(n_in):
    """Signed 8-bit digits per weight of the packed EventLinear form (0: n_in not packable)."""
    return int(N.lib().bs_event_dense_digits(int(n_in)))


class _PackedW(dict):
    """``pack_dense``'s result.  ``P['finite']`` is read from the packed buffer's status word
    on first use (one synchronisation), so packing alone does not stop the host."""

    def __missing__(self, key):
        if key != 'finite':
            raise KeyError(key)
        v = int(self['packed'][:4].view(torch.int32).item()) == 0
        self['finite'] = v
        return v


def pack_dense(W):
    """Pack W [n_in, n_out] fp32 for ``event_dense_packed`` (bs_event_dense_pack): per-column
    fixed-point digits in the matrix-core operand order.  Returns a dict with the packed
    buffer and ``finite`` (False when a weight is inf or NaN: the packed product then returns
    NaN everywhere), read from the device on first access (one synchronisation)."""
    W = W.contiguous()
    n_in, n_out = int(W.shape[0]), int(W.shape[1])
    nbytes = int(N.lib().bs_event_dense_packed_bytes(n_in, n_out))
    if nbytes <= 0:
        raise ValueError(f'pack_dense: n_in = {n_in} exceeds the packed form (65536 inputs)')
    buf = torch.empty(nbytes, dtype=torch.uint8, device=W.device)   # 256-byte aligned
    N.check(N.lib().bs_event_dense_pack(N.ptr(W), n_in, n_out, N.ptr(buf), nbytes,
                                        N.stream_handle(W.device)), 'bs_event_dense_pack')
    return _PackedW(packed=buf, n_in=n_in, n_out=n_out, L=dense_digits(n_in))


def event_dense_packed(spk, P, out=None):
    """spk [B, n_in] (or [n_in]; any nonzero value is an event) x the packed W -> [B, n_out]
    fp32: exact fixed-point sums, one rounding (bs_event_dense_packed_f32)."""
    squeeze = spk.dim() == 1
    s2 = _spk_view(spk.reshape(1, -1) if squeeze else spk)
    B, n_in = s2.shape
    if n_in != P['n_in']:
        raise ValueError(f'event_dense_packed: spikes have {n_in} inputs, W has {P["n_in"]}')
    buf = P['packed']
    if out is None:
        out = torch.empty(B, P['n_out'], dtype=torch.float32, device=buf.device)
    N.check(N.lib().bs_event_dense_packed_f32(N.ptr(s2), _spk_dtype(s2), B, n_in, N.ptr(buf),
                                              P['n_out'], N.ptr(out),
                                              N.stream_handle(buf.device)),
            'bs_event_dense_packed_f32')
    return out[0] if squeeze else out


def event_dense_packed_lif_step(spk, P, V, ge, gi, ref, params, inh=False, cur_out=None,
                                spk_out=None):
    """One launch: cur = event_dense_packed(spk, P), then coba_lif_step on the [B, n_out]
    state (flattened or 2-D) with cur as the excitatory (or, ``inh``, inhibitory) input.
    Bit-identical to the two calls; returns spk_out (0/1 bytes) when given, else None."""
    s2 = _spk_view(spk.reshape(1, -1) if spk.dim() == 1 else spk)
    B, n_in = s2.shape
    if n_in != P['n_in']:
        raise ValueError(f'event_dense_packed_lif_step: spikes have {n_in} inputs, W has '
                         f'{P["n_in"]}')
    n = B * P['n_out']
    for name, t, dt in (('V', V, torch.float32), ('ge', ge, torch.float32),
                        ('gi', gi, torch.float32), ('ref', ref, torch.int32)):
        if t.numel() != n or not t.is_contiguous() or t.dtype != dt:
            raise ValueError(f'event_dense_packed_lif_step: {name} must be contiguous {dt} '
                             f'with {n} elements')
    lo, hi = s2.data_ptr(), s2.data_ptr() + s2.numel() * s2.element_size()
    for name, t in (('spk_out', spk_out), ('cur_out', cur_out)):
        if t is not None and t.data_ptr() < hi and lo < t.data_ptr() + t.numel() * t.element_size():
            raise ValueError(f'event_dense_packed_lif_step: {name} overlaps the spike input '
                             f'(double-buffer the spikes of a recurrent step)')
    buf = P['packed']
    N.check(N.lib().bs_event_dense_packed_lif_step(
        N.ptr(s2), _spk_dtype(s2), B, n_in, N.ptr(buf), P['n_out'], 1 if inh else 0, N.ptr(V),
        N.ptr(ge), N.ptr(gi), N.ptr(ref), ctypes_ref(params), N.ptr(cur_out), N.ptr(spk_out),
        N.stream_handle(buf.device)), 'bs_event_dense_packed_lif_step')
    return spk_out

def event_dense_chunks(batch, n_in, n_out):
    """(S, L): the chunk plan that fixes the order of bs_event_dense_f32's additions."""
    L = ctypes.c_int32(0)
    S = int(N.lib().bs_event_dense_chunks(int(batch), int(n_in), int(n_out), ctypes.byref(L)))
    return S, int(L.value)


def conn_fixed_num(seed, n_pre, k, n_post, afferent_ratio=None, device=None):
    """numpy.random.RandomState(seed).randint(0, n_post, (n_pre, k)) drawn on the device
    (int32 [n_pre, k]) and, if ``afferent_ratio`` is given, the next ``random(n_pre) <
    afferent_ratio`` of the same stream (bool [n_pre])."""
    N.require_gpu()
    dev = torch.device('cuda', torch.cuda.current_device()) if device is None else device
    if not 0 <= int(seed) < 2 ** 32:
        raise ValueError('Seed must be between 0 and 2**32 - 1')
    sel_on = afferent_ratio is not None
    nbytes = int(N.lib().bs_conn_fixed_num_workspace_size(int(n_pre), int(k), int(n_post),
                                                          int(sel_on)))
    if nbytes == 0:
        N.check(N.BS_ERR_INVALID, 'bs_conn_fixed_num_workspace_size')
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    idx = torch.empty((int(n_pre), int(k)), dtype=torch.int32, device=dev)
    sel = torch.empty(int(n_pre), dtype=torch.uint8, device=dev) if sel_on else None
    N.check(N.lib().bs_conn_fixed_num(int(seed), int(n_pre), int(k), int(n_post), N.ptr(idx),
                                      float(afferent_ratio) if sel_on else 0.0, N.ptr(sel),
                                      N.ptr(ws), nbytes, N.stream_handle(dev)),
            'bs_conn_fixed_num')
    return idx, (sel.view(torch.bool) if sel_on else None)


def csr_from_selected(indices, selected):
    """(indptr int32 [n_pre + 1], indices int32 [nnz]) of the selected rows of ``indices``."""
    n_pre, k = indices.shape
    dev = indices.device
    sel = selected.contiguous().view(torch.uint8)
    indptr = torch.empty(n_pre + 1, dtype=torch.int32, device=dev)
    s = N.stream_handle(dev)
    N.check(N.lib().bs_csr_from_selected(N.ptr(indices), n_pre, k, N.ptr(sel), N.ptr(indptr),
                                         None, s), 'bs_csr_from_selected')
    nnz = int(indptr[-1].item())
    out = torch.empty(nnz, dtype=torch.int32, device=dev)
    N.check(N.lib().bs_csr_from_selected(N.ptr(indices.contiguous()), n_pre, k, N.ptr(sel),
                                         N.ptr(indptr), N.ptr(out), s), 'bs_csr_from_selected')
    return indptr, out


def conn_fixed_num_unique(seed, n_pre, k, n_post, device=None):
    """k distinct targets per row (int32 [n_pre, k]), Philox4x32-10 keyed by ``seed``."""
    N.require_gpu()
    dev = torch.device('cuda', torch.cuda.current_device()) if device is None else device
    idx = torch.empty((int(n_pre), int(k)), dtype=torch.int32, device=dev)
    N.check(N.lib().bs_conn_fixed_num_unique(int(seed) & (2 ** 64 - 1), int(n_pre), int(k),
                                             int(n_post), N.ptr(idx), N.stream_handle(dev)),
            'bs_conn_fixed_num_unique')
    return idx


def refractory_steps(tau_ref, dt, rule='open'):
    """Steps a neuron is held after its spike step: those k >= 1 with k*dt < tau_ref
    (``rule='open'``, 49 at 5 ms / 0.1 ms) or k*dt <= tau_ref (``'closed'``, 50: the
    ``t - t_last <= tau_ref`` test of BrainPy's LifRef taken on the exact dt grid)."""
    if rule not in ('open', 'closed'):
        raise ValueError(f"ref_rule must be 'open' or 'closed', got {rule!r}")
    q = float(tau_ref) / float(dt)
    n = int(np.ceil(q - 1e-9)) - 1 if rule == 'open' else int(np.floor(q + 1e-9))
    return max(n, 0)


def lif_params(V_rest=-60., V_th=-50., V_reset=-60., tau=20., R=1., tau_ref=5., I_ext=20.,
               E_e=0., E_i=-80., tau_e=5., tau_i=10., dt=0.1, out='coba', scale_e=1.,
               scale_i=1., spk_reset='hard', ref_rule='open', deferred_reset=False):
    """bs_lif_params.  ``out='coba'``: synaptic current g * (E - V); ``out='cuba'``: g * scale
    (brainpy.state CUBA; E_e / E_i unused).  ``spk_reset='soft'``: a spike subtracts
    V_th - V_reset from V instead of setting V_reset.  ``ref_rule``: refractory_steps.
    ``deferred_reset``: the reset is applied at the start of the neuron's next step (a
    spiking neuron keeps V' >= V_th until then; the step reads the previous spikes)."""
    if out not in ('coba', 'cuba'):
        raise ValueError(f"out must be 'coba' or 'cuba', got {out!r}")
    if spk_reset not in ('hard', 'soft'):
        raise ValueError(f"spk_reset must be 'hard' or 'soft', got {spk_reset!r}")
    ref_steps = refractory_steps(tau_ref, dt, ref_rule)
    inv_tau = float(np.float32(1.0) / np.float32(tau))   # fp32 reciprocal of the constant
    return N.LifParams(V_rest, V_th, V_reset, inv_tau, R, I_ext, E_e, E_i, dt,
                       float(np.float32(np.exp(-dt / tau_e))),
                       float(np.float32(np.exp(-dt / tau_i))), ref_steps,
                       1 if out == 'cuba' else 0, scale_e, scale_i,
                       1 if spk_reset == 'soft' else 0, 1 if deferred_reset else 0)


def hh_params(ENa=50., gNa=120., EK=-77., gK=36., EL=-54.387, gL=0.03, C=1.0, V_th=20.,
              I_ext=0., E_e=0., E_i=-80., tau_e=5., tau_i=10., dt=0.05):
    inv_C = float(np.float32(1.0) / np.float32(C))
    return N.HhParams(ENa, gNa, EK, gK, EL, gL, inv_C, V_th, I_ext, E_e, E_i, dt,
                      float(np.float32(np.exp(-dt / tau_e))),
                      float(np.float32(np.exp(-dt / tau_i))))


def _input_array(I_ext, V):
    """A per-neuron external input as a contiguous fp32 tensor of V's size on V's device."""
    if I_ext is None:
        return None
    t = torch.as_tensor(I_ext, dtype=torch.float32, device=V.device)
    return t.expand(V.shape).contiguous() if t.shape != V.shape else t.contiguous()


_LIF_ARRAYS = ('V_rest', 'V_th', 'V_reset', 'inv_tau', 'R', 'ref_steps')


_HH_ARRAYS = ('ENa', 'gNa', 'EK', 'gK', 'EL', 'gL', 'inv_C', 'V_th')


def hh_arrays(V, **arrays):
    """Per-neuron HH parameters for ``coba_hh_step(..., arrays=)`` (any of ENa, gNa, EK, gK,
    EL, gL, inv_C, V_th), fp32 and broadcast to V's shape on V's device."""
    out = {}
    for k, v in arrays.items():
        if k not in _HH_ARRAYS:
            raise ValueError(f'unknown per-neuron HH parameter {k!r}')
        if v is not None:
            t = torch.as_tensor(v, dtype=torch.float32, device=V.device)
            out[k] = torch.broadcast_to(t, V.shape).contiguous()
    return out


def lif_arrays(V, **arrays):
    """Per-neuron LIF parameters for ``coba_lif_step(..., arrays=)``: each given value (any
    of V_rest, V_th, V_reset, inv_tau, R, ref_steps) broadcast to V's shape on V's device
    (ref_steps int32, the others fp32); the tensors stay referenced by the returned dict."""
    out = {}
    for k, v in arrays.items():
        if k not in _LIF_ARRAYS:
            raise ValueError(f'unknown per-neuron LIF parameter {k!r}')
        if v is None:
            continue
        dt = torch.int32 if k == 'ref_steps' else torch.float32
        t = torch.as_tensor(v, dtype=dt, device=V.device)
        out[k] = torch.broadcast_to(t, V.shape).contiguous()
    return out


def coba_lif_step(V, ge, gi, ref, in_e, in_i, params, spk_out=None, I_ext=None, arrays=None,
                  spk_prev=None):
    """One COBA/CUBA-LIF step of every neuron; ``I_ext`` (optional, broadcast to V) is each
    neuron's external input in place of ``params.I_ext``; ``arrays`` (``lif_arrays``) per-neuron
    parameters in place of the scalars (bs_coba_lif_step_arr).  With
    ``params.deferred_reset`` the previous step's spikes (``spk_prev``, or those ``spk_out``
    holds; none when neither is given) are reset first, and the new spikes are returned in a
    new tensor unless ``spk_out`` is given."""
    n = V.numel()
    if params.deferred_reset:
        if spk_out is None:
            spk_out = (torch.zeros(n, dtype=torch.uint8, device=V.device) if spk_prev is None
                       else spk_prev.reshape(-1).to(torch.uint8, copy=True))
        elif spk_prev is not None:
            spk_out.copy_(spk_prev.reshape(-1))
    elif spk_out is None:
        spk_out = torch.empty(n, dtype=torch.uint8, device=V.device)
    arr = _input_array(I_ext, V)
    pa = None
    if arrays:
        pa = N.LifArrays(*[N.ptr(arrays.get(k)) for k in _LIF_ARRAYS])
    N.check(N.lib().bs_coba_lif_step_arr(n, N.ptr(V), N.ptr(ge), N.ptr(gi), N.ptr(ref),
                                         N.ptr(in_e), N.ptr(in_i), N.ptr(arr),
                                         ctypes.byref(pa) if pa is not None else None,
                                         ctypes_ref(params), N.ptr(spk_out),
                                         N.stream_handle(V.device)), 'bs_coba_lif_step')
    return spk_out


def hh_init(V, m, h, n):
    N.check(N.lib().bs_hh_init(V.numel(), N.ptr(V), N.ptr(m), N.ptr(h), N.ptr(n),
                               N.stream_handle(V.device)), 'bs_hh_init')


def coba_hh_step(V, m, h, n, ge, gi, in_e, in_i, params, spk_out=None, I_ext=None,
                 arrays=None):
    """One COBA-HH step of every neuron; ``I_ext`` and ``arrays`` (``hh_arrays``) as in
    ``coba_lif_step`` (bs_coba_hh_step_arr)."""
    if spk_out is None:
        spk_out = torch.empty(V.numel(), dtype=torch.uint8, device=V.device)
    arr = _input_array(I_ext, V)
    pa = N.HhArrays(*[N.ptr(arrays.get(k)) for k in _HH_ARRAYS]) if arrays else None
    N.check(N.lib().bs_coba_hh_step_arr(V.numel(), N.ptr(V), N.ptr(m), N.ptr(h), N.ptr(n),
                                        N.ptr(ge), N.ptr(gi), N.ptr(in_e), N.ptr(in_i),
                                        N.ptr(arr), ctypes.byref(pa) if pa is not None else None,
                                        ctypes_ref(params), N.ptr(spk_out),
                                        N.stream_handle(V.device)), 'bs_coba_hh_step')
    return spk_out


def ctypes_ref(s):
    import ctypes
    return ctypes.byref(s)
