"""bs_spike_compact_noalloc (static per-device scratch, no allocation) against
bs_spike_compact (caller workspace): equal index lists and counts, call after call."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def lib():
    import torch
    if not torch.cuda.is_available():
        pytest.fail('GPU tests need a ROCm GPU')
    from brainstate_amd import _native as N
    return N


def _both(N, torch, spk, dtype_code):
    """(count, idx) from the workspace entry point and from the no-alloc one."""
    n = spk.numel()
    dev = spk.device
    stream = N.stream_handle(dev)
    ws = torch.zeros(int(N.lib().bs_spike_compact_workspace_size(n)), dtype=torch.uint8,
                     device=dev)
    out = []
    for noalloc in (False, True):
        idx = torch.full((max(n, 1),), -7, dtype=torch.int32, device=dev)
        cnt = torch.full((1,), -7, dtype=torch.int32, device=dev)
        if noalloc:
            rc = N.lib().bs_spike_compact_noalloc(N.ptr(spk), dtype_code, n, N.ptr(idx),
                                                  N.ptr(cnt), stream)
            N.check(rc, 'bs_spike_compact_noalloc')
        else:
            rc = N.lib().bs_spike_compact(N.ptr(spk), dtype_code, n, N.ptr(idx), N.ptr(cnt),
                                          N.ptr(ws), stream)
            N.check(rc, 'bs_spike_compact')
        torch.cuda.synchronize()
        c = int(cnt.item())
        out.append((c, idx[:c].cpu().numpy()))
    return out


@pytest.mark.parametrize('dtype', ['u8', 'f32'])
def test_noalloc_compaction_equals_workspace_entry(lib, dtype):
    import torch
    N = lib
    # two calls in a row, the second smaller (the scratch keeps the first call's contents),
    # then a larger one again and one tile exactly
    for n, p, seed in [(1_000_003, 0.01, 1), (70_001, 0.3, 2), (4_000_000, 0.002, 3),
                       (4096, 0.5, 4), (1, 1.0, 5)]:
        print('[case] noalloc compaction', dtype, n, p, flush=True)
        m = np.random.RandomState(seed).rand(n) < p
        if dtype == 'u8':
            spk = torch.from_numpy(m.astype(np.uint8)).cuda()
            code = N.BS_SPK_U8
        else:
            spk = torch.from_numpy(np.where(m, np.float32(0.7), np.float32(0))).cuda()
            code = N.BS_SPK_F32
        (ca, ia), (cb, ib) = _both(N, torch, spk, code)
        ref = np.flatnonzero(m).astype(np.int32)
        assert ca == cb == ref.size
        assert np.array_equal(ia, ref) and np.array_equal(ib, ref)


def test_noalloc_compaction_limits(lib):
    import torch
    N = lib
    cnt = torch.full((1,), -1, dtype=torch.int32, device='cuda')
    stream = N.stream_handle(cnt.device)
    assert N.lib().bs_spike_compact_noalloc(None, N.BS_SPK_U8, 0, None, N.ptr(cnt), stream) == 0
    torch.cuda.synchronize()
    assert int(cnt.item()) == 0
    big = (1 << 26) + 1
    rc = N.lib().bs_spike_compact_noalloc(None, N.BS_SPK_U8, big, None, N.ptr(cnt), stream)
    assert rc == N.BS_ERR_INVALID and b'exceeds the maximum' in N.lib().bs_last_error()
