"""The C-ABI library loads and exports every symbol include/brainstate_amd.h declares (CPU)."""
import ctypes
import os
import re

import pytest

from brainstate_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'brainstate_amd.h')


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r'BS_API\s+[\w\s\*]+?\b(bs_\w+)\s*\(', text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ('bs_spike_compact', 'bs_event_scatter_f32', 'bs_event_gather_f32',
              'bs_event_dense_f32', 'bs_coba_lif_step', 'bs_coba_hh_step', 'bs_coba_lif_run',
              'bs_coba_hh_run', 'bs_last_error'):
        assert s in syms


def test_library_exports_every_declared_symbol():
    if not os.path.exists(N.LIB_PATH):
        pytest.skip('library not built (python -m brainstate_amd.build)')
    lib = ctypes.CDLL(N.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    # the binding table covers the header exactly
    assert sorted(N.SIGNATURES) == declared_symbols()


def test_host_only_calls_without_gpu():
    if not os.path.exists(N.LIB_PATH):
        pytest.skip('library not built')
    lib = N.load_library()
    assert lib.bs_version() >= 1
    assert lib.bs_spike_compact_workspace_size(0) == 256
    assert lib.bs_spike_compact_workspace_size(4096) == 256 + 8
    assert lib.bs_spike_compact_workspace_size(4097) == 256 + 16
    assert lib.bs_net_workspace_size(None) == 0 and b'net is NULL' in lib.bs_last_error()
    # argument validation happens before any device work
    rc = lib.bs_spike_compact(None, 7, 10, None, None, None, None)
    assert rc == N.BS_ERR_INVALID
    assert b'dtype' in lib.bs_last_error()
    rc = lib.bs_coba_lif_run(None, None, None, 1, 0, None, None, None, None, None)
    assert rc == N.BS_ERR_INVALID and b'net is NULL' in lib.bs_last_error()


def test_struct_layouts_match_header():
    # field counts/order of the ctypes mirrors (sizes of plain C structs on x86-64)
    assert ctypes.sizeof(N.LifParams) == 12 * 4
    assert ctypes.sizeof(N.HhParams) == 14 * 4
    assert ctypes.sizeof(N.LifState) == 4 * 8
    assert ctypes.sizeof(N.HhState) == 6 * 8
    assert [f[0] for f in N.Net._fields_][:4] == ['n', 'n_exc', 'k_e', 'k_i']
