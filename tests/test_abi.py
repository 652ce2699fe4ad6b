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
    # one 8-byte status word per tile of 16,384 spikes after a 256-byte header
    assert lib.bs_spike_compact_workspace_size(16384) == 256 + 8
    assert lib.bs_spike_compact_workspace_size(16385) == 256 + 16
    assert lib.bs_net_workspace_size(None) == 0 and b'net is NULL' in lib.bs_last_error()
    # argument validation happens before any device work
    rc = lib.bs_spike_compact(None, 7, 10, None, None, None, None)
    assert rc == N.BS_ERR_INVALID
    assert b'dtype' in lib.bs_last_error()
    rc = lib.bs_coba_lif_run(None, None, None, 1, 0, None, None, None, None, None)
    assert rc == N.BS_ERR_INVALID and b'net is NULL' in lib.bs_last_error()


def test_event_dense_chunk_plan_host_only():
    """The chunk plan of bs_event_dense_f32 is a function of the shape only (no device)."""
    if not os.path.exists(N.LIB_PATH):
        pytest.skip('library not built')
    lib = N.load_library()
    L = ctypes.c_int32(0)
    # config [4]: 32 column tiles of 128 x 1 batch group -> 8 chunks of 512 rows
    assert lib.bs_event_dense_chunks(64, 4096, 4096, ctypes.byref(L)) == 8 and L.value == 512
    # few inputs: one chunk (plain ascending sum), no workspace
    assert lib.bs_event_dense_chunks(64, 200, 256, ctypes.byref(L)) == 1 and L.value == 256
    assert lib.bs_event_dense_workspace_size(64, 200, 256) == 0
    # at most 8 chunks of >= 256 rows; a wide output keeps one chunk
    assert lib.bs_event_dense_chunks(1, 40000, 64, ctypes.byref(L)) == 8 and L.value == 5056
    assert lib.bs_event_dense_chunks(64, 512, 256, ctypes.byref(L)) == 2 and L.value == 256
    assert lib.bs_event_dense_chunks(64, 4096, 1 << 16, ctypes.byref(L)) == 1
    for b, ni, no in ((64, 4096, 4096), (3, 2500, 66), (130, 1000, 70), (1, 40000, 64)):
        S = lib.bs_event_dense_chunks(b, ni, no, ctypes.byref(L))
        assert (S - 1) * L.value < ni <= S * L.value and L.value % 64 == 0
        tiles, groups = -(-no // 128), -(-b // 64)
        ws = lib.bs_event_dense_workspace_size(b, ni, no)
        tick = lib.bs_event_dense_ticket_bytes(b, ni, no)
        if S == 1:
            assert ws == 0 and tick == 0
        else:
            assert tick == -(-(tiles * groups * 4) // 256) * 256
            assert ws == tick + S * b * no * 4
    # a chunked shape without its workspace is refused before any device work
    rc = lib.bs_event_dense_f32(ctypes.c_void_p(16), 0, 64, 4096, ctypes.c_void_p(16), 4096, 1,
                                ctypes.c_void_p(16), None, 0, None)
    assert rc == N.BS_ERR_INVALID and b'workspace' in lib.bs_last_error()



def test_event_dense_packed_sizes_host_only():
    """Digits per weight and the packed size (header, column maxima, 1 KiB digit blocks per
    (16-column tile, 64-input block, digit)) are host-side functions of the shape; argument
    checks fail before any device work."""
    if not os.path.exists(N.LIB_PATH):
        pytest.skip('library not built')
    from oracle import event
    lib = N.load_library()
    for n in (0, 1, 64, 65, 4096, 16384, 16385, 65536, 65537, -3):
        assert lib.bs_event_dense_digits(n) == event.dense_digits(n)
    for n_in, n_out in [(4096, 4096), (1, 1), (100, 33), (65536, 17), (0, 5)]:
        L = event.dense_digits(n_in)
        kb, nt = -(-n_in // 64), -(-n_out // 16)
        kb = -(-kb // 8) * 8        # whole pipeline stages of the 4 waves
        bits = -(-(nt * 16 * 4) // 256) * 256
        assert lib.bs_event_dense_packed_bytes(n_in, n_out) == 256 + bits + nt * kb * L * 1024
    assert lib.bs_event_dense_packed_bytes(65537, 4) == 0
    assert lib.bs_event_dense_packed_bytes(4, -1) == 0
    rc = lib.bs_event_dense_pack(None, 70000, 4, None, 0, None)
    assert rc == N.BS_ERR_INVALID and b'exceeds' in lib.bs_last_error()
    rc = lib.bs_event_dense_packed_f32(None, 0, 1, 64, None, 16, None, None)
    assert rc == N.BS_ERR_INVALID and b'aligned' in lib.bs_last_error()


def test_struct_layouts_match_header():
    # field counts/order of the ctypes mirrors (sizes of plain C structs on x86-64)
    assert ctypes.sizeof(N.LifParams) == 17 * 4
    assert [f[0] for f in N.LifParams._fields_][11:] == ['ref_steps', 'cuba', 'scale_e',
                                                         'scale_i', 'soft_reset',
                                                         'deferred_reset']
    assert ctypes.sizeof(N.HhParams) == 14 * 4
    assert ctypes.sizeof(N.LifState) == 4 * 8
    assert ctypes.sizeof(N.HhState) == 6 * 8
    assert [f[0] for f in N.Net._fields_][:4] == ['n', 'n_exc', 'k_e', 'k_i']


def test_lif_params_offsets_match_the_compiled_header(tmp_path):
    """The header compiled by the host compiler puts bs_lif_params' fields where the ctypes
    mirror reads them."""
    import shutil
    import subprocess
    cc = shutil.which('gcc')
    if cc is None:
        pytest.skip('no host C compiler')
    src = tmp_path / 'off.c'
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "brainstate_amd.h"\n'
                   'int main(void) { printf("%zu %zu %zu %zu %zu %zu %zu\\n", '
                   'sizeof(bs_lif_params), offsetof(bs_lif_params, ref_steps), '
                   'offsetof(bs_lif_params, cuba), offsetof(bs_lif_params, scale_e), '
                   'offsetof(bs_lif_params, scale_i), offsetof(bs_lif_params, soft_reset), '
                   'offsetof(bs_lif_params, deferred_reset)); '
                   'return 0; }\n')
    exe = tmp_path / 'off'
    subprocess.run([cc, '-I', os.path.join(ROOT, 'include'), str(src), '-o', str(exe)],
                   check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    L = N.LifParams
    assert got == [ctypes.sizeof(L), L.ref_steps.offset, L.cuba.offset, L.scale_e.offset,
                   L.scale_i.offset, L.soft_reset.offset, L.deferred_reset.offset]
