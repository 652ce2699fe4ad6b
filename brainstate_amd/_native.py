"""ctypes binding of the C ABI in include/brainstate_amd.h.

The HIP library is the only compute path: if ``_lib/libbsamd.so`` is missing or no GPU
is visible, every operator raises.  Tensors are torch device tensors used as plain
device memory; pointers and the current HIP stream are handed to the C ABI.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, '_lib', 'libbsamd.so')

BS_OK, BS_ERR_INVALID, BS_ERR_LAUNCH, BS_ERR_UNSUPPORTED = 0, 1, 2, 3
BS_SPK_U8, BS_SPK_F32 = 0, 1

c_i32 = ctypes.c_int32
c_f32 = ctypes.c_float
c_vp = ctypes.c_void_p
c_size = ctypes.c_size_t


class LifParams(ctypes.Structure):
    _fields_ = [(n, c_f32) for n in ('V_rest', 'V_th', 'V_reset', 'inv_tau', 'R', 'I_ext', 'E_e',
                                       'E_i', 'dt', 'decay_e', 'decay_i')] + [
        ('ref_steps', c_i32), ('cuba', c_i32), ('scale_e', c_f32), ('scale_i', c_f32),
        ('soft_reset', c_i32), ('deferred_reset', c_i32)]


class HhParams(ctypes.Structure):
    _fields_ = [(n, c_f32) for n in ('ENa', 'gNa', 'EK', 'gK', 'EL', 'gL', 'inv_C', 'V_th',
                                       'I_ext', 'E_e', 'E_i', 'dt', 'decay_e', 'decay_i')]


class Net(ctypes.Structure):
    _fields_ = [('n', c_i32), ('n_exc', c_i32), ('k_e', c_i32), ('k_i', c_i32),
                ('idx_e', c_vp), ('w_e', c_vp), ('w_e_homo', c_f32),
                ('idx_i', c_vp), ('w_i', c_vp), ('w_i_homo', c_f32),
                ('spk', c_vp), ('blocks_per_cu', c_i32), ('delay_steps', c_i32),
                ('I_ext', c_vp)]


class LifArrays(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in ('V_rest', 'V_th', 'V_reset', 'inv_tau', 'R', 'ref_steps')]


class HhArrays(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in ('ENa', 'gNa', 'EK', 'gK', 'EL', 'gL', 'inv_C', 'V_th')]


class LifState(ctypes.Structure):
    _fields_ = [('V', c_vp), ('ge', c_vp), ('gi', c_vp), ('ref', c_vp)]


class HhState(ctypes.Structure):
    _fields_ = [('V', c_vp), ('m', c_vp), ('h', c_vp), ('n', c_vp), ('ge', c_vp), ('gi', c_vp)]


# name -> (restype, argtypes); every symbol declared in include/brainstate_amd.h
SIGNATURES = {
    'bs_event_matvec_batch_f32': (ctypes.c_int, [c_vp, c_i32, c_i32, c_i32, c_vp, c_vp, c_i32,
                                                 c_vp, c_f32, c_i32, c_vp, c_i32, c_vp]),
    'bs_value_matvec_batch_f32': (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, c_vp, c_i32, c_vp,
                                                 c_f32, c_i32, c_vp, c_i32, c_vp]),
    'bs_conn_fixed_num_workspace_size': (c_size, [c_i32, c_i32, c_i32, c_i32]),
    'bs_conn_fixed_num': (ctypes.c_int, [ctypes.c_uint32, c_i32, c_i32, c_i32, c_vp,
                                         ctypes.c_double, c_vp, c_vp, c_size, c_vp]),
    'bs_csr_from_selected': (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp]),
    'bs_conn_fixed_num_unique': (ctypes.c_int, [ctypes.c_uint64, c_i32, c_i32, c_i32, c_vp,
                                                c_vp]),
    'bs_delay_write': (ctypes.c_int, [c_vp, c_i32, ctypes.c_int64, c_i32, c_vp, c_vp]),
    'bs_delay_gather': (ctypes.c_int, [c_vp, c_i32, ctypes.c_int64, c_i32, c_i32, c_i32, c_vp,
                                       c_vp, ctypes.c_int64, c_vp, c_vp]),
    'bs_delay_taps_f32': (ctypes.c_int, [c_vp, c_i32, ctypes.c_int64, c_i32, c_vp, c_vp, c_vp,
                                         ctypes.c_int64, c_vp, c_vp]),
    'bs_last_error': (ctypes.c_char_p, []),
    'bs_version': (ctypes.c_int, []),
    'bs_spike_compact_workspace_size': (c_size, [c_i32]),
    'bs_spike_compact': (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp]),
    'bs_spike_compact_noalloc': (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, c_vp, c_vp]),
    'bs_exp_euler_f32': (ctypes.c_int, [ctypes.c_int64, c_vp, c_vp, c_vp, c_f32, c_vp, c_vp]),
    'bs_exp_euler_f64': (ctypes.c_int, [ctypes.c_int64, c_vp, c_vp, c_vp, ctypes.c_double, c_vp,
                                        c_vp]),
    'bs_event_scatter_f32': (ctypes.c_int, [c_vp, c_vp, c_i32, c_vp, c_vp, c_i32, c_vp, c_f32,
                                            c_i32, c_vp, c_i32, c_vp]),
    'bs_event_matvec_f32': (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, c_vp, c_i32, c_vp, c_f32,
                                           c_i32, c_vp, c_i32, c_vp]),
    'bs_value_matvec_f32': (ctypes.c_int, [c_vp, c_i32, c_vp, c_vp, c_i32, c_vp, c_f32, c_i32,
                                           c_vp, c_i32, c_vp]),
    'bs_event_matvec_vjp_f32': (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, c_vp, c_i32, c_vp,
                                               c_f32, c_i32, c_vp, c_vp, c_vp, c_vp]),
    'bs_event_dense_vjp_f32': (ctypes.c_int, [c_vp, c_i32, c_i32, c_i32, c_vp, c_i32, c_vp,
                                              c_vp, c_vp, c_vp]),
    'bs_bucket_plan': (ctypes.c_int, [c_i32, c_vp]),
    'bs_bucket_build': (ctypes.c_int, [c_i32, c_vp, c_vp, c_i32, c_vp, c_i32, c_i32, c_i32, c_vp,
                                       c_vp, c_vp, c_vp, c_vp, c_vp]),
    'bs_event_bucket_workspace_size': (c_size, [c_i32, c_i32, c_i32]),
    'bs_event_bucket_f32': (ctypes.c_int, [c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp,
                                           c_vp, c_vp, c_f32, c_vp, c_i32, c_vp, c_size, c_i32,
                                           c_vp, c_vp]),
    'bs_spike_pack': (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, c_vp]),
    'bs_event_gather_f32': (ctypes.c_int, [c_vp, c_i32, c_vp, c_vp, c_vp, c_f32, c_i32, c_vp,
                                           c_vp]),
    'bs_event_dense_chunks': (ctypes.c_int, [c_i32, c_i32, c_i32, c_vp]),
    'bs_event_dense_workspace_size': (c_size, [c_i32, c_i32, c_i32]),
    'bs_event_dense_ticket_bytes': (c_size, [c_i32, c_i32, c_i32]),
    'bs_event_dense_f32': (ctypes.c_int, [c_vp, c_i32, c_i32, c_i32, c_vp, c_i32, c_i32, c_vp,
                                          c_vp, c_size, c_vp]),
    'bs_event_dense_digits': (c_i32, [c_i32]),
    'bs_event_dense_packed_bytes': (ctypes.c_int64, [c_i32, c_i32]),
    'bs_event_dense_pack': (ctypes.c_int, [c_vp, c_i32, c_i32, c_vp, ctypes.c_int64, c_vp]),
    'bs_event_dense_packed_f32': (ctypes.c_int, [c_vp, c_i32, c_i32, c_i32, c_vp, c_i32, c_vp,
                                                 c_vp]),
    'bs_event_dense_packed_lif_step': (ctypes.c_int, [c_vp, c_i32, c_i32, c_i32, c_vp, c_i32,
                                                      c_i32, c_vp, c_vp, c_vp, c_vp,
                                                      ctypes.POINTER(LifParams), c_vp, c_vp,
                                                      c_vp]),
    'bs_coba_lif_step': (ctypes.c_int, [c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                        ctypes.POINTER(LifParams), c_vp, c_vp]),
    'bs_coba_lif_step_in': (ctypes.c_int, [c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                           ctypes.POINTER(LifParams), c_vp, c_vp]),
    'bs_event_matvec_vjp_batch_f32': (ctypes.c_int, [c_vp, c_i32, c_i32, c_i32, c_vp, c_vp,
                                                     c_i32, c_vp, c_f32, c_i32, c_vp, c_vp,
                                                     c_vp, c_vp]),
    'bs_coba_lif_step_arr': (ctypes.c_int, [c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                            ctypes.POINTER(LifArrays),
                                            ctypes.POINTER(LifParams), c_vp, c_vp]),
    'bs_coba_hh_step_arr': (ctypes.c_int, [c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                           c_vp, c_vp, ctypes.POINTER(HhArrays),
                                           ctypes.POINTER(HhParams), c_vp, c_vp]),
    'bs_hh_init': (ctypes.c_int, [c_i32, c_vp, c_vp, c_vp, c_vp, c_vp]),
    'bs_coba_hh_step_in': (ctypes.c_int, [c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                          c_vp, ctypes.POINTER(HhParams), c_vp, c_vp]),
    'bs_coba_hh_step': (ctypes.c_int, [c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                       ctypes.POINTER(HhParams), c_vp, c_vp]),
    'bs_net_workspace_size': (c_size, [ctypes.POINTER(Net)]),
    'bs_net_prepare': (ctypes.c_int, [ctypes.POINTER(Net), c_vp, c_vp]),
    'bs_coba_lif_run': (ctypes.c_int, [ctypes.POINTER(Net), ctypes.POINTER(LifState),
                                       ctypes.POINTER(LifParams), ctypes.c_int64, c_i32, c_vp,
                                       c_vp, c_vp, c_vp, c_vp]),
    'bs_coba_hh_run': (ctypes.c_int, [ctypes.POINTER(Net), ctypes.POINTER(HhState),
                                      ctypes.POINTER(HhParams), ctypes.c_int64, c_i32, c_vp,
                                      c_vp, c_vp, c_vp, c_vp]),
    'bs_coba_lif_run_inputs': (ctypes.c_int, [ctypes.POINTER(Net), ctypes.POINTER(LifState),
                                              ctypes.POINTER(LifParams), c_vp, ctypes.c_int64,
                                              c_i32, c_vp, c_vp, c_vp, c_vp, c_vp]),
    'bs_coba_hh_run_inputs': (ctypes.c_int, [ctypes.POINTER(Net), ctypes.POINTER(HhState),
                                             ctypes.POINTER(HhParams), c_vp, ctypes.c_int64,
                                             c_i32, c_vp, c_vp, c_vp, c_vp, c_vp]),
    'bs_net_grid_blocks': (ctypes.c_int, [ctypes.POINTER(Net)]),
    'bs_net_error': (ctypes.c_int, [c_vp, c_vp]),
    'bs_net_seed_spikes': (ctypes.c_int, [c_vp, c_vp, ctypes.c_int64, c_vp, c_vp]),
}

_lib = None


class NativeError(RuntimeError):
    pass


def load_library(path=LIB_PATH):
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise NativeError(f'brainstate_amd HIP library not built: {path} missing '
                          f'(run `python -m brainstate_amd.build`)')
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def lib():
    return load_library()


def check(rc, what):
    if rc != BS_OK:
        msg = lib().bs_last_error().decode(errors='replace')
        raise NativeError(f'{what} failed (status {rc}): {msg}')


def require_gpu():
    import torch
    if not torch.cuda.is_available():
        raise NativeError('brainstate_amd needs a ROCm GPU (torch.cuda.is_available() is False)')


def ptr(t):
    """Device pointer of a tensor (None -> NULL).  Tensors wrapped by torch.func transforms
    (the tangents handed to a custom Function's jvp rule) are unwrapped to the tensor that
    holds the storage; the kernels only read such operands."""
    if t is None:
        return None
    try:
        return ctypes.c_void_p(t.data_ptr())
    except RuntimeError:
        from torch._C import _functorch as ft
        while ft.is_functorch_wrapped_tensor(t):
            t = ft.get_unwrapped(t)
        return ctypes.c_void_p(t.data_ptr())


def stream_handle(device=None):
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
