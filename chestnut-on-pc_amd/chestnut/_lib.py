"""ctypes binding of libchestnut.so (include/chestnut.h).

Nonzero return codes raise RuntimeError with the library's message, the
reference's convention for CUDA status codes (run_pinned2.py:1317-1320).
There is no fallback: without the built library every entry point raises.
"""
import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, 'libchestnut.so')
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(_HERE)), 'include', 'chestnut.h')

_lib = None

c_void_p, c_int, c_long, c_size_t, c_float, c_double, c_char_p = (
    ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_size_t, ctypes.c_float, ctypes.c_double, ctypes.c_char_p)
P = ctypes.POINTER

_SIGS = {
    'ck_last_error': (c_char_p, []),
    'ck_version': (c_int, [P(c_int), P(c_int)]),
    'ck_create': (c_int, [c_char_p, P(c_void_p)]),
    'ck_destroy': (c_int, [c_void_p]),
    'ck_param_count': (c_int, [c_void_p, P(c_int)]),
    'ck_param_info': (c_int, [c_void_p, c_int, ctypes.c_char_p, c_size_t, P(c_size_t), P(c_int)]),
    'ck_upload_param': (c_int, [c_void_p, c_char_p, c_void_p, c_size_t]),
    'ck_output_size': (c_int, [c_void_p, P(c_int)]),
    'ck_output_slices': (c_int, [c_void_p, ctypes.c_char_p, c_size_t]),
    'ck_run_frame': (c_int, [c_void_p, c_void_p, c_void_p, c_void_p]),
    'ck_run_frame_nv12': (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_void_p, c_void_p, c_void_p]),
    'ck_set_graph': (c_int, [c_void_p, c_int]),
    'ck_graph_nodes': (c_int, [c_void_p, P(c_size_t)]),
    'ck_reset': (c_int, [c_void_p]),
    'ck_frame_launch': (c_int, [c_void_p]),
    'ck_synchronize': (c_int, [c_void_p]),
    'ck_stream': (c_int, [c_void_p, P(c_void_p)]),
    'ck_plan_size': (c_int, [c_void_p, P(c_int)]),
    'ck_plan_entry': (c_int, [c_void_p, c_int, ctypes.c_char_p, c_size_t, ctypes.c_char_p, c_size_t,
                              P(c_double), P(c_double)]),
    'ck_kernel_times': (c_int, [c_void_p, P(c_float), c_int]),
    'ck_run_range': (c_int, [c_void_p, c_int, c_int]),
    'ck_time_launches': (c_int, [c_void_p, P(c_int), c_int, c_int, P(c_float)]),
    'ck_time_in_frames': (c_int, [c_void_p, P(c_int), c_int, c_int, P(c_float), P(c_float)]),
    'ck_tensor': (c_int, [c_void_p, c_char_p, P(c_void_p), P(c_size_t)]),
    'ck_state_count': (c_int, [c_void_p, P(c_int)]),
    'ck_decoded_layout': (c_int, [c_void_p, P(c_int), ctypes.c_char_p, c_size_t]),
    'ck_state_info': (c_int, [c_void_p, c_int, ctypes.c_char_p, c_size_t, P(c_size_t), P(c_int)]),
    'ck_read_tensor': (c_int, [c_void_p, c_char_p, c_void_p, c_size_t]),
    'ck_write_tensor': (c_int, [c_void_p, c_char_p, c_void_p, c_size_t]),
    'ck_gemv': (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    'ck_gemm_workspace': (c_int, [c_int, c_int, c_int, c_int, P(c_int), P(c_int), P(c_size_t)]),
    'ck_gemm': (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_long, c_long, c_long,
                        c_int, c_int, c_int, c_void_p, c_size_t, c_void_p]),
    'ck_gemm_noalloc': (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_long, c_long, c_long,
                                c_int, c_int, c_int, c_void_p]),
    'ck_gemm_epi': (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_long, c_long, c_long,
                            c_int, c_int, c_int, c_void_p, c_size_t, c_void_p]),
    'ck_wmma_rdna4': (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    'ck_mfma_kat': (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    'ck_pack_yuv': (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p]),
    'ck_frames_to_tensor': (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p]),
    'ck_img_gather': (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p, c_void_p]),
    'ck_state_hashes': (c_int, [c_void_p, c_void_p, c_int]),
    'ck_time_launch_chain': (c_int, [c_int, c_int, c_int, c_int, P(c_float), c_void_p]),
    'ck_time_operand_stream': (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, P(c_float), c_void_p]),
    'ck_warp_nv12': (c_int, [c_void_p, c_void_p, c_size_t, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                             c_int, c_int, c_void_p, c_void_p]),
    'ck_attention': (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    'ck_layernorm': (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_float, c_void_p]),
}


def header_functions(path=HEADER_PATH):
    """Names of every function include/chestnut.h declares."""
    src = open(path).read()
    src = re.sub(r'/\*.*?\*/', '', src, flags=re.S)
    return sorted(set(re.findall(r'\b(ck_\w+)\s*\(', src)))


def lib():
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f'{LIB_PATH} is not built: run chestnut-on-pc_amd/build.py '
                               '(or __graft_entry__.build()) first')
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise RuntimeError(lib().ck_last_error().decode(errors='replace'))
    return rc


def call(name, *args):
    return check(getattr(lib(), name)(*args))
