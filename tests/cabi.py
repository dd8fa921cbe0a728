"""ctypes binding of libcrispybits_hip.so for the tests that call the C ABI directly (the
boundary checks of test_abi.py and the allocation-free entry point): every entry point of
include/crispybits_hip.h with its argument types, so integer arguments that are device
addresses pass as 64-bit pointers."""
import ctypes

from crispybits_kernels import _C

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64

SIGS = {
    "cbk_last_error": (ctypes.c_char_p, []),
    "cbk_abi_version": (_I, []),
    "cbk_sm_count": (_I, [_I, ctypes.POINTER(_I)]),
    "cbk_tile_n": (_I, []),
    "cbk_max_rho": (_I, [_I, _I, _I, ctypes.POINTER(_I)]),
    "cbk_decode_plan": (_I, [_I, _L, _L, _I, _L, _L, _L, _I, _I, _I, _I, _I, _I, _I, _P]),
    "cbk_gemv_partial_floats": (_L, [_I, _L, _L, _L, _I, _I]),
    "cbk_packed_gemv": (_I, [_P, _I, _L, _L, _P, _P, _P, _P, _L, _I, _I, _I, _I, _I, _P, _P, _P, _I, _P]),
    "cbk_packed_gemv_noalloc": (_I, [_P, _I, _L, _L, _P, _P, _P, _P, _L, _I, _I, _I, _I, _I, _P, _I, _P]),
    "cbk_fused_gate_up": (_I, [_P, _I, _L, _L, _P, _P, _P, _P, _P, _P, _L, _I, _I, _I, _I, _P, _P, _P, _I, _P]),
    "cbk_fused_qkv": (_I, [_P, _I, _L, _L,
                           _P, _P, _P, _P, _L, _P, _P, _P, _P, _L, _P, _P, _P, _P, _L,
                           _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _P]),
    "cbk_fused_qkv_mixed": (_I, [_P, _I, _L, _L,
                                 _P, _P, _P, _P, _L, _P, _P, _P, _P, _L, _P, _P, _P, _P, _L,
                                 _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _P]),
    "cbk_packed_gemm": (_I, [_P, _I, _L, _L, _P, _P, _P, _P, _L, _I, _I, _I, _I, _P, _I, _P]),
    "cbk_packed_gemm_gate_up": (_I, [_P, _I, _L, _L, _P, _P, _P, _P, _P, _P, _L, _I, _I, _P, _I, _P]),
    "cbk_unpack_codes": (_I, [_P, _L, _L, _I, _P, _I, _P]),
    "cbk_quantize_pack": (_I, [_P, _I, _L, _L, _I, _I, _I, _P, _P, _P, _I, _I, _P]),
    "cbk_timer_start": (_I, [_I]),
    "cbk_timer_stop": (_I, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I), ctypes.POINTER(ctypes.c_double), _I]),
    "cbk_stream_probe": (_I, [_P, _L, _I, _I, _I, _P, _I, _P]),
}

lib = ctypes.CDLL(_C.LIB_PATH)
for _name, (_res, _args) in SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def last_error() -> str:
    return lib.cbk_last_error().decode()
