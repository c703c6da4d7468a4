"""ctypes binding of libkvq_int8.so (the C ABI declared in include/kvq_int8.h).

The library is built in-tree by int8-kvcache_amd/build.py. There is no fallback: if it is missing or
stale, load() raises, so nothing silently runs another implementation.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkvq_int8.so")
ABI_VERSION = 11

_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p
_f64 = ctypes.c_double

# name -> argument types, in the order of include/kvq_int8.h
SIGNATURES = {
    "kvq_quant_cache": [_ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr,
                        _i64, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, _ptr],
    "kvq_quant_q": [_ptr, _i64, _i64, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr],
    "kvq_int8_decode_attention": [_ptr, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _i64, _i64,
                                  _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _ptr, _i64, _i64, _i64, _ptr, _i64,
                                  _ptr, _i64, _f64, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i64, _ptr],
    "kvq_int8_decode_attention_ex": [_ptr, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _i64,
                                     _i64, _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _ptr, _i64, _i64, _i64, _ptr,
                                     _i64, _ptr, _i64, _f64, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i64,
                                     _i64, _i64, _ptr],
    "kvq_int8_decode_attention_noalloc": [_ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64,
                                          _i64, _i64, _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _ptr, _i64, _i64,
                                          _i64, _ptr, _i64, _ptr, _i64, _f64, _i64, _i64, _i64, _i64, _ptr],
    "kvq_noalloc_scratch_bytes": [],
    "kvq_dequant_pages": [_ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _ptr,
                          _i64, _ptr, _ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr],
    "kvq_paged_prefill_attention": [_ptr, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _i64, _i64,
                                    _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _ptr, _i64,
                                    _i64, _f64, _ptr],
    "kvq_int8_prefill_attention": [_ptr, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _i64, _i64,
                                   _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _ptr, _i64,
                                   _i64, _f64, _ptr, _i64, _ptr, _i64, _i64, _ptr],
    "kvq_prefill_rows_per_tile": [],
    "kvq_set_attention_events": [_ptr, _ptr],
    "kvq_stream_read": [_ptr, _i64, _ptr, _i64, _ptr],
    "kvq_mfma_probe": [_ptr, _i64, _ptr, _i64, _ptr],
    "kvq_stream_rw": [_ptr, _i64, _ptr, _i64, _i64, _ptr],
    "kvq_stream_scatter": [_ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64,
                           _i64, _i64, _i64, _ptr],
    "kvq_last_error": [],
    "kvq_abi_version": [],
}

_LIB = None


class NativeError(RuntimeError):
    """Raised when the library rejects a call or the HIP runtime reports a launch error."""


def load():
    """Load (once) and return the ctypes library handle."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise NativeError(f"{LIB_PATH} is not built: run `python int8-kvcache_amd/build.py` "
                              "(or __graft_entry__.build()) first")
        lib = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_char_p if name == "kvq_last_error" else ctypes.c_int
        if lib.kvq_abi_version() != ABI_VERSION:
            raise NativeError(f"{LIB_PATH} has ABI {lib.kvq_abi_version()}, expected {ABI_VERSION}: rebuild it")
        _LIB = lib
    return _LIB


def call(name, *args):
    """Call an entry point; a nonzero status becomes NativeError(kvq_last_error())."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        raise NativeError(f"{name}: {lib.kvq_last_error().decode()}")
