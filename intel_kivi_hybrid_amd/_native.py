"""ctypes binding of ``libkivi_hip.so`` (declared in ``include/kivi_hip.h``).

This is the only place that loads the native library.  There is no fallback:
if the library is missing or fails to load, importing the package's ``_C``
raises ``ImportError`` (the reference's single import seam behaves the same
way, src/kivi_sycl/extension/loader.py:8-17).
"""

from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libkivi_hip.so")

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_int = ctypes.c_int
_pvp = ctypes.POINTER(ctypes.c_void_p)

# name -> argtypes; every entry point returns int (status) unless listed in
# _RESTYPES.
SIGNATURES = {
    "kivi_last_error": [],
    "kivi_clear_error": [],
    "kivi_abi_version": [],
    "kivi_stream_synchronize": [_vp],
    "kivi_event_record": [_vp, ctypes.POINTER(_vp)],
    "kivi_event_wait": [_vp],
    "kivi_event_query": [_vp],
    "kivi_event_destroy": [_vp],
    "kivi_quantize_keys_per_channel": [_vp, _vp, _vp, _vp, _i64, _i32, _vp],
    "kivi_quantize_values_per_token": [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _vp],
    "kivi_dequantize_keys_per_channel": [_vp, _vp, _vp, _vp, _i64, _i32, _vp],
    "kivi_dequantize_values_per_token": [_vp, _vp, _vp, _vp, _i64, _i32, _vp],
    "kivi_quant_dequant_roundtrip_keys": [_vp, _vp, _i64, _i32, _vp],
    "kivi_quant_dequant_roundtrip_values": [_vp, _vp, _i64, _i32, _i32, _vp],
    "kivi_quantize_keys_per_channel_ev": [_vp, _vp, _vp, _vp, _i64, _i32, _vp, _pvp],
    "kivi_quantize_values_per_token_ev": [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _vp, _pvp],
    "kivi_dequantize_keys_per_channel_ev": [_vp, _vp, _vp, _vp, _i64, _i32, _vp, _pvp],
    "kivi_dequantize_values_per_token_ev": [_vp, _vp, _vp, _vp, _i64, _i32, _vp, _pvp],
    "kivi_quant_dequant_roundtrip_keys_ev": [_vp, _vp, _i64, _i32, _vp, _pvp],
    "kivi_quant_dequant_roundtrip_values_ev": [_vp, _vp, _i64, _i32, _i32, _vp, _pvp],
    "kivi_store_flush": [_vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp],
    "kivi_store_flush_chunks": [_vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _vp, _vp,
                                _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32,
                                _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp],
    "kivi_store_append": [_vp, _vp, _i32, _i64, _i64, _i64, _i32, _vp, _vp, _i32, _i32, _i32,
                          _i32, _i32, _i32, _vp],
    # host arrays (ctypes arrays or their addresses) for the per-layer fields
    "kivi_store_append_layers": [_i32, _vp, _vp, _vp, _i32, _i32, _vp, _vp, _i32, _i32, _i32,
                                 _i32, _i32, _vp, _vp],
    "kivi_store_code_layout": [_i32, _i32, _i32],
    "kivi_packed_decode_attention_supported": [_i32, _i32, _i32, _i32, _i32],
    "kivi_packed_decode_attention_workspace_size": [_i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                                    _i32, _i32],
    "kivi_packed_decode_attention_append": [_vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp,
                                            _vp, _vp, _vp, _i32, _vp, _vp, ctypes.c_size_t, _i32,
                                            _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                            _i32, _i32, _f32, _i32, _vp],
    "kivi_packed_decode_attention": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp,
                                     _vp, ctypes.c_size_t, _i32, _i32, _i32, _i32, _i32,
                                     _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _vp],
    "kivi_packed_attention_workspace_size": [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                             _i32, _i32],
    "kivi_packed_attention": [_vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32,
                              _vp, _vp, ctypes.c_size_t, _i32, _i32, _i32, _i32, _i32, _i32,
                              _i32, _i32, _i32, _i32, _i32, _f32, _i32, _vp],
    "kivi_packed_attention_masked": [_vp, _i32, _i32, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp,
                                     _vp, _vp, _vp, _i32, _vp, _vp, ctypes.c_size_t, _i32, _i32,
                                     _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
                                     _i32, _vp],
    "kivi_packed_decode_attention_noalloc": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32,
                                             _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                             _i32, _i32, _i32, _i32, _f32, _i32, _vp],
}

_RESTYPES = {
    "kivi_last_error": ctypes.c_char_p,
    "kivi_clear_error": None,
    "kivi_packed_decode_attention_workspace_size": ctypes.c_size_t,
    "kivi_packed_attention_workspace_size": ctypes.c_size_t,
}

_lib = None


def load():
    """Load the library once; raises ImportError when it cannot be loaded."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} (the compiled HIP extension) was not found.\n"
            "Build it in-place with:\n\n"
            "  python -m intel_kivi_hybrid_amd.build\n")
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as exc:
        raise ImportError(f"failed to load {LIB_PATH}: {exc}") from exc
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, _int)
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().kivi_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


class KiviNativeError(RuntimeError):
    """A native entry point returned a non-zero status."""


def check(status: int, what: str) -> None:
    if status != 0:
        raise KiviNativeError(f"{what} failed (status {status}): {last_error()}")
