"""Test infrastructure only: ctypes wrapper over the C oracle + torch mirror.

The C source (``oracle/kivi_oracle.c``) restates the reference codec
(src/csrc/kernels/internal/quant_tile.hpp:35-91,
src/csrc/kernels/quantize_kernels.cpp:24-106,
src/csrc/kernels/dequantize_kernels.cpp:17-111) under IEEE fp32.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libkivi_oracle.so")
_lib = None


def build() -> str:
    """Compile ``libkivi_oracle.so`` with the committed Makefile."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "libkivi_oracle.so"],
                   check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    f32p = ctypes.POINTER(ctypes.c_float)
    u8p = ctypes.POINTER(ctypes.c_uint8)
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    lib.kivi_oracle_quantize_groups.argtypes = [f32p, u8p, f32p, f32p, i64, i32]
    lib.kivi_oracle_quantize_groups.restype = None
    lib.kivi_oracle_dequantize_groups.argtypes = [u8p, f32p, f32p, f32p, i64, i32]
    lib.kivi_oracle_dequantize_groups.restype = None
    lib.kivi_oracle_roundtrip_groups.argtypes = [f32p, f32p, i64, i32]
    lib.kivi_oracle_roundtrip_groups.restype = None
    lib.kivi_oracle_count_ties.argtypes = [f32p, i64, i32]
    lib.kivi_oracle_count_ties.restype = i64
    lib.kivi_oracle_num_threads.argtypes = []
    lib.kivi_oracle_num_threads.restype = ctypes.c_int
    lib.kivi_oracle_set_num_threads.argtypes = [ctypes.c_int]
    lib.kivi_oracle_set_num_threads.restype = None
    _lib = lib
    return lib


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _flat_f32(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32)).reshape(-1)


def _check_group(n: int, group_size: int) -> int:
    if group_size <= 0 or group_size % 4:
        raise ValueError(f"group_size must be positive and divisible by 4, got {group_size}")
    if n % group_size:
        raise ValueError(f"{n} elements is not a whole number of groups of {group_size}")
    return n // group_size


def quantize_groups(x, group_size: int):
    """Flat groups of ``group_size`` -> (packed u8 [n*G/4], scales, zeros)."""
    flat = _flat_f32(x)
    n_groups = _check_group(flat.size, group_size)
    packed = np.empty(flat.size // 4, dtype=np.uint8)
    scales = np.empty(n_groups, dtype=np.float32)
    zeros = np.empty(n_groups, dtype=np.float32)
    if n_groups:
        _load().kivi_oracle_quantize_groups(
            _ptr(flat, ctypes.c_float), _ptr(packed, ctypes.c_uint8),
            _ptr(scales, ctypes.c_float), _ptr(zeros, ctypes.c_float),
            n_groups, group_size)
    return packed, scales, zeros


def dequantize_groups(packed, scales, zeros, group_size: int) -> np.ndarray:
    packed = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8)).reshape(-1)
    scales = _flat_f32(scales)
    zeros = _flat_f32(zeros)
    n_groups = scales.size
    if zeros.size != n_groups or packed.size != n_groups * (group_size // 4):
        raise ValueError("packed/scales/zeros sizes disagree")
    out = np.empty(n_groups * group_size, dtype=np.float32)
    if n_groups:
        _load().kivi_oracle_dequantize_groups(
            _ptr(packed, ctypes.c_uint8), _ptr(scales, ctypes.c_float),
            _ptr(zeros, ctypes.c_float), _ptr(out, ctypes.c_float),
            n_groups, group_size)
    return out


def roundtrip_groups(x, group_size: int) -> np.ndarray:
    flat = _flat_f32(x)
    n_groups = _check_group(flat.size, group_size)
    out = np.empty_like(flat)
    if n_groups:
        _load().kivi_oracle_roundtrip_groups(
            _ptr(flat, ctypes.c_float), _ptr(out, ctypes.c_float),
            n_groups, group_size)
    return out


def count_ties(x, group_size: int) -> int:
    flat = _flat_f32(x)
    n_groups = _check_group(flat.size, group_size)
    if not n_groups:
        return 0
    return int(_load().kivi_oracle_count_ties(_ptr(flat, ctypes.c_float),
                                              n_groups, group_size))


def num_threads() -> int:
    return int(_load().kivi_oracle_num_threads())


def set_num_threads(n: int) -> None:
    _load().kivi_oracle_set_num_threads(int(n))


def unpack_codes(packed, group_size: int) -> np.ndarray:
    """Packed bytes -> one 2-bit code per element (element 4j+k = byte j bits 2k)."""
    p = np.asarray(packed, dtype=np.uint8).reshape(-1)
    codes = np.stack([(p >> (2 * k)) & 3 for k in range(4)], axis=-1)
    return codes.reshape(-1).astype(np.uint8)


def mirror_roundtrip(x, group_size: int):
    """The reference's torch mirror of the fused round-trip
    (tests/unit/test_manager_bookkeeping.py:54-66,
    tests/integration/test_roundtrip_kernels.py:21-27).  It rounds half to
    even (torch.round), so it equals the kernel semantics only on inputs with
    no exact .5 quotient; count_ties() finds those."""
    import torch
    t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.asarray(x, np.float32))
    flat = t.reshape(-1, group_size)
    mn = flat.min(dim=1, keepdim=True).values
    mx = flat.max(dim=1, keepdim=True).values
    scale = (mx - mn) / 3.0 + 1e-10
    q = torch.clamp(torch.round((flat - mn) / scale), 0.0, 3.0)
    return (q * scale + mn).reshape(t.shape)
