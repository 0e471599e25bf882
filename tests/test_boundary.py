"""CPU tests of the drop-in boundary: the C-ABI library loads and exports every
symbol include/kivi_hip.h declares, and the Python ``_C`` facade validates
arguments exactly like the reference (src/csrc/ops/kv_cache_ops.cpp:19-171,
src/csrc/include/kivi/common.hpp:64-75) without touching a GPU.
"""

import ctypes
import os
import re

import pytest
import torch

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "kivi_hip.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kivi_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared_symbols()
    for required in ("kivi_quantize_keys_per_channel", "kivi_quantize_values_per_token",
                     "kivi_dequantize_keys_per_channel", "kivi_dequantize_values_per_token",
                     "kivi_quant_dequant_roundtrip_keys",
                     "kivi_quant_dequant_roundtrip_values",
                     "kivi_event_record", "kivi_event_wait", "kivi_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from intel_kivi_hybrid_amd import _native
    lib = ctypes.CDLL(_native.LIB_PATH)
    missing = [n for n in _declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # and the Python binding binds exactly the declared set
    assert sorted(_native.SIGNATURES) == _declared_symbols()


def test_abi_version_and_error_string():
    from intel_kivi_hybrid_amd import _native
    lib = _native.load()
    assert lib.kivi_abi_version() == 7
    # invalid arguments are rejected on the host, before any launch
    rc = lib.kivi_quantize_keys_per_channel(None, None, None, None, 4, 32, None)
    assert rc == 1 and "null" in _native.last_error()
    buf = (ctypes.c_float * 8)()
    rc = lib.kivi_quantize_keys_per_channel(ctypes.addressof(buf), ctypes.addressof(buf),
                                            ctypes.addressof(buf), ctypes.addressof(buf),
                                            1, 6, None)
    assert rc == 1 and "divisible by 4, got 6" in _native.last_error()
    rc = lib.kivi_quantize_values_per_token(ctypes.addressof(buf), ctypes.addressof(buf),
                                            ctypes.addressof(buf), ctypes.addressof(buf),
                                            2, 20, 8, None)
    assert rc == 1 and "head_dim must be positive and divisible by group_size" in _native.last_error()


# ----------------------------------------------------------------------------
# Facade validation, message for message (CPU tensors: the device check is the
# last check of check_tensor, so dtype/contiguity errors come first).
# ----------------------------------------------------------------------------
@pytest.fixture(scope="module")
def C():
    from intel_kivi_hybrid_amd import _C
    return _C


def _keys_args(dtype=torch.float32):
    x = torch.zeros(1, 2, 4, 32, dtype=dtype)
    packed = torch.empty(1, 2, 4, 8, dtype=torch.uint8)
    scales = torch.empty(1, 2, 4)
    zeros = torch.empty(1, 2, 4)
    return x, packed, scales, zeros


def test_device_check_message(C):
    x, packed, scales, zeros = _keys_args()
    with pytest.raises(RuntimeError, match=r"^input must be on cuda but got cpu$"):
        C.quantize_keys(x, packed, scales, zeros, 32)


def test_dtype_check_message(monkeypatch, C):
    x, packed, scales, zeros = _keys_args(torch.float16)
    with pytest.raises(RuntimeError, match=r"^input must be Float but got Half$"):
        C.quantize_keys(x, packed, scales, zeros, 32)
    # input passes check_tensor only on the expected device type
    monkeypatch.setattr(C, "_DEVICE_TYPE", "cpu")
    x, _, scales, zeros = _keys_args()
    with pytest.raises(RuntimeError, match=r"^output must be Byte but got Float$"):
        C.quantize_keys(x, torch.empty(1, 2, 4, 8), scales, zeros, 32)


def test_contiguity_check_message(C):
    x, packed, scales, zeros = _keys_args()
    with pytest.raises(RuntimeError, match=r"^input must be contiguous$"):
        C.quantize_keys(x.transpose(2, 3), packed, scales, zeros, 32)


def test_all_twelve_ops_and_event_exist(C):
    names = ["quantize_keys", "quantize_values", "dequantize_keys", "dequantize_values",
             "quant_dequant_roundtrip_keys", "quant_dequant_roundtrip_values"]
    for n in names:
        assert callable(getattr(C, n)) and callable(getattr(C, n + "_async"))
    assert hasattr(C.KiviEvent, "wait")


def test_keyword_names_match_reference(C):
    import inspect
    sig = lambda f: list(inspect.signature(f).parameters)          # noqa: E731
    assert sig(C.quantize_keys) == ["input", "output", "scales", "zeros", "group_size"]
    assert sig(C.quantize_values) == ["input", "output", "scales", "zeros", "head_dim", "group_size"]
    assert sig(C.dequantize_keys) == ["input", "scales", "zeros", "output", "group_size"]
    assert sig(C.dequantize_values) == ["input", "scales", "zeros", "output", "head_dim", "group_size"]
    assert sig(C.quant_dequant_roundtrip_keys) == ["input", "output", "group_size"]
    assert sig(C.quant_dequant_roundtrip_values) == ["input", "output", "head_dim", "group_size"]
    assert sig(C.quantize_keys_async) == sig(C.quantize_keys)


def test_group_size_type_errors(C):
    x, packed, scales, zeros = _keys_args()
    with pytest.raises(TypeError):
        C.quantize_keys(x, packed, scales, zeros, 32.0)


# Size rules need device tensors to get past check_tensor; they are restated
# here against the validators directly, with "meta"-free CPU tensors patched
# through the private validators (same code path the ops call).
def _on_fake_device(monkeypatch, C):
    monkeypatch.setattr(C, "_DEVICE_TYPE", "cpu")


def test_size_rule_messages(monkeypatch, C):
    _on_fake_device(monkeypatch, C)
    x, packed, scales, zeros = _keys_args()
    with pytest.raises(RuntimeError, match=r"group_size must be positive and divisible by 4, got 6"):
        C._validate_quant_keys(x, packed, scales, zeros, 6)
    with pytest.raises(RuntimeError, match=r"zeros size \(3\) must match scales size \(8\)"):
        C._validate_quant_keys(x, packed, scales, torch.empty(3), 32)
    with pytest.raises(RuntimeError, match=r"input size \(256\) must equal num_channels\(8\) \* group_size\(16\) = 128"):
        C._validate_quant_keys(x, packed, scales, zeros, 16)
    with pytest.raises(RuntimeError, match=r"output size \(32\) must equal num_channels\(8\) \* \(group_size/4\) = 64"):
        C._validate_quant_keys(x, torch.empty(32, dtype=torch.uint8), scales, zeros, 32)
    with pytest.raises(RuntimeError, match=r"scales must be non-empty"):
        C._validate_quant_keys(x, packed, torch.empty(0), torch.empty(0), 32)
    v = torch.zeros(2, 3, 8, 64)
    with pytest.raises(RuntimeError, match=r"head_dim must be positive and divisible by group_size"):
        C._validate_quant_values(v, torch.empty(2, 3, 8, 16, dtype=torch.uint8),
                                 torch.empty(96), torch.empty(96), 48, 32)
    with pytest.raises(RuntimeError, match=r"refusing to silently truncate"):
        C._validate_quant_values(torch.zeros(100), torch.empty(25, dtype=torch.uint8),
                                 torch.empty(1), torch.empty(1), 64, 32)
    with pytest.raises(RuntimeError, match=r"round-trip is shape-preserving"):
        C._validate_roundtrip_keys(torch.zeros(64), torch.zeros(32), 32)
    with pytest.raises(RuntimeError, match=r"input must be non-empty"):
        C._validate_roundtrip_values(torch.zeros(0), torch.zeros(0), 64, 32)
    # valid arguments return the launch count the kernels use
    assert C._validate_quant_keys(x, packed, scales, zeros, 32) == 8
    assert C._validate_quant_values(v, torch.empty(2, 3, 8, 16, dtype=torch.uint8),
                                    torch.empty(96), torch.empty(96), 64, 32) == 48
    assert C._validate_dequant_values(torch.empty(2, 3, 8, 16, dtype=torch.uint8),
                                      torch.empty(96), torch.empty(96), v, 64, 32) == 96


def test_store_entry_points_reject_bad_arguments():
    """The store and fused-append entry points validate on the host and
    return an error code with a message, before any launch."""
    from intel_kivi_hybrid_amd import _native
    lib = _native.load()
    buf = (ctypes.c_float * 64)()
    p = ctypes.addressof(buf)
    # append: slot outside the ring, too many tokens, bad dtype codes, a
    # 16-bit ring fed another type
    rc = lib.kivi_store_append(p, p, 0, 0, 0, 0, 1, p, p, 0, 1, 1, 8, 4, 4, None)
    assert rc == 1 and "slot 4 outside [0, 4)" in _native.last_error()
    rc = lib.kivi_store_append(p, p, 0, 0, 0, 0, 5, p, p, 0, 1, 1, 8, 4, 0, None)
    assert rc == 1 and "exceed the ring capacity" in _native.last_error()
    rc = lib.kivi_store_append(p, p, 7, 0, 0, 0, 1, p, p, 0, 1, 1, 8, 4, 0, None)
    assert rc == 1 and "new_dtype 7" in _native.last_error()
    rc = lib.kivi_store_append(p, p, 0, 0, 0, 0, 1, p, p, 1, 1, 1, 8, 4, 0, None)
    assert rc == 1 and "res_dtype 1" in _native.last_error()
    # several layers' appends: per-layer arrays checked entry by entry
    ptrs = (ctypes.c_void_p * 2)(p, p)
    strides = (ctypes.c_int64 * 6)(0, 0, 0, 0, 0, 0)
    slots = (ctypes.c_int32 * 2)(0, 4)
    ap = ctypes.addressof
    assert lib.kivi_store_append_layers(0, None, None, None, 0, 1, None, None, 0, 1, 1, 8, 4,
                                        None, None) == 0
    rc = lib.kivi_store_append_layers(-1, None, None, None, 0, 1, None, None, 0, 1, 1, 8, 4,
                                      None, None)
    assert rc == 1 and "n_layers -1" in _native.last_error()
    rc = lib.kivi_store_append_layers(2, ap(ptrs), None, ap(strides), 0, 1, ap(ptrs), ap(ptrs),
                                      0, 1, 1, 8, 4, ap(slots), None)
    assert rc == 1 and "null layer array" in _native.last_error()
    rc = lib.kivi_store_append_layers(2, ap(ptrs), ap(ptrs), ap(strides), 0, 1, ap(ptrs),
                                      ap(ptrs), 0, 1, 1, 8, 4, ap(slots), None)
    assert rc == 1 and "slot 4 outside [0, 4) (layer 1)" in _native.last_error()
    rc = lib.kivi_store_append_layers(2, ap(ptrs), ap(ptrs), ap(strides), 2, 1, ap(ptrs),
                                      ap(ptrs), 1, 1, 1, 8, 4, ap(slots), None)
    assert rc == 1 and "res_dtype 1" in _native.last_error()
    # flush of more chunks than the run holds
    rc = lib.kivi_store_flush_chunks(p, p, 0, p, p, 0, 0, 0, 8, 3, p, p, p, p, p, p, None, None,
                                     0, 1, 1, 8, 4, 4, 8, 0, 2, 4, 0, 2, None)
    assert rc == 1 and "2 chunks of 4 need 8 tokens, 5 available" in _native.last_error()
    # chunk range beyond the capacity
    rc = lib.kivi_store_flush_chunks(p, p, 0, None, None, 0, 0, 0, 0, 0, p, p, p, p, p, p, None,
                                     None, 0, 1, 1, 8, 4, 4, 8, 0, 8, 2, 1, 2, None)
    assert rc == 1 and "outside capacity 2" in _native.last_error()
    # unknown ring type
    rc = lib.kivi_store_flush_chunks(p, p, 3, None, None, 0, 0, 0, 0, 0, p, p, p, p, p, p, None,
                                     None, 0, 1, 1, 8, 4, 4, 8, 0, 8, 2, 0, 1, None)
    assert rc == 1 and "res_dtype 3" in _native.last_error()
    # fused append needs aligned new-token rows (four elements of the ring's
    # type) and a window holding the token
    rc = lib.kivi_packed_decode_attention_append(p, p + 4, p, 0, 0, p, p, p, p, p, p, p, p, 0,
                                                 p, None, 0, 1, 4, 4, 64, 32, 32, 1, 0, 32, 0, 1,
                                                 ctypes.c_float(0.1), 0, None)
    assert rc == 1 and "16-byte aligned" in _native.last_error()
    rc = lib.kivi_packed_decode_attention_append(p, p + 4, p, 0, 0, p, p, p, p, p, p, p, p, 1,
                                                 p, None, 0, 1, 4, 4, 64, 32, 32, 1, 0, 32, 0, 1,
                                                 ctypes.c_float(0.1), 0, None)
    assert rc == 1 and "8-byte aligned" in _native.last_error()
    rc = lib.kivi_packed_decode_attention_append(p, p, p, 0, 0, p, p, p, p, p, p, p, p, 0, p,
                                                 None, 0, 1, 4, 4, 64, 32, 32, 1, 0, 32, 0, 0,
                                                 ctypes.c_float(0.1), 0, None)
    assert rc == 1 and "must hold the new token" in _native.last_error()
    rc = lib.kivi_packed_decode_attention(p, p, p, p, p, p, p, p, p, 4, p, None, 0, 1, 4, 4,
                                          64, 32, 32, 1, 0, 32, 0, 1, ctypes.c_float(0.1), 0,
                                          None)
    assert rc == 1 and "res_dtype 4" in _native.last_error()
    # several query tokens: causal ones must sit in the window, q_len >= 1
    rc = lib.kivi_packed_attention(p, 3, 1, None, p, p, p, p, p, p, p, p, 0, p, None, 0, 1, 4,
                                   4, 64, 32, 32, 1, 1, 32, 0, 2, ctypes.c_float(0.1), 0, None)
    assert rc == 1 and "3 query tokens needs them in the residual" in _native.last_error()
    rc = lib.kivi_packed_attention(p, 0, 0, None, p, p, p, p, p, p, p, p, 0, p, None, 0, 1, 4,
                                   4, 64, 32, 32, 1, 1, 32, 0, 2, ctypes.c_float(0.1), 0, None)
    assert rc == 1 and "q_len 0 must be positive" in _native.last_error()


def test_noalloc_rejects_oversize_partials_on_host():
    """The allocation-free attention entry point refuses a launch whose split
    partials exceed its static scratch array, on the host, before it touches
    a device (64 rows x 32 heads x 64 splits x (128 + 2) floats = 68 MB >
    8 MiB)."""
    from intel_kivi_hybrid_amd import _native
    lib = _native.load()
    rc = lib.kivi_packed_decode_attention_noalloc(
        None, None, None, None, None, None, None, None, None, 0, None,
        64, 32, 8, 128, 32, 32, 2000, 1000, 128, 0, 0, 0.088, 64, None)
    assert rc == 1
    msg = _native.last_error()
    assert "allocation-free entry point holds at most 8388608" in msg, msg


def test_noalloc_refuses_oversized_split_partials():
    """The allocation-free entry point refuses, before anything runs (so on
    a host without a GPU too), a launch whose split partials exceed its
    static scratch array: an explicit 64-way split at config 4's shape needs
    64 x 8 x 4 rows x 64 splits x (128 + 2) floats = 68 MB > 8 MiB."""
    from intel_kivi_hybrid_amd import _native
    lib = _native.load()
    lib.kivi_clear_error()
    null = ctypes.c_void_p(0)
    rc = lib.kivi_packed_decode_attention_noalloc(
        null, null, null, null, null, null, null, null, null, 0, null,
        64, 32, 8, 128, 32, 32, 300, 252, 128, 0, 128, 0.088, 64, null)
    assert rc == 1                                   # KIVI_ERR_INVALID_ARGUMENT
    msg = _native.last_error()
    assert "split partials" in msg and str(8 << 20) in msg, msg
