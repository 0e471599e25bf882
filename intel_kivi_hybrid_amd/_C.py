"""``_C`` -- the drop-in for the reference's compiled module ``kivi_sycl._C``.

Same twelve functions, keyword names, argument meaning and error behaviour as
the reference binding (src/csrc/bindings/pybind_module.cpp:9-82): the caller
allocates every output, the ops write in place, the blocking ops return
``None`` after the device work has finished and the ``*_async`` ops return a
:class:`KiviEvent`.  Validation follows src/csrc/ops/kv_cache_ops.cpp:19-171
message for message and raises ``RuntimeError`` (what ``TORCH_CHECK`` raises
in Python); the device check expects ROCm-torch's ``cuda`` device type where
the reference expected ``xpu`` (src/csrc/include/kivi/common.hpp:64-75).

Work is launched on ``torch.cuda.current_stream()`` of the tensors' device,
through the C ABI of ``libkivi_hip.so``; nothing here computes on the host.
"""

from __future__ import annotations

import ctypes
import functools

import torch

from . import _native
from ._device import device_index, on_device, stream_handle

_lib = _native.load()

__all__ = [
    "KiviEvent",
    "quantize_keys", "quantize_values", "dequantize_keys", "dequantize_values",
    "quant_dequant_roundtrip_keys", "quant_dequant_roundtrip_values",
    "quantize_keys_async", "quantize_values_async", "dequantize_keys_async",
    "dequantize_values_async", "quant_dequant_roundtrip_keys_async",
    "quant_dequant_roundtrip_values_async", "set_lazy_events",
]

_DEVICE_TYPE = "cuda"   # ROCm torch reports HIP devices as "cuda"

# torch::toString(ScalarType) spellings used in the reference's messages.
_DTYPE_NAMES = {
    torch.float32: "Float", torch.float64: "Double", torch.float16: "Half",
    torch.bfloat16: "BFloat16", torch.uint8: "Byte", torch.int8: "Char",
    torch.int16: "Short", torch.int32: "Int", torch.int64: "Long",
    torch.bool: "Bool",
}


def _dtype_name(dt) -> str:
    return _DTYPE_NAMES.get(dt, str(dt).replace("torch.", ""))


def _fail(*parts) -> None:
    raise RuntimeError("".join(str(p) for p in parts))


def _check(cond: bool, *parts) -> None:
    if not cond:
        _fail(*parts)


def _check_int(value, name: str) -> int:
    if isinstance(value, bool) or not isinstance(value, int):
        raise TypeError(f"{name} must be an int, got {type(value).__name__}")
    if not -(1 << 31) <= value < (1 << 31):
        raise TypeError(f"{name} does not fit in a C int: {value}")
    return value


def _check_tensor(t, name: str, dtype) -> None:
    """common.hpp:64-75: contiguous, exact dtype, device type."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    _check(t.is_contiguous(), name, " must be contiguous")
    _check(t.dtype == dtype, name, " must be ", _dtype_name(dtype), " but got ",
           _dtype_name(t.dtype))
    _check(t.device.type == _DEVICE_TYPE, name, " must be on ", _DEVICE_TYPE,
           " but got ", t.device.type)


def _check_same_device(*tensors) -> torch.device:
    dev = tensors[0].device
    for t in tensors[1:]:
        _check(t.device == dev, "all tensors must be on the same device, got ",
               dev, " and ", t.device)
    return dev


# --------------------------------------------------------------------------
# Validation: kv_cache_ops.cpp:19-171.  Each returns the count the kernel
# launch needs.
# --------------------------------------------------------------------------
def _validate_quant_keys(input, output, scales, zeros, group_size) -> int:
    _check_tensor(input, "input", torch.float32)
    _check_tensor(output, "output", torch.uint8)
    _check_tensor(scales, "scales", torch.float32)
    _check_tensor(zeros, "zeros", torch.float32)
    _check(group_size > 0 and group_size % 4 == 0,
           "group_size must be positive and divisible by 4, got ", group_size)
    n = scales.numel()
    _check(n > 0, "scales must be non-empty")
    _check(zeros.numel() == n, "zeros size (", zeros.numel(),
           ") must match scales size (", n, ")")
    _check(input.numel() == n * group_size, "input size (", input.numel(),
           ") must equal num_channels(", n, ") * group_size(", group_size, ") = ",
           n * group_size)
    _check(output.numel() == n * (group_size // 4), "output size (", output.numel(),
           ") must equal num_channels(", n, ") * (group_size/4) = ",
           n * (group_size // 4))
    return n


def _validate_quant_values(input, output, scales, zeros, head_dim, group_size) -> int:
    _check_tensor(input, "input", torch.float32)
    _check_tensor(output, "output", torch.uint8)
    _check_tensor(scales, "scales", torch.float32)
    _check_tensor(zeros, "zeros", torch.float32)
    _check(group_size > 0 and group_size % 4 == 0,
           "group_size must be positive and divisible by 4")
    _check(head_dim > 0 and head_dim % group_size == 0,
           "head_dim must be positive and divisible by group_size")
    _check(input.numel() % head_dim == 0, "input.numel() (", input.numel(),
           ") must be divisible by head_dim (", head_dim,
           ") — refusing to silently truncate trailing elements")
    n_tok = input.numel() // head_dim
    gpt = head_dim // group_size
    _check(n_tok > 0, "input must be non-empty")
    _check(scales.numel() == n_tok * gpt, "scales size (", scales.numel(),
           ") must equal num_tokens(", n_tok, ") * groups_per_token(", gpt, ")")
    _check(zeros.numel() == scales.numel(), "zeros size (", zeros.numel(),
           ") must match scales size (", scales.numel(), ")")
    _check(output.numel() == n_tok * (head_dim // 4), "output size (", output.numel(),
           ") must equal num_tokens(", n_tok, ") * (head_dim/4) = ",
           n_tok * (head_dim // 4))
    return n_tok


def _validate_dequant_keys(input, scales, zeros, output, group_size) -> int:
    _check_tensor(input, "input", torch.uint8)
    _check_tensor(scales, "scales", torch.float32)
    _check_tensor(zeros, "zeros", torch.float32)
    _check_tensor(output, "output", torch.float32)
    _check(group_size > 0 and group_size % 4 == 0,
           "group_size must be positive and divisible by 4, got ", group_size)
    n = scales.numel()
    _check(n > 0, "scales must be non-empty")
    _check(zeros.numel() == n, "zeros size (", zeros.numel(),
           ") must match scales size (", n, ")")
    _check(input.numel() == n * (group_size // 4), "input (packed) size (", input.numel(),
           ") must equal num_channels(", n, ") * (group_size/4) = ", n * (group_size // 4))
    _check(output.numel() == n * group_size, "output size (", output.numel(),
           ") must equal num_channels(", n, ") * group_size = ", n * group_size)
    return n


def _validate_dequant_values(input, scales, zeros, output, head_dim, group_size) -> int:
    _check_tensor(input, "input", torch.uint8)
    _check_tensor(scales, "scales", torch.float32)
    _check_tensor(zeros, "zeros", torch.float32)
    _check_tensor(output, "output", torch.float32)
    _check(group_size > 0 and group_size % 4 == 0,
           "group_size must be positive and divisible by 4, got ", group_size)
    _check(head_dim > 0 and head_dim % group_size == 0,
           "head_dim must be positive and divisible by group_size")
    n = scales.numel()
    _check(n > 0, "scales must be non-empty")
    _check(zeros.numel() == n, "zeros size (", zeros.numel(),
           ") must match scales size (", n, ")")
    _check(input.numel() == n * (group_size // 4), "input (packed) size (", input.numel(),
           ") must equal num_groups(", n, ") * (group_size/4) = ", n * (group_size // 4))
    _check(output.numel() == n * group_size, "output size (", output.numel(),
           ") must equal num_groups(", n, ") * group_size = ", n * group_size)
    return n


def _validate_roundtrip_keys(input, output, group_size) -> int:
    _check_tensor(input, "input", torch.float32)
    _check_tensor(output, "output", torch.float32)
    _check(group_size > 0 and group_size % 4 == 0,
           "group_size must be positive and divisible by 4, got ", group_size)
    _check(input.numel() % group_size == 0, "input.numel() (", input.numel(),
           ") must be divisible by group_size (", group_size, ")")
    _check(output.numel() == input.numel(), "output size (", output.numel(),
           ") must equal input size (", input.numel(),
           ") — round-trip is shape-preserving")
    n = input.numel() // group_size
    _check(n > 0, "input must be non-empty")
    return n


def _validate_roundtrip_values(input, output, head_dim, group_size) -> int:
    _check_tensor(input, "input", torch.float32)
    _check_tensor(output, "output", torch.float32)
    _check(group_size > 0 and group_size % 4 == 0,
           "group_size must be positive and divisible by 4")
    _check(head_dim > 0 and head_dim % group_size == 0,
           "head_dim must be positive and divisible by group_size")
    _check(input.numel() % head_dim == 0, "input.numel() (", input.numel(),
           ") must be divisible by head_dim (", head_dim, ")")
    _check(output.numel() == input.numel(), "output size (", output.numel(),
           ") must equal input size (", input.numel(),
           ") — round-trip is shape-preserving")
    n = input.numel() // head_dim
    _check(n > 0, "input must be non-empty")
    return n


# --------------------------------------------------------------------------
# Launch plumbing.
# --------------------------------------------------------------------------
def _stream_of(device: torch.device) -> int:
    return stream_handle(device)


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


class KiviEvent:
    """Handle for work submitted by a ``*_async`` op (event.hpp:16-31).

    ``wait()`` blocks until the work completes and raises ``RuntimeError`` on
    a device-side error; ``query()`` tells, without blocking, whether it has.
    As in the reference, where the event wraps the submitted kernel's own
    ``sycl::event`` (kv_cache_ops.cpp:245-303), the HIP event is the
    completion event of the op's own kernel launch (hipExtLaunchKernel), so
    ``wait()`` and ``query()`` cover that op alone, whatever is queued behind
    it later, and no marker sits between it and the next kernel.

    Lazy recording is opt-in (:func:`set_lazy_events`): the event is then
    recorded (as a marker) at the first ``wait()`` or ``query()``, which
    covers the op and any work queued on the same stream after it.  The op's
    tensors and its stream are kept alive until the event is released."""

    __slots__ = ("_device", "_stream", "_ev", "_keep", "_done")

    def __init__(self, device: torch.device, stream: "torch.cuda.Stream", keep=()):
        self._device = device
        self._stream = stream
        self._ev = None
        self._keep = keep
        self._done = False

    def _record(self) -> None:
        if self._ev is None:
            ev = ctypes.c_void_p()
            with torch.cuda.device(self._device):
                _native.check(_lib.kivi_event_record(ctypes.c_void_p(self._stream.cuda_stream),
                                                     ctypes.byref(ev)), "kivi_event_record")
            self._ev = ev

    def _release(self) -> None:
        ev, self._ev = self._ev, None
        if ev is not None:
            _lib.kivi_event_destroy(ev)
        self._keep = ()
        self._stream = None
        self._done = True

    def wait(self) -> None:
        if self._done:
            return
        self._record()
        try:
            _native.check(_lib.kivi_event_wait(self._ev), "KiviEvent.wait")
        finally:
            self._release()

    def query(self) -> bool:
        """True once the work has completed (non-blocking)."""
        if self._done:
            return True
        self._record()
        rc = _lib.kivi_event_query(self._ev)
        if rc < 0:
            _native.check(-rc, "KiviEvent.query")
        if rc == 1:
            self._release()
            return True
        return False

    def __del__(self):
        ev = getattr(self, "_ev", None)
        if ev is not None and _lib is not None:
            try:
                _lib.kivi_event_destroy(ev)
            except Exception:   # interpreter shutdown
                pass


def _run(device: torch.device, blocking: bool, what: str, fn, *args, keep=()):
    """Runs the C-ABI op ``fn`` on the device's current stream.  Blocking:
    synchronise the stream.  Async (per-op events): the op's ``_ev`` entry
    point, whose event is the completion event of the op's own kernel launch
    (no marker queued behind it).  Async with lazy events: the plain entry
    point, the event recorded at first use."""
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device)
        sp = ctypes.c_void_p(stream.cuda_stream)
        if not blocking and not _lazy_events:
            handle = ctypes.c_void_p()
            _native.check(getattr(_lib, fn.__name__ + "_ev")(*args, sp, ctypes.byref(handle)),
                          what)
            ev = KiviEvent(device, stream, keep)
            ev._ev = handle
            return ev
        _native.check(fn(*args, sp), what)
        if blocking:
            _native.check(_lib.kivi_stream_synchronize(sp), what)
            return None
        return KiviEvent(device, stream, keep)


_lazy_events = False


def set_lazy_events(lazy: bool) -> bool:
    """Chooses the ``*_async`` ops' :class:`KiviEvent`: the completion event
    of the op's own kernel launch (the default, the reference's per-op
    semantics) or, with ``lazy=True``, a marker recorded at the event's first
    ``wait()``/``query()``.  Returns the previous setting.  Not part of the
    reference's API."""
    global _lazy_events
    prev, _lazy_events = _lazy_events, bool(lazy)
    return prev


# --------------------------------------------------------------------------
# The twelve ops (pybind_module.cpp:18-81).
# --------------------------------------------------------------------------
def _quantize_keys(input, output, scales, zeros, group_size, blocking):
    group_size = _check_int(group_size, "group_size")
    n = _validate_quant_keys(input, output, scales, zeros, group_size)
    dev = _check_same_device(input, output, scales, zeros)
    return _run(dev, blocking, "quantize_keys", _lib.kivi_quantize_keys_per_channel,
                _ptr(input), _ptr(output), _ptr(scales), _ptr(zeros), n, group_size,
                keep=(input, output, scales, zeros))


def _quantize_values(input, output, scales, zeros, head_dim, group_size, blocking):
    head_dim = _check_int(head_dim, "head_dim")
    group_size = _check_int(group_size, "group_size")
    n_tok = _validate_quant_values(input, output, scales, zeros, head_dim, group_size)
    dev = _check_same_device(input, output, scales, zeros)
    return _run(dev, blocking, "quantize_values", _lib.kivi_quantize_values_per_token,
                _ptr(input), _ptr(output), _ptr(scales), _ptr(zeros), n_tok, head_dim,
                group_size, keep=(input, output, scales, zeros))


def _dequantize_keys(input, scales, zeros, output, group_size, blocking):
    group_size = _check_int(group_size, "group_size")
    n = _validate_dequant_keys(input, scales, zeros, output, group_size)
    dev = _check_same_device(input, scales, zeros, output)
    return _run(dev, blocking, "dequantize_keys", _lib.kivi_dequantize_keys_per_channel,
                _ptr(input), _ptr(scales), _ptr(zeros), _ptr(output), n, group_size,
                keep=(input, scales, zeros, output))


def _dequantize_values(input, scales, zeros, output, head_dim, group_size, blocking):
    head_dim = _check_int(head_dim, "head_dim")
    group_size = _check_int(group_size, "group_size")
    n = _validate_dequant_values(input, scales, zeros, output, head_dim, group_size)
    dev = _check_same_device(input, scales, zeros, output)
    return _run(dev, blocking, "dequantize_values", _lib.kivi_dequantize_values_per_token,
                _ptr(input), _ptr(scales), _ptr(zeros), _ptr(output), n, group_size,
                keep=(input, scales, zeros, output))


def _roundtrip_keys(input, output, group_size, blocking):
    group_size = _check_int(group_size, "group_size")
    n = _validate_roundtrip_keys(input, output, group_size)
    dev = _check_same_device(input, output)
    return _run(dev, blocking, "quant_dequant_roundtrip_keys",
                _lib.kivi_quant_dequant_roundtrip_keys, _ptr(input), _ptr(output), n,
                group_size, keep=(input, output))


def _roundtrip_values(input, output, head_dim, group_size, blocking):
    head_dim = _check_int(head_dim, "head_dim")
    group_size = _check_int(group_size, "group_size")
    n_tok = _validate_roundtrip_values(input, output, head_dim, group_size)
    dev = _check_same_device(input, output)
    return _run(dev, blocking, "quant_dequant_roundtrip_values",
                _lib.kivi_quant_dequant_roundtrip_values, _ptr(input), _ptr(output),
                n_tok, head_dim, group_size, keep=(input, output))


def quantize_keys(input, output, scales, zeros, group_size):
    """Asymmetric 2-bit key quantization (per-channel)."""
    return _quantize_keys(input, output, scales, zeros, group_size, True)


def quantize_values(input, output, scales, zeros, head_dim, group_size):
    """Asymmetric 2-bit value quantization (per-token)."""
    return _quantize_values(input, output, scales, zeros, head_dim, group_size, True)


def dequantize_keys(input, scales, zeros, output, group_size):
    """Asymmetric 2-bit key dequantization (per-channel)."""
    return _dequantize_keys(input, scales, zeros, output, group_size, True)


def dequantize_values(input, scales, zeros, output, head_dim, group_size):
    """Asymmetric 2-bit value dequantization (per-token)."""
    return _dequantize_values(input, scales, zeros, output, head_dim, group_size, True)


def quant_dequant_roundtrip_keys(input, output, group_size):
    """Fused quantize->dequantize round-trip (per-channel); output is
    bit-identical to quantize_keys followed by dequantize_keys."""
    return _roundtrip_keys(input, output, group_size, True)


def quant_dequant_roundtrip_values(input, output, head_dim, group_size):
    """Fused quantize->dequantize round-trip (per-token)."""
    return _roundtrip_values(input, output, head_dim, group_size, True)


def quantize_keys_async(input, output, scales, zeros, group_size):
    """Non-blocking quantize_keys -- returns a KiviEvent, does not wait."""
    return _quantize_keys(input, output, scales, zeros, group_size, False)


def quantize_values_async(input, output, scales, zeros, head_dim, group_size):
    """Non-blocking quantize_values -- returns a KiviEvent, does not wait."""
    return _quantize_values(input, output, scales, zeros, head_dim, group_size, False)


def dequantize_keys_async(input, scales, zeros, output, group_size):
    """Non-blocking dequantize_keys -- returns a KiviEvent, does not wait."""
    return _dequantize_keys(input, scales, zeros, output, group_size, False)


def dequantize_values_async(input, scales, zeros, output, head_dim, group_size):
    """Non-blocking dequantize_values -- returns a KiviEvent, does not wait."""
    return _dequantize_values(input, scales, zeros, output, head_dim, group_size, False)


def quant_dequant_roundtrip_keys_async(input, output, group_size):
    """Non-blocking quant_dequant_roundtrip_keys -- returns a KiviEvent."""
    return _roundtrip_keys(input, output, group_size, False)


def quant_dequant_roundtrip_values_async(input, output, head_dim, group_size):
    """Non-blocking quant_dequant_roundtrip_values -- returns a KiviEvent."""
    return _roundtrip_values(input, output, head_dim, group_size, False)


# --------------------------------------------------------------------------
# Fused packed-KV decode attention (no reference counterpart; see
# include/kivi_hip.h).  Not part of the reference's twelve ops.
# --------------------------------------------------------------------------
_ws_cache = {}


def _workspace(device, nbytes: int):
    if nbytes == 0:
        return None
    key = (device_index(device), stream_handle(device))
    buf = _ws_cache.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _ws_cache[key] = buf
    return buf


def packed_decode_attention(q, store, softmax_scale=None, out=None, num_splits=0,
                            workspace=None):
    """o = softmax(q . [K_hat; K_res]^T * scale) . [V_hat; V_res] for one query
    token per sequence, straight from a :class:`PackedKVStore`.

    q: [B, Hq, D] or [B, Hq, 1, D] fp32 on the store's device.  Returns
    ``out`` ([B, Hq, D] fp32), launched on the current stream (asynchronous).

    A decode step makes this call once per layer, so the checks are ordered
    for the common case: one combined test each, the detailed messages only
    on failure."""
    if not (isinstance(q, torch.Tensor) and q.is_cuda and q.dtype is torch.float32
            and q.is_contiguous()):
        _check_tensor(q, "q", torch.float32)
    B, D = store.B, store.D
    shp = q.shape
    nd = len(shp)
    if not ((nd == 3 or (nd == 4 and shp[2] == 1)) and shp[0] == B and shp[-1] == D):
        _fail("q must be [B, Hq, D] or [B, Hq, 1, D] matching the store, got ", tuple(shp))
    Hq = shp[1]
    dev = q.get_device()
    _check(dev == device_index(store.device), "q must be on the store's device")
    if out is None:
        out = q.new_empty((B, Hq, D))
    else:
        _check_tensor(out, "out", torch.float32)
        _check(out.numel() == B * Hq * D, "out must hold B*Hq*D elements")
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    need = store.workspace_bytes(Hq, num_splits)
    if workspace is None:
        workspace = _workspace(dev, need)
    elif need:
        _check(workspace.is_contiguous() and workspace.numel() * workspace.element_size() >= need,
               "workspace must be contiguous and hold ", need, " bytes")
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    res_dt = store.res_dtype_code
    pend = getattr(store, "_pending", None)
    if pend is not None:
        # the staged token goes into the ring within this launch
        kn, vn = pend
        # (plain ints for the pointers: the entry points' argtypes convert them)
        with on_device(dev):
            _native.check(_lib.kivi_packed_decode_attention_append(
                q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kn.stride(0), kn.stride(1),
                store.k_codes.data_ptr(), store.k_scale.data_ptr(), store.k_zero.data_ptr(),
                store.v_codes.data_ptr(), store.v_scale.data_ptr(), store.v_zero.data_ptr(),
                store.k_res.data_ptr(), store.v_res.data_ptr(), res_dt, out.data_ptr(),
                workspace.data_ptr() if workspace is not None else 0, ws_bytes,
                B, Hq, store.H, D, store.G, store.Gv, store.capacity, store.n_chunks, store.R,
                store.res_start, store.res_len, scale, int(num_splits),
                stream_handle(dev)), "packed_decode_attention")
        store._pending = None
        return out
    with on_device(dev):
        _native.check(_lib.kivi_packed_decode_attention(
            q.data_ptr(), store.k_codes.data_ptr(), store.k_scale.data_ptr(),
            store.k_zero.data_ptr(), store.v_codes.data_ptr(), store.v_scale.data_ptr(),
            store.v_zero.data_ptr(), store.k_res.data_ptr(), store.v_res.data_ptr(), res_dt,
            out.data_ptr(), workspace.data_ptr() if workspace is not None else 0, ws_bytes,
            B, Hq, store.H, D, store.G, store.Gv, store.capacity, store.n_chunks, store.R,
            store.res_start, store.res_len, scale, int(num_splits),
            stream_handle(dev)), "packed_decode_attention")
    return out


def hidden_positions(key_mask, device=None):
    """The hidden-position words of kivi_packed_attention_masked from a
    key-padding mask ``[B, T]`` (HF's 2-D ``attention_mask`` convention:
    nonzero / True = the position is attended): ``[B, ceil(T / 32)]`` int32,
    bit ``p % 32`` of word ``p // 32`` of row b set when position p of
    sequence b is hidden.  Computed on ``device`` (default: the mask's)."""
    _check(torch.is_tensor(key_mask) and key_mask.dim() == 2,
           "key_mask must be a [B, T] tensor")
    dev = key_mask.device if device is None else torch.device(device)
    vis = key_mask.to(dev) != 0
    B, T = vis.shape
    W = (T + 31) // 32
    bits = torch.zeros(B, W * 32, dtype=torch.int64, device=dev)
    bits[:, :T] = (~vis).to(torch.int64)
    words = (bits.view(B, W, 32) << torch.arange(32, device=dev)).sum(-1)    # < 2^32
    return torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)


def packed_attention(q, store, causal=True, softmax_scale=None, out=None, num_splits=0,
                     workspace=None, kv_start=None, key_mask=None, hidden=None):
    """Attention of ``L`` query tokens per sequence over a
    :class:`PackedKVStore`, ``q [B, Hq, L, D]`` fp32 (the layout HF attention
    functions receive); returns ``[B, L, Hq, D]`` fp32 (the layout they
    return).  ``causal``: the L queries are the residual window's last L
    tokens and token i attends to the cache up to itself (a multi-token
    forward on a non-empty cache); otherwise every query sees the whole
    context (one query token sees it either way).  ``kv_start`` (B ints, a
    list or an int32 tensor): sequence b's first visible context position,
    for a left-padded batch; positions before it take no weight.  Checked
    against the context length when given on the host.  ``key_mask``
    ``[B, T]`` over the whole context (T = quantised + window tokens; nonzero
    = attended, HF's 2-D padding mask), or ``hidden`` (its words,
    :func:`hidden_positions`, computed once for many calls): any other
    padding pattern (right padding, holes), hidden from every query token;
    a query row that sees no position gets zeros.  Launched on the current
    stream."""
    _check(q.dtype == torch.float32, "q must be float32, got ", _dtype_name(q.dtype))
    _check(q.dim() == 4 and q.shape[0] == store.B and q.shape[3] == store.D,
           "q must be [B, Hq, L, D] matching the store, got ", tuple(q.shape))
    _check(q.device == store.device, "q must be on the store's device")
    B, Hq, L, D = q.shape
    store._commit()
    if causal and L > 1:
        _check(L <= store.res_len, "causal attention of ", L, " query tokens needs them in "
               "the residual window (", store.res_len, " tokens)")
    ks_ptr = 0
    if kv_start is not None:
        if not (torch.is_tensor(kv_start) and kv_start.device == q.device):
            starts = [int(x) for x in (kv_start.tolist() if torch.is_tensor(kv_start)
                                       else kv_start)]
            T = store.quantized_tokens + store.res_len
            last = T - L if causal else T - 1
            _check(len(starts) == B and all(0 <= x <= last for x in starts),
                   "kv_start must hold ", B, " positions in [0, ", last, "], got ", starts)
            kv_start = torch.tensor(starts, dtype=torch.int32).to(q.device)
        _check(kv_start.dtype == torch.int32 and kv_start.numel() == B and
               kv_start.is_contiguous(), "kv_start must be a contiguous int32 tensor of ", B,
               " positions")
        ks_ptr = kv_start.data_ptr()
    if key_mask is not None:
        _check(hidden is None, "pass key_mask or hidden, not both")
        T = store.quantized_tokens + store.res_len
        _check(tuple(key_mask.shape) == (B, T), "key_mask must be [B=", B, ", T=", T,
               "] over the whole context, got ", tuple(key_mask.shape))
        hidden = hidden_positions(key_mask, q.device)
    if hidden is not None:
        W = (store.quantized_tokens + store.res_len + 31) // 32
        _check(hidden.dtype == torch.int32 and hidden.dim() == 2 and hidden.shape[0] == B and
               hidden.shape[1] >= W and hidden.stride(1) == 1 and hidden.device == q.device,
               "hidden must be an int32 [B, >=", W, "] tensor with contiguous rows on the "
               "query's device")
    qk = q.transpose(1, 2).contiguous()                                  # [B, L, Hq, D]
    if out is None:
        out = torch.empty(B, L, Hq, D, dtype=torch.float32, device=q.device)
    else:
        _check_tensor(out, "out", torch.float32)
        _check(out.numel() == B * L * Hq * D, "out must hold B*L*Hq*D elements")
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    need = int(_lib.kivi_packed_attention_workspace_size(
        B, L, Hq, store.H, D, store.G, store.Gv, store.n_chunks, store.res_len, num_splits))
    if workspace is None:
        workspace = _workspace(q.device, need)
    elif need:
        _check(workspace.is_contiguous() and workspace.numel() * workspace.element_size() >= need,
               "workspace must be contiguous and hold ", need, " bytes")
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    if hidden is not None:
        entry = functools.partial(_lib.kivi_packed_attention_masked,
                                  ctypes.c_void_p(qk.data_ptr()), L, 1 if causal else 0,
                                  ctypes.c_void_p(ks_ptr), ctypes.c_void_p(hidden.data_ptr()),
                                  hidden.stride(0))
    else:
        entry = functools.partial(_lib.kivi_packed_attention, ctypes.c_void_p(qk.data_ptr()),
                                  L, 1 if causal else 0, ctypes.c_void_p(ks_ptr))
    with on_device(q.device):
        _native.check(entry(
            ctypes.c_void_p(store.k_codes.data_ptr()),
            ctypes.c_void_p(store.k_scale.data_ptr()), ctypes.c_void_p(store.k_zero.data_ptr()),
            ctypes.c_void_p(store.v_codes.data_ptr()), ctypes.c_void_p(store.v_scale.data_ptr()),
            ctypes.c_void_p(store.v_zero.data_ptr()), ctypes.c_void_p(store.k_res.data_ptr()),
            ctypes.c_void_p(store.v_res.data_ptr()), store.res_dtype_code,
            ctypes.c_void_p(out.data_ptr()),
            ctypes.c_void_p(workspace.data_ptr() if workspace is not None else 0), ws_bytes,
            B, Hq, store.H, D, store.G, store.Gv, store.capacity, store.n_chunks, store.R,
            store.res_start, store.res_len, scale, int(num_splits),
            ctypes.c_void_p(_stream_of(q.device))), "packed_attention")
    return out
