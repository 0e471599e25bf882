"""GPU parity of the 2-bit codec against the CPU oracle, through the C ABI
(via the ``_C`` facade).  Bar: packed bytes, scales, zeros and dequantised
floats bit-exact; fused round-trip bit-identical to quantize + dequantize
(tests/integration/test_roundtrip_kernels.py:47,72 in the reference).
"""

import numpy as np
import pytest
import torch

from oracle import codec
from tests.conftest import seeded_kv

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C(hip_device):
    from intel_kivi_hybrid_amd import _C
    return _C


def _bits(t):
    a = t.detach().cpu().contiguous().numpy()
    return a.view(np.uint32) if a.dtype == np.float32 else a


def _quantize_gpu(C, x, G, kind, head_dim=None):
    dev = torch.device("cuda:0")
    xd = x.to(dev)
    n = x.numel()
    packed = torch.empty(n // 4, dtype=torch.uint8, device=dev)
    scales = torch.empty(n // G, dtype=torch.float32, device=dev)
    zeros = torch.empty(n // G, dtype=torch.float32, device=dev)
    if kind == "key":
        C.quantize_keys(xd, packed, scales, zeros, G)
    else:
        C.quantize_values(xd, packed, scales, zeros, head_dim, G)
    return xd, packed, scales, zeros


def _assert_codec_parity(C, x, G, kind="key", head_dim=None):
    print(f"[codec parity] kind={kind} shape={tuple(x.shape)} G={G}", flush=True)
    xd, packed, scales, zeros = _quantize_gpu(C, x, G, kind, head_dim)
    op, os_, oz = codec.quantize_groups(x.numpy(), G)
    assert np.array_equal(_bits(packed), op), "packed bytes differ from the oracle"
    assert np.array_equal(_bits(scales), os_.view(np.uint32)), "scales differ"
    assert np.array_equal(_bits(zeros), oz.view(np.uint32)), "zeros differ"
    deq = torch.empty_like(xd)
    if kind == "key":
        C.dequantize_keys(packed, scales, zeros, deq, G)
    else:
        C.dequantize_values(packed, scales, zeros, deq, head_dim, G)
    od = codec.dequantize_groups(op, os_, oz, G)
    assert np.array_equal(_bits(deq).reshape(-1), od.view(np.uint32)), "dequant differs"
    fused = torch.empty_like(xd)
    if kind == "key":
        C.quant_dequant_roundtrip_keys(xd, fused, G)
    else:
        C.quant_dequant_roundtrip_values(xd, fused, head_dim, G)
    assert torch.equal(fused, deq), "fused round-trip != quantize + dequantize"
    return packed, scales, zeros


# ---- the reference's own test shapes and known answers ---------------------
def test_known_answer_228(C, kat):
    k = kat["packed_228_four_channels"]
    x = torch.tensor(k["input"], dtype=torch.float32).reshape(1, 1, 4, 4)
    packed, scales, zeros = _assert_codec_parity(C, x, 4)
    assert packed.cpu().tolist() == k["packed"]
    assert scales.cpu().tolist() == k["scale"] and zeros.cpu().tolist() == k["zero"]


def test_tie_group_rounds_half_away(C, kat):
    k = kat["tie_244"]
    x = torch.tensor(k["input"], dtype=torch.float32).reshape(1, 1, 1, 4)
    packed, _, _ = _assert_codec_parity(C, x, 4)
    assert packed.cpu().tolist() == k["packed_kernel"]


@pytest.mark.parametrize("shape,G", [((1, 1, 1, 4), 4), ((1, 1, 4, 32), 32)])
def test_constant_input(C, shape, G):
    x = torch.full(shape, 5.0)
    packed, scales, zeros = _assert_codec_parity(C, x, G)
    assert torch.all(scales.cpu() == torch.tensor(1e-10, dtype=torch.float32))
    out = torch.empty(shape, device="cuda:0")
    C.quant_dequant_roundtrip_keys(x.cuda(), out, G)
    assert torch.all(out.cpu() == 5.0)


@pytest.mark.parametrize("shape,G,kind,D", [
    ((1, 2, 4, 32), 32, "key", None),        # test_kivi.py:53-83
    ((1, 2, 8, 64), 32, "value", 64),        # test_kivi.py:106-138
    ((2, 4, 64, 32), 32, "key", None),       # test_kivi.py:209-243
    ((2, 4, 32, 64), 32, "value", 64),
    ((2, 3, 64, 32), 32, "key", None),       # test_roundtrip_kernels.py:30-51
    ((2, 3, 8, 64), 32, "value", 64),        # test_roundtrip_kernels.py:54-76
])
def test_reference_test_shapes(C, shape, G, kind, D):
    x = seeded_kv(shape, seed=sum(shape) + G, kind="key" if kind == "key" else "value")
    _assert_codec_parity(C, x, G, kind, D)


# ---- every kernel variant: segment widths 1..64 lanes and the serial path ----
@pytest.mark.parametrize("G", [4, 8, 12, 16, 20, 32, 64, 96, 128, 256, 512])
def test_group_sizes(C, G):
    x = seeded_kv((3, 5, 7, G), seed=G, kind="key")
    _assert_codec_parity(C, x, G)
    v = seeded_kv((2, 3, 17, 2 * G), seed=G + 1, kind="value")
    _assert_codec_parity(C, v, G, "value", 2 * G)


def test_ragged_group_count(C):
    # a group count that leaves partial tiles and partial waves
    x = seeded_kv((1, 1, 1037, 32), seed=5, kind="key")
    _assert_codec_parity(C, x, 32)


def test_dequantize_unaligned_buffers(C):
    """Dequantisation from packed bytes at any offset into an output at any
    4-byte offset gives the oracle's bits (an unaligned output takes scalar
    stores)."""
    x = seeded_kv((1, 2, 301, 64), seed=17, kind="key")
    _, packed, scales, zeros = _quantize_gpu(C, x, 64, "key")
    ref = codec.dequantize_groups(_bits(packed), _bits(scales).view(np.float32),
                                  _bits(zeros).view(np.float32), 64).view(np.uint32)
    n = x.numel()
    shifted = torch.empty(n // 4 + 1, dtype=torch.uint8, device="cuda:0")[1:]
    shifted.copy_(packed)
    assert shifted.data_ptr() % 4 != 0
    for p, out in ((packed, torch.empty(n, device="cuda:0")),
                   (shifted, torch.empty(n, device="cuda:0")),
                   (packed, torch.empty(n + 1, device="cuda:0")[1:])):
        C.dequantize_keys(p, scales, zeros, out.reshape(x.shape), 64)
        assert np.array_equal(_bits(out).reshape(-1), ref)


def test_quantize_codes_at_any_offset(C):
    """Quantisation into a code buffer 4-byte aligned (paired 32-bit code
    stores), 2-byte aligned (16-bit stores) or at an odd byte offset
    (per-byte stores) gives the oracle's codes, scales and zeros."""
    for kind, shape, G, D in (("key", (2, 3, 64, 256), 32, None),
                              ("value", (2, 3, 256, 64), 32, 64)):
        x = seeded_kv(shape, seed=31, kind=kind)
        xd = x.cuda()
        n = x.numel()
        op, os_, oz = codec.quantize_groups(x.numpy(), G)
        for off in (0, 2, 1):
            buf = torch.empty(n // 4 + 4, dtype=torch.uint8, device="cuda:0")
            packed = buf[off:off + n // 4]
            assert packed.data_ptr() % 4 == off
            scales = torch.empty(n // G, device="cuda:0")
            zeros = torch.empty(n // G, device="cuda:0")
            if kind == "key":
                C.quantize_keys(xd, packed, scales, zeros, G)
            else:
                C.quantize_values(xd, packed, scales, zeros, D, G)
            assert np.array_equal(_bits(packed), op), (kind, off)
            assert np.array_equal(_bits(scales), os_.view(np.uint32)), (kind, off)
            assert np.array_equal(_bits(zeros), oz.view(np.uint32)), (kind, off)


def test_unaligned_input_takes_scalar_path(C):
    base = seeded_kv((1, 1, 65, 32), seed=9, kind="key").reshape(-1)
    x = base[1:1 + 64 * 32].reshape(1, 1, 64, 32)   # 4-byte, not 16-byte aligned
    xd = base.cuda()[1:1 + 64 * 32].reshape(1, 1, 64, 32)
    assert xd.data_ptr() % 16 != 0 and xd.is_contiguous()
    packed = torch.empty(64 * 8, dtype=torch.uint8, device="cuda:0")
    scales = torch.empty(64, device="cuda:0")
    zeros = torch.empty(64, device="cuda:0")
    C.quantize_keys(xd, packed, scales, zeros, 32)
    op, os_, oz = codec.quantize_groups(x.numpy(), 32)
    assert np.array_equal(_bits(packed), op)
    assert np.array_equal(_bits(scales), os_.view(np.uint32))
    out = torch.empty(64 * 32 + 1, device="cuda:0")[1:]
    C.quant_dequant_roundtrip_keys(xd, out.reshape(1, 1, 64, 32), 32)
    assert np.array_equal(_bits(out), codec.roundtrip_groups(x.numpy(), 32).view(np.uint32))


def test_special_values(C):
    x = torch.tensor([
        float("nan"), 1.0, 2.0, 4.0,                  # NaN ignored, coded 0
        2e30, 3e30, 4e30, 5e30,                       # reference min init 1e30 wins
        -5e30, -4e30, -3e30, -2e30,                   # reference max init -1e30 wins
        0.0, -0.0, 1.0, 2.0,                          # signed zeros
        1e-40, -1e-40, 3e-41, 0.0,                    # denormals
        -3e38, 3e38, 0.0, 1.0,                        # range overflows to inf
        float("inf"), 1.0, 2.0, 3.0,
        float("-inf"), 1.0, 2.0, 3.0,
    ], dtype=torch.float32).reshape(1, 1, 8, 4)
    print("[codec parity] special values", flush=True)
    xd, packed, scales, zeros = _quantize_gpu(C, x, 4, "key")
    op, os_, oz = codec.quantize_groups(x.numpy(), 4)
    assert np.array_equal(_bits(packed), op)
    assert np.array_equal(_bits(scales), os_.view(np.uint32))
    assert np.array_equal(_bits(zeros), oz.view(np.uint32))


def test_exhaustive_small_groups(C):
    import itertools
    values = [-3.0, -1.0, -0.5, 0.0, 0.25, 0.5, 1.0, 1.5, 2.75]
    x = torch.tensor(list(itertools.product(values, repeat=4)), dtype=torch.float32)
    _assert_codec_parity(C, x, 4)


def test_tie_heavy_inputs_take_exact_path(C):
    # quotients landing exactly on k+0.5 (integers with scale 1) and just next
    # to it (one ulp away) exercise the fast-path guard
    g = torch.Generator().manual_seed(1)
    base = torch.randint(0, 7, (4096, 32), generator=g).float() * 0.5
    base[:, 0] = 0.0
    base[:, 1] = 3.0
    jitter = torch.nextafter(base, torch.full_like(base, 10.0))
    x = torch.where(torch.rand(base.shape, generator=g) < 0.3, jitter, base)
    x[:, 1] = 3.0
    _assert_codec_parity(C, x, 32)


# ---- benchmark config 2 at full size ---------------------------------------
def test_config2_full_size_bit_exact(C):
    """keys [8,32,128,4096] G=32 along tokens, values [8,32,4096,128] G=32."""
    k = seeded_kv((8, 32, 4096, 128), seed=1236, kind="key").transpose(2, 3).contiguous()
    ties = codec.count_ties(k.numpy(), 32)
    print(f"[config2] key ties: {ties}", flush=True)
    _assert_codec_parity(C, k, 32)
    del k
    v = seeded_kv((8, 32, 4096, 128), seed=1237, kind="value")
    print(f"[config2] value ties: {codec.count_ties(v.numpy(), 32)}", flush=True)
    _assert_codec_parity(C, v, 32, "value", 128)


# ---- async ops ----------------------------------------------------------------
def test_async_ops_and_event(C):
    x = seeded_kv((2, 3, 64, 32), seed=21, kind="key").cuda()
    n = x.numel()
    packed = torch.empty(n // 4, dtype=torch.uint8, device="cuda:0")
    scales = torch.empty(n // 32, device="cuda:0")
    zeros = torch.empty(n // 32, device="cuda:0")
    ev = C.quantize_keys_async(x, packed, scales, zeros, 32)
    assert isinstance(ev, C.KiviEvent)
    ev.wait()
    out = torch.empty_like(x)
    C.dequantize_keys_async(packed, scales, zeros, out, 32).wait()
    fused = torch.empty_like(x)
    C.quant_dequant_roundtrip_keys_async(x, fused, 32).wait()
    assert torch.equal(out, fused)
    v = seeded_kv((2, 3, 8, 64), seed=22, kind="value").cuda()
    vp = torch.empty(v.numel() // 4, dtype=torch.uint8, device="cuda:0")
    vs = torch.empty(v.numel() // 32, device="cuda:0")
    vz = torch.empty(v.numel() // 32, device="cuda:0")
    C.quantize_values_async(v, vp, vs, vz, 64, 32).wait()
    vo = torch.empty_like(v)
    C.dequantize_values_async(vp, vs, vz, vo, 64, 32).wait()
    vf = torch.empty_like(v)
    C.quant_dequant_roundtrip_values_async(v, vf, 64, 32).wait()
    assert torch.equal(vo, vf)
    assert np.array_equal(_bits(vf).reshape(-1),
                          codec.roundtrip_groups(v.cpu().numpy(), 32).view(np.uint32))


def test_event_recorded_at_submission(C):
    """By default an async op's event is recorded right after the op, as the
    reference's per-op sycl::event (kv_cache_ops.cpp:245-303): it exists
    before any wait(), waiting covers that op, repeated calls return at once,
    and results are exact."""
    import time
    x = seeded_kv((4, 8, 128, 256), seed=23, kind="key")
    xd = x.cuda()
    n = xd.numel()
    packed = torch.empty(n // 4, dtype=torch.uint8, device="cuda:0")
    scales = torch.empty(n // 32, device="cuda:0")
    zeros = torch.empty(n // 32, device="cuda:0")
    ev = C.quantize_keys_async(xd, packed, scales, zeros, 32)
    assert ev._ev is not None                  # marker recorded at submission
    out = torch.empty_like(xd)
    ev2 = C.dequantize_keys_async(packed, scales, zeros, out, 32)   # queued behind it
    assert ev2._ev is not None and ev2._ev.value != ev._ev.value
    ev.wait()
    assert ev.query() and ev._ev is None       # released after the wait
    ev.wait()                                  # a second wait returns at once
    op, os_, oz = codec.quantize_groups(x.numpy(), 32)
    assert np.array_equal(packed.cpu().numpy(), op)
    deadline = time.monotonic() + 30.0
    while not ev2.query():
        assert time.monotonic() < deadline, "dequantize never completed"
    ev2.wait()
    ref = codec.dequantize_groups(op, os_, oz, 32).reshape(x.shape)
    assert np.array_equal(_bits(out.cpu()).reshape(-1), ref.view(np.uint32).reshape(-1))


def test_lazy_event_recorded_at_first_use(C):
    """With lazy events switched on, an async op's event is recorded at its
    first wait()/query(), after the op on its stream: waiting then covers the
    op (and any work queued behind it), repeated calls return at once, and
    results are exact."""
    import time
    prev = C.set_lazy_events(True)
    try:
        x = seeded_kv((4, 8, 128, 256), seed=23, kind="key")
        xd = x.cuda()
        n = xd.numel()
        packed = torch.empty(n // 4, dtype=torch.uint8, device="cuda:0")
        scales = torch.empty(n // 32, device="cuda:0")
        zeros = torch.empty(n // 32, device="cuda:0")
        ev = C.quantize_keys_async(xd, packed, scales, zeros, 32)
        assert ev._ev is None                      # no marker put on the stream yet
        out = torch.empty_like(xd)
        ev2 = C.dequantize_keys_async(packed, scales, zeros, out, 32)   # queued behind it
        ev.wait()
        assert ev.query() and ev._ev is None       # released after the wait
        ev.wait()                                  # a second wait returns at once
        op, os_, oz = codec.quantize_groups(x.numpy(), 32)
        assert np.array_equal(packed.cpu().numpy(), op)
        deadline = time.monotonic() + 30.0
        while not ev2.query():
            assert time.monotonic() < deadline, "dequantize never completed"
        ev2.wait()
        ref = codec.dequantize_groups(op, os_, oz, 32).reshape(x.shape)
        assert np.array_equal(_bits(out.cpu()).reshape(-1), ref.view(np.uint32).reshape(-1))
    finally:
        C.set_lazy_events(prev)


def test_launch_event_entry_points(C):
    """The ``*_ev`` C-ABI entry points (the ``*_async`` ops' path) hand back
    the completion event of the op's own kernel launch: a live handle whose
    wait returns once the op is done, with exact results; on a rejected
    argument the handle stays NULL and the error code comes back."""
    import ctypes
    lib = C._lib
    x = seeded_kv((2, 4, 64, 128), seed=29, kind="key")
    xd = x.cuda()
    n = xd.numel()
    packed = torch.empty(n // 4, dtype=torch.uint8, device="cuda:0")
    scales = torch.empty(n // 32, device="cuda:0")
    zeros = torch.empty(n // 32, device="cuda:0")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ev = ctypes.c_void_p()
    rc = lib.kivi_quantize_keys_per_channel_ev(xd.data_ptr(), packed.data_ptr(),
                                               scales.data_ptr(), zeros.data_ptr(), n // 32, 32,
                                               stream, ctypes.byref(ev))
    assert rc == 0 and ev.value
    assert lib.kivi_event_wait(ev) == 0
    assert lib.kivi_event_query(ev) == 1
    assert lib.kivi_event_destroy(ev) == 0
    op, os_, oz = codec.quantize_groups(x.numpy(), 32)
    assert np.array_equal(packed.cpu().numpy(), op)
    assert np.array_equal(scales.cpu().numpy(), os_)
    out = torch.empty_like(xd)
    ev = ctypes.c_void_p()
    rc = lib.kivi_quant_dequant_roundtrip_values_ev(xd.data_ptr(), out.data_ptr(), n // 128, 128,
                                                    32, stream, ctypes.byref(ev))
    assert rc == 0 and ev.value
    assert lib.kivi_event_wait(ev) == 0
    lib.kivi_event_destroy(ev)
    ref = codec.roundtrip_groups(x.numpy(), 32)
    assert np.array_equal(_bits(out.cpu()).reshape(-1), ref.view(np.uint32).reshape(-1))
    ev = ctypes.c_void_p(1234)
    rc = lib.kivi_quantize_values_per_token_ev(xd.data_ptr(), packed.data_ptr(), scales.data_ptr(),
                                               zeros.data_ptr(), n // 128, 128, 3, stream,
                                               ctypes.byref(ev))
    assert rc == 1                          # KIVI_ERR_INVALID_ARGUMENT
    assert ev.value is None
