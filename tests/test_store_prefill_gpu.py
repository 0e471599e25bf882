"""GPU parity of the batched flush: one launch quantises every chunk an
append owes, reading the residual ring and the caller's new-token tensor in
place (the flush loop of KiviCache.add_tokens and its host transpose,
src/kivi_sycl/cache/manager.py:242-249,332-334).

Bar: bit-exact codes, scales, zeros and dequantised history against the
oracle's quantisation of the same tokens (bf16/fp16 inputs: of their exact
fp32 widening, which is what the reference's .float() makes of them)."""

import pytest
import torch

from tests.kv_helpers import check_store_bit_exact, fill_store, make_kv

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def store_cls(hip_device):
    from intel_kivi_hybrid_amd.store import PackedKVStore
    return PackedKVStore


SHAPES = [
    (1, 2, 8, 4, 4, 8, 30),          # the reference unit-test geometry, plain code layout
    (1, 12, 64, 32, 32, 32, 200),    # config 1 geometry
    (2, 3, 128, 32, 128, 48, 170),   # Gv != G, R not a multiple of G
    (4, 8, 128, 32, 32, 128, 1000),  # config 4 shape, a long prompt
    (2, 2, 256, 64, 32, 128, 300),   # G*D = 16384: the untiled kernel
    (2, 2, 256, 32, 64, 64, 200),    # compile-time shapes: D=256
    (2, 2, 128, 64, 128, 128, 300),  # G=64, one value group per token
    (1, 4, 64, 64, 32, 64, 200),     # G=64, D=64
]


@pytest.mark.parametrize("B,H,D,G,Gv,R,T", SHAPES)
@pytest.mark.parametrize("history", [False, True])
def test_prompt_in_one_call(store_cls, B, H, D, G, Gv, R, T, history):
    print(f"[prefill] B={B} H={H} D={D} G={G} Gv={Gv} R={R} T={T} hist={history}", flush=True)
    k, v = make_kv(B, H, T, D, seed=3 * T + D)
    st = store_cls(B, H, D, G, R, "cuda:0", group_size_v=Gv, keep_history=history)
    n = st.extend(k.cuda(), v.cuda(), flush_at=R)
    expect = 0 if T < R else (T - R) // G + 1
    assert n == expect and st.n_chunks == expect and st.res_len == T - expect * G
    check_store_bit_exact(st, k, v)


@pytest.mark.parametrize("B,H,D,G,Gv,R,T", SHAPES[1:4])
def test_one_call_equals_group_by_group(store_cls, B, H, D, G, Gv, R, T):
    """The one-launch path stores exactly what feeding the tokens a group at a
    time (one flush launch per chunk) stores."""
    k, v = make_kv(B, H, T, D, seed=T)
    a = store_cls(B, H, D, G, R, "cuda:0", group_size_v=Gv, keep_history=True)
    b = store_cls(B, H, D, G, R, "cuda:0", group_size_v=Gv, keep_history=True)
    a.extend(k.cuda(), v.cuda(), flush_at=R)
    fill_store(b, k, v, R)
    assert (a.n_chunks, a.res_len) == (b.n_chunks, b.res_len)
    n = a.n_chunks
    for name in ("k_codes", "k_scale", "k_zero", "v_codes", "v_scale", "v_zero"):
        assert torch.equal(getattr(a, name)[:, :, :n], getattr(b, name)[:, :, :n]), name
    assert torch.equal(a.k_hist[:, :, :n * G], b.k_hist[:, :, :n * G])
    assert torch.equal(a.v_hist[:, :, :n * G], b.v_hist[:, :, :n * G])
    for x, y in zip(a.residual(), b.residual()):
        assert torch.equal(x, y)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,G,Gv", [(128, 32, 32), (8, 4, 4)])
def test_half_precision_inputs(store_cls, dtype, D, G, Gv):
    """bf16/fp16 K/V are read as they are and quantise exactly as their fp32
    widening does; the residual keeps the widened values."""
    B, H, T, R = 2, 4, 333, 64
    k, v = make_kv(B, H, T, D, seed=77)
    kh, vh = k.to(dtype), v.to(dtype)
    st = store_cls(B, H, D, G, R, "cuda:0", group_size_v=Gv, keep_history=True)
    st.extend(kh.cuda(), vh.cuda(), flush_at=R)
    check_store_bit_exact(st, kh.float(), vh.float())


@pytest.mark.parametrize("layout", ["transposed", "fused_qkv", "unaligned"])
def test_strided_inputs(store_cls, layout):
    """Non-contiguous K/V (the [B,T,H,D] -> [B,H,T,D] view HF attention makes,
    K/V slices of a fused QKV projection, rows not 16-byte aligned) are read
    in place and give the contiguous result."""
    B, H, T, D, G, R = 2, 4, 290, 64, 32, 64
    k, v = make_kv(B, H, T, D, seed=5)
    if layout == "transposed":
        kb = k.transpose(1, 2).contiguous().cuda().transpose(1, 2)
        vb = v.transpose(1, 2).contiguous().cuda().transpose(1, 2)
    elif layout == "fused_qkv":
        qkv = torch.empty(B, T, 3, H, D)
        qkv[:, :, 1] = k.transpose(1, 2)
        qkv[:, :, 2] = v.transpose(1, 2)
        qkv = qkv.cuda()
        kb, vb = qkv[:, :, 1].transpose(1, 2), qkv[:, :, 2].transpose(1, 2)
    else:
        pad_k = torch.zeros(B, H, T, D + 1)
        pad_v = torch.zeros(B, H, T, D + 1)
        pad_k[..., 1:] = k
        pad_v[..., 1:] = v
        kb, vb = pad_k.cuda()[..., 1:], pad_v.cuda()[..., 1:]
    assert not kb.is_contiguous() and kb.stride(-1) == 1
    st = store_cls(B, H, D, G, R, "cuda:0", keep_history=True)
    st.extend(kb, vb, flush_at=R)
    check_store_bit_exact(st, k, v)


@pytest.mark.parametrize("first,second", [(50, 200), (63, 1), (40, 97), (10, 64)])
def test_chunks_straddle_ring_and_new_tokens(store_cls, first, second):
    """With tokens already in the (wrapped) ring, the owed chunks take the
    ring's tokens first and continue into the new ones."""
    B, H, D, G, R = 2, 3, 64, 32, 64
    T = 37 + first + second
    k, v = make_kv(B, H, T, D, seed=first * 7 + second)
    st = store_cls(B, H, D, G, R, "cuda:0", keep_history=True)
    st.extend(k[:, :, :37].cuda(), v[:, :, :37].cuda(), flush_at=R)   # res_start moves on
    st.extend(k[:, :, 37:37 + first].cuda(), v[:, :, 37:37 + first].cuda(), flush_at=R)
    st.extend(k[:, :, 37 + first:].cuda(), v[:, :, 37 + first:].cuda(), flush_at=R)
    expect = 0 if T < R else (T - R) // G + 1
    assert st.n_chunks == expect and st.res_len == T - expect * G
    check_store_bit_exact(st, k, v)


def _tie_heavy(B, H, T, D, seed):
    """K/V whose codes sit on rounding ties: bf16-grid values (a coarse grid
    puts (x - min) / scale within a hair of k + 0.5 in ~40% of 64-lane
    waves), plus groups made of exact ties ({0, 0.5, 1.5, 2.5, 3} * step:
    scale = step, quotients exactly 0.5, 1.5, 2.5) and constant groups."""
    k, v = make_kv(B, H, T, D, seed)
    k = k.to(torch.bfloat16).float()
    v = v.to(torch.bfloat16).float()
    g = torch.Generator().manual_seed(seed + 5)
    pattern = torch.tensor([0.0, 0.5, 1.5, 2.5, 3.0])
    for h in range(H):
        step = float(2.0 ** int(torch.randint(-6, 6, (1,), generator=g)))
        # keys: channel 3 of head h cycles through exact-tie multiples (per
        # 32-token group its min is 0 and max 3*step, so scale = step)
        idx = torch.arange(T) % 5
        k[:, h, :, 3] = pattern[idx] * step
        # values: token 7 of every 32 holds exact ties along its channels
        for t in range(7, T, 32):
            v[:, h, t, :] = pattern[torch.arange(D) % 5] * step
        k[:, h, :, 5] = 1.25                     # constant channel: scale 1e-10
    return k, v


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,D,G,Gv,R,T", [(2, 4, 128, 32, 32, 128, 1200),
                                            (1, 4, 64, 32, 32, 64, 700),
                                            (2, 2, 128, 64, 128, 128, 600)])
def test_prompt_on_rounding_ties(store_cls, dtype, B, H, D, G, Gv, R, T):
    """Inputs full of exact and near rounding ties (bf16 grids, crafted tie
    groups, constant groups) through the one-launch flush: codes, scales,
    zeros and history bit-exact against the oracle (round half away from
    zero of the correctly rounded quotient, quant_tile.hpp:53-70)."""
    print(f"[prefill-ties] {dtype} B={B} H={H} D={D} G={G} Gv={Gv} R={R} T={T}", flush=True)
    k, v = _tie_heavy(B, H, T, D, seed=T + D)
    st = store_cls(B, H, D, G, R, "cuda:0", group_size_v=Gv, keep_history=True)
    st.extend(k.to("cuda:0", dtype), v.to("cuda:0", dtype), flush_at=R)
    check_store_bit_exact(st, k, v)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_prompt_with_huge_ranges(store_cls, dtype):
    """Groups whose scale exceeds 2^120 (values near 1e37, where the divide-
    free exact quotient's argument does not hold) take the correctly rounded
    divide for their tensor; every code, scale and zero stays bit-exact."""
    B, H, D, G, Gv, R, T = 2, 2, 128, 32, 32, 128, 300
    k, v = make_kv(B, H, T, D, seed=77)
    k[0, 1, :, 9] *= 3e36            # one key channel of every chunk
    v[1, 0, 40:45, :] *= 3e36        # the value groups of five tokens
    k, v = k.to(dtype).float(), v.to(dtype).float()
    st = store_cls(B, H, D, G, R, "cuda:0", group_size_v=Gv, keep_history=True)
    st.extend(k.to("cuda:0", dtype), v.to("cuda:0", dtype), flush_at=R)
    check_store_bit_exact(st, k, v)
