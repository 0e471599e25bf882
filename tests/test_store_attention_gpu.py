"""GPU parity of the HBM-resident store (flush) and the fused packed decode
attention, against the CPU oracle.

Flush bar: codes (through the documented byte transposes), scales, zeros and
the served dequantised history bit-exact.  Attention bar: within 1e-3
relative (max |o - o_ref| / max |o_ref| per (batch, head)) of float64 SDPA
over the oracle-dequantised history plus the fp32 residual.
"""

import numpy as np
import pytest
import torch

from oracle.attention import decode_attention
from tests.kv_helpers import (check_store_bit_exact, fill_store, make_kv, oracle_history,
                              rel_err, seeded_q)

pytestmark = pytest.mark.gpu

ATTN_TOL = 1e-3


@pytest.fixture(scope="module")
def store_cls(hip_device):
    from intel_kivi_hybrid_amd.store import PackedKVStore
    return PackedKVStore


@pytest.mark.parametrize("B,H,D,G,Gv,R,T", [
    (1, 2, 8, 4, 4, 8, 30),          # the reference unit-test geometry (G=4, R=8, D=8)
    (1, 12, 64, 32, 32, 32, 200),    # benchmark config 1 geometry
    (2, 3, 128, 32, 128, 48, 170),   # Gv != G, ring wrap (R not a multiple of G)
    (2, 2, 64, 16, 16, 40, 133),
])
def test_flush_bit_exact(store_cls, B, H, D, G, Gv, R, T):
    print(f"[flush] B={B} H={H} D={D} G={G} Gv={Gv} R={R} T={T}", flush=True)
    k, v = make_kv(B, H, T, D, seed=T + D)
    st = store_cls(B, H, D, G, R, "cuda:0", group_size_v=Gv, keep_history=True)
    fill_store(st, k, v, R)
    n_flush = 0 if T < R else (T - R) // G + 1
    assert st.n_chunks == n_flush and st.res_len == T - n_flush * G
    check_store_bit_exact(st, k, v)


def _attention_case(store_cls, B, Hq, Hkv, D, G, Gv, R, T, splits=0, seed=0):
    print(f"[attn] B={B} Hq={Hq} Hkv={Hkv} D={D} G={G} Gv={Gv} R={R} T={T} splits={splits}",
          flush=True)
    k, v = make_kv(B, Hkv, T, D, seed=seed + T)
    st = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    fill_store(st, k, v, R)
    q = seeded_q(B, Hq, D, seed=seed + 99)
    out = st.attention(q.cuda(), num_splits=splits)
    torch.cuda.synchronize()
    kh, vh = oracle_history(k, v, st.n_chunks, G, Gv)
    q0 = st.n_chunks * G
    ref = decode_attention(q.numpy(), kh, vh, k[:, :, q0:].numpy(), v[:, :, q0:].numpy())
    err = rel_err(out.cpu().numpy(), ref)
    print(f"[attn]   chunks={st.n_chunks} res={st.res_len} rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL
    return err


@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (8, 4), (16, 4), (32, 4)])
@pytest.mark.parametrize("D", [64, 128])
def test_attention_gqa_ratios(store_cls, Hq, Hkv, D):
    _attention_case(store_cls, 2, Hq, Hkv, D, 32, 32, 64, 300)


# Ratios of query to kv heads that are not a power of two (Llama-3.2-3B 3,
# Qwen2.5-14B 5, Qwen2-7B 7) pad the launch's rows to the next power of two;
# more than 8 (multi-query models) take one launch per group of 8 heads.
@pytest.mark.parametrize("Hq,Hkv", [(6, 2), (10, 2), (12, 2), (14, 2), (28, 4), (24, 2),
                                    (32, 2), (40, 1)])
@pytest.mark.parametrize("D", [64, 128])
def test_attention_any_head_ratio(store_cls, Hq, Hkv, D):
    _attention_case(store_cls, 2, Hq, Hkv, D, 32, 32, 64, 300)


@pytest.mark.parametrize("Hq,Hkv,splits", [(14, 2, 0), (14, 2, 3), (24, 2, 1), (40, 1, 5)])
def test_attention_any_head_ratio_long(store_cls, Hq, Hkv, splits):
    """Long enough for the mode where one wave takes the window (1 split),
    and split merges, with padded rows and head groups."""
    _attention_case(store_cls, 1, Hq, Hkv, 128, 32, 32, 128, 2400, splits=splits, seed=5)


@pytest.mark.parametrize("Hq,Hkv", [(6, 2), (24, 2)])
def test_attention_any_head_ratio_plain_layout(store_cls, Hq, Hkv):
    """The generic kernel (plain layout, G=16) with padded rows and head groups."""
    _attention_case(store_cls, 2, Hq, Hkv, 64, 16, 16, 32, 100)


@pytest.mark.parametrize("Hq,Hkv", [(14, 2), (24, 2)])
def test_fused_append_any_head_ratio(store_cls, Hq, Hkv):
    """A decode step whose token the attention launch itself files in the ring:
    with head groups every launch reads the token from its own tensor, and
    the result matches the call that reads it from the ring bit for bit."""
    B, D, G, R, T = 2, 128, 32, 128, 700
    print(f"[attn] fused append Hq={Hq} Hkv={Hkv}", flush=True)
    k, v = make_kv(B, Hkv, T, D, seed=17)
    st = store_cls(B, Hkv, D, G, R, "cuda:0")
    fill_store(st, k[:, :, :T - 1], v[:, :, :T - 1], R)
    st.stage_token(k[:, :, T - 1:].cuda(), v[:, :, T - 1:].cuda())
    q = seeded_q(B, Hq, D, seed=18).cuda()
    fused = st.attention(q).cpu().numpy()
    ring = st.attention(q).cpu().numpy()
    assert np.array_equal(fused.view(np.uint32), ring.view(np.uint32))
    kh, vh = oracle_history(k, v, st.n_chunks, G, G)
    q0 = st.n_chunks * G
    ref = decode_attention(q.cpu().numpy(), kh, vh, k[:, :, q0:].numpy(), v[:, :, q0:].numpy())
    err = rel_err(fused, ref)
    print(f"[attn]   rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL


@pytest.mark.parametrize("T", [1, 40, 127])
@pytest.mark.parametrize("ring", [torch.float32, torch.bfloat16])
def test_window_only_context(store_cls, T, ring):
    """A context still wholly in the residual window (no chunk yet) runs on
    the matrix-core kernel's window pass; the same call through the C ABI
    with no chunk arrays at all (null pointers, no capacity) runs on the
    generic kernel.  Both against the oracle; then a decode step whose token
    the launch files itself, bit-identical to reading it from the ring."""
    import ctypes
    from intel_kivi_hybrid_amd import _native
    B, Hq, Hkv, D, G, R = 2, 8, 2, 128, 32, 128
    print(f"[attn] window only T={T} ring={ring}", flush=True)
    k, v = make_kv(B, Hkv, T + 1, D, seed=60 + T)
    st = store_cls(B, Hkv, D, G, R, "cuda:0", residual_dtype=ring)
    st.extend(k[:, :, :T].cuda().to(ring), v[:, :, :T].cuda().to(ring), flush_at=R)
    assert (st.n_chunks, st.res_len) == (0, T)
    kq, vq = k.to(ring).float(), v.to(ring).float()     # what the ring holds
    q = seeded_q(B, Hq, D, seed=61).cuda()
    out = st.attention(q).cpu().numpy()
    empty = np.zeros((B, Hkv, 0, D), np.float32)
    ref = decode_attention(q.cpu().numpy(), empty, empty, kq[:, :, :T].numpy(),
                           vq[:, :, :T].numpy())
    err = rel_err(out, ref)
    print(f"[attn]   matrix-core window pass rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL
    lib = _native.load()
    gen = torch.full_like(q, float("nan"))
    vp = lambda x: ctypes.c_void_p(x.data_ptr())       # noqa: E731
    _native.check(lib.kivi_packed_decode_attention(
        vp(q), None, None, None, None, None, None, vp(st.k_res), vp(st.v_res),
        st.res_dtype_code, vp(gen), None, 0, B, Hq, Hkv, D, G, G, 0, 0, R, st.res_start,
        st.res_len, float(D ** -0.5), 0, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
        "kivi_packed_decode_attention")
    err = rel_err(gen.cpu().numpy(), ref)
    print(f"[attn]   generic kernel (no chunk arrays) rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL
    st.stage_token(k[:, :, T:].cuda().to(ring), v[:, :, T:].cuda().to(ring))
    fused = st.attention(q).cpu().numpy()
    again = st.attention(q).cpu().numpy()
    assert np.array_equal(fused.view(np.uint32), again.view(np.uint32))
    ref = decode_attention(q.cpu().numpy(), empty, empty, kq.numpy(), vq.numpy())
    err = rel_err(fused, ref)
    print(f"[attn]   fused append rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL


@pytest.mark.parametrize("G,Gv,R,T", [
    (16, 16, 32, 100), (32, 128, 128, 400), (64, 64, 64, 400), (32, 32, 32, 32),
    (32, 32, 128, 127),   # residual only, no chunk yet
    (32, 32, 32, 64),     # residual empty right after a flush
    (32, 32, 48, 77),     # ring wrap
])
def test_attention_group_shapes(store_cls, G, Gv, R, T):
    _attention_case(store_cls, 2, 8, 2, 128, G, Gv, R, T)


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 64])
def test_attention_split_counts_agree(store_cls, splits):
    _attention_case(store_cls, 1, 8, 2, 128, 32, 32, 128, 2000, splits=splits, seed=3)


# Up to 32 splits merge in registers, more through LDS: 6000 tokens give 183
# chunks, room for 46 splits of four chunks.
@pytest.mark.parametrize("splits", [16, 17, 32, 33, 46])
def test_attention_merge_paths(store_cls, splits):
    _attention_case(store_cls, 1, 8, 2, 128, 32, 32, 128, 6000, splits=splits, seed=4)


def test_attention_reference_cosine_gate(store_cls, kat):
    """The reference's only attention check (test_attention_fix.py:33-115):
    KIVI attention vs fp32 attention cosine > 0.85 at B=1, H=2, cache 32,
    D=64, G=32 (one token per query here; the reference used 3)."""
    g = kat["attention_cosine_gate"]
    torch.manual_seed(42)
    B, H, T, D, G = g["B"], g["H"], g["cache_len"], g["D"], g["G"]
    q = torch.randn(B, H, D)
    k = torch.randn(B, H, T, D)
    v = torch.randn(B, H, T, D)
    st = store_cls(B, H, D, G, G, "cuda:0")
    fill_store(st, k, v, G)
    assert st.n_chunks == 1 and st.res_len == 0
    out = st.attention(q.cuda()).cpu().double()
    ref = decode_attention(q.numpy(), k.numpy(), v.numpy(), None, None)
    cos = torch.nn.functional.cosine_similarity(out.reshape(1, -1),
                                                torch.from_numpy(ref).reshape(1, -1)).item()
    print(f"[attn] cosine vs fp32 = {cos:.4f}", flush=True)
    assert cos > g["min_cosine"]


@pytest.mark.parametrize("B,Hq,Hkv,D,G,Gv,R,T", [
    (2, 32, 8, 128, 32, 32, 128, 4196),     # config-4 head geometry, 2 sequences
    (1, 16, 2, 256, 32, 64, 64, 1000),      # D=256, Gv=64
    (1, 16, 2, 128, 64, 64, 128, 2000),     # GQA 8, G=64
    (2, 4, 4, 256, 64, 256, 64, 700),       # MHA, D=256, one value group per token
    (3, 8, 4, 64, 32, 64, 96, 1500),        # D=64, Gv=64
    (2, 8, 2, 64, 32, 32, 64, 1200),        # D=64, G=32, GQA 4 (4 waves per SIMD)
    (2, 4, 2, 64, 32, 32, 64, 900),         # D=64, G=32, GQA 2 (4 waves per SIMD)
    (1, 4, 4, 64, 32, 32, 48, 700),         # D=64, G=32, MHA (4 waves per SIMD)
    (1, 16, 2, 64, 32, 32, 64, 800),        # D=64, G=32, GQA 8
    (1, 16, 2, 256, 64, 64, 128, 1500),     # GQA 8, D=256, G=64, Gv=64: two 4-head launches
    (2, 16, 2, 256, 64, 128, 128, 900),     # GQA 8, D=256, G=64, Gv=128: two 4-head launches
    (1, 12, 2, 256, 64, 128, 128, 900),     # GQA 6, D=256, G=64, Gv=128: 4 + 2 heads
])
def test_attention_matrix_core_shapes(store_cls, B, Hq, Hkv, D, G, Gv, R, T):
    """Every matrix-core instantiation family against float64 attention."""
    st_layout = store_cls(1, 1, D, G, R, "cuda:0", group_size_v=Gv).code_layout
    assert st_layout == 1
    _attention_case(store_cls, B, Hq, Hkv, D, G, Gv, R, T, seed=7)


def test_attention_outlier_heavy_scores(store_cls):
    """Large query norms make the softmax nearly one-hot and exercise the
    running-maximum rescale path (scores jump by far more than 8 in log2)."""
    B, Hq, Hkv, D, G, R, T = 1, 8, 2, 128, 32, 64, 900
    k, v = make_kv(B, Hkv, T, D, seed=41)
    k[:, :, 700] *= 6.0                       # a late, dominant key
    st = store_cls(B, Hkv, D, G, R, "cuda:0")
    fill_store(st, k, v, R)
    q = seeded_q(B, Hq, D, seed=43) * 40.0
    out = st.attention(q.cuda())
    torch.cuda.synchronize()
    kh, vh = oracle_history(k, v, st.n_chunks, G, G)
    q0 = st.n_chunks * G
    ref = decode_attention(q.numpy(), kh, vh, k[:, :, q0:].numpy(), v[:, :, q0:].numpy())
    err = rel_err(out.cpu().numpy(), ref)
    print(f"[attn] outlier-heavy rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL


def test_split_workspace_reuse(store_cls):
    """Split launches merge their partials in a second kernel.  On one
    workspace, calls with different split counts, interleaved with a smaller
    store's calls, give the oracle's result every time and the same bits
    for the same split count."""
    B, Hq, Hkv, D, G, R, T = 2, 8, 2, 128, 32, 128, 2000
    k, v = make_kv(B, Hkv, T, D, seed=21)
    st = store_cls(B, Hkv, D, G, R, "cuda:0")
    fill_store(st, k, v, R)
    small = store_cls(1, Hkv, D, G, R, "cuda:0")
    fill_store(small, k[:1, :, :700], v[:1, :, :700], R)
    q = seeded_q(B, Hq, D, seed=22).cuda()
    kh, vh = oracle_history(k, v, st.n_chunks, G, G)
    q0 = st.n_chunks * G
    ref = decode_attention(q.cpu().numpy(), kh, vh, k[:, :, q0:].numpy(), v[:, :, q0:].numpy())
    ws = torch.empty(1 << 22, dtype=torch.uint8, device="cuda:0")
    first = None
    for splits in (7, 3, 64, 7, 2, 7):
        out = st.attention(q, num_splits=splits, workspace=ws)
        small.attention(q[:1], num_splits=5, workspace=ws)
        o = out.cpu().numpy()
        assert rel_err(o, ref) <= ATTN_TOL
        if splits == 7:
            if first is None:
                first = o.copy()
            assert np.array_equal(o.view(np.uint32), first.view(np.uint32))


def test_split_merge_head_dim_96_negative_scores(store_cls):
    """head_dim 96 (a plain-layout store: the generic kernel) with forced
    splits: the merge kernel's blocks are whole waves, so its (m, l)
    reduction is right even when every split's maximum score lies far below
    zero (here about -160 in log2 units), where a partial wave's inactive
    lanes used to pull the maximum up to 0 and every weight underflowed."""
    B, Hq, Hkv, D, G, R, T = 1, 2, 2, 96, 32, 32, 300
    k, v = make_kv(B, Hkv, T, D, seed=96)
    k = k.abs() + 5.0                                 # every key component positive
    st = store_cls(B, Hkv, D, G, R, "cuda:0")
    assert st.code_layout == 0
    fill_store(st, k, v, R)
    q = torch.full((B, Hq, D), -2.0)                  # scores ~ -2 * sum(k) / sqrt(D)
    kh, vh = oracle_history(k, v, st.n_chunks, G, G)
    q0 = st.n_chunks * G
    ref = decode_attention(q.numpy(), kh, vh, k[:, :, q0:].numpy(), v[:, :, q0:].numpy())
    for splits in (4, 7):
        out = st.attention(q.cuda(), num_splits=splits).cpu().numpy()
        assert np.isfinite(out).all()
        err = rel_err(out, ref)
        print(f"[attn] D=96 negative scores, {splits} splits: rel_err={err:.3e}", flush=True)
        assert err <= ATTN_TOL


def test_store_on_device_without_index(store_cls):
    """A store made with ``device="cuda"`` is on the current device by index,
    so queries on that device (``cuda:0``) are its own: decode and
    multi-token attention give the bits of a store made with ``"cuda:0"``."""
    B, Hq, Hkv, D, G, R, T = 2, 8, 2, 64, 32, 64, 300
    print("[attn] store on device 'cuda'", flush=True)
    k, v = make_kv(B, Hkv, T, D, seed=31)
    plain = store_cls(B, Hkv, D, G, R, "cuda")
    named = store_cls(B, Hkv, D, G, R, "cuda:0")
    assert plain.device == torch.device("cuda", torch.cuda.current_device())
    fill_store(plain, k, v, R)
    fill_store(named, k, v, R)
    q = seeded_q(B, Hq, D, seed=32).cuda()
    assert torch.equal(plain.attention(q), named.attention(q))
    q3 = torch.randn(B, Hq, 3, D, generator=torch.Generator().manual_seed(33)).cuda()
    assert torch.equal(plain.attention(q3), named.attention(q3))


@pytest.mark.parametrize("B,T,splits", [(8, 4096, 4), (12, 8192, 4), (24, 8192, 2)])
def test_attention_mid_batch_plans(store_cls, B, T, splits):
    """Mid batches at config 4's heads run the split plan's middle ground:
    256 workgroups with 8 chunks per wave (B=8, 4K context), 384 with 16
    (B=12, 8K: one wave per workgroup takes the window) and 384 with 32 (B=24,
    8K), each split merged; the automatic plan's split count is the one
    stated, and the output matches the float64 oracle at 1e-3."""
    Hq, Hkv, D, G, R = 32, 8, 128, 32, 128
    k, v = make_kv(B, Hkv, T, D, seed=T + B)
    st = store_cls(B, Hkv, D, G, R, "cuda:0", chunk_capacity=T // G + 1)
    st.extend(k.cuda(), v.cuda(), flush_at=R)
    ws = st.workspace_bytes(Hq)
    assert ws == B * Hkv * 4 * splits * (D + 2) * 4
    print(f"[attn] mid batch B={B} T={T}: chunks={st.n_chunks} res={st.res_len} "
          f"splits={splits}", flush=True)
    q = seeded_q(B, Hq, D, seed=B)
    out = st.attention(q.cuda())
    torch.cuda.synchronize()
    kh, vh = oracle_history(k, v, st.n_chunks, G, G)
    q0 = st.n_chunks * G
    ref = decode_attention(q.numpy(), kh, vh, k[:, :, q0:].numpy(), v[:, :, q0:].numpy())
    err = rel_err(out.cpu().numpy(), ref)
    print(f"[attn]   rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL
