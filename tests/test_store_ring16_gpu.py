"""GPU checks of the 16-bit residual ring: a store whose ring holds bf16 or
fp16 K/V (what a half-precision model produces) against a store with an fp32
ring fed the same values.  The kernels widen 16-bit elements exactly, so the
two must agree bit for bit: codes, scales, zeros and history of every chunk,
the residual window, and every decode-attention output (fused append, split
partials, flushes through the ring and across ring and new tokens).  The fp32
ring itself is held to the oracle by the other store tests.

Replaces, for half-precision models, the fp32 residual of
src/kivi_sycl/cache/manager.py:226-231 (a torch.cat of the model's K/V
widened to fp32)."""

import pytest
import torch

from tests.kv_helpers import make_kv, seeded_q

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def store_cls(hip_device):
    from intel_kivi_hybrid_amd.store import PackedKVStore
    return PackedKVStore


CASES = [
    # B, Hq, Hkv, D, G, Gv, R, prompt, steps, splits
    (2, 8, 2, 128, 32, 128, 64, 150, 70, 0),    # fast flush + matrix-core attention
    (1, 8, 8, 128, 32, 32, 96, 500, 40, 4),     # split partials + merge
    (1, 4, 2, 256, 64, 64, 128, 300, 70, 0),    # untiled generic flush (G*D > tile)
    (2, 4, 2, 128, 16, 16, 32, 90, 40, 0),      # plain code order: generic kernels
    (2, 8, 2, 64, 32, 32, 64, 150, 70, 0),      # D=64, G=32 (4 waves per SIMD)
]


def _same(a, b, what):
    assert a.dtype == b.dtype and a.shape == b.shape, what
    assert torch.equal(a, b), what


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,Hq,Hkv,D,G,Gv,R,P,steps,splits", CASES)
def test_ring16_matches_fp32_ring(store_cls, dtype, B, Hq, Hkv, D, G, Gv, R, P, steps, splits):
    print(f"[ring16] {dtype} B={B} Hq={Hq} Hkv={Hkv} D={D} G={G} Gv={Gv} R={R} P={P} "
          f"steps={steps} splits={splits}", flush=True)
    k, v = make_kv(B, Hkv, P + steps, D, seed=D + G)
    kh, vh = k.to(dtype).cuda(), v.to(dtype).cuda()
    a = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv, keep_history=True)
    b = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv, keep_history=True,
                  residual_dtype=dtype)
    assert b.k_res.dtype == dtype and b.res_dtype_code in (1, 2)
    # prompt: one batched flush reading the new tokens (and, below, the ring)
    fa = a.extend(kh[:, :, :P], vh[:, :, :P], flush_at=R)
    fb = b.extend(kh[:, :, :P], vh[:, :, :P], flush_at=R)
    assert fa == fb and a.n_chunks == b.n_chunks and a.res_len == b.res_len
    n_prompt = a.n_chunks
    for t in range(P, P + steps):
        a.stage_token(kh[:, :, t:t + 1], vh[:, :, t:t + 1])
        b.stage_token(kh[:, :, t:t + 1], vh[:, :, t:t + 1])
        # the 16-bit ring takes the token inside the attention launch; the
        # fp32 ring, fed another type, by a separate append
        assert b._pending is not None and a._pending is None
        q = seeded_q(B, Hq, D, seed=t).cuda()
        oa = a.attention(q, num_splits=splits)
        ob = b.attention(q, num_splits=splits)
        assert torch.equal(oa, ob), f"attention differs at step {t}"
        while a.res_len >= R:
            a.flush()
            b.flush()
    torch.cuda.synchronize()
    # decode steps flushed through the ring too
    assert a.n_chunks == b.n_chunks and a.n_chunks > n_prompt
    n = a.n_chunks
    for name in ("k_codes", "k_scale", "k_zero", "v_codes", "v_scale", "v_zero"):
        _same(getattr(a, name)[:, :, :n], getattr(b, name)[:, :, :n], name)
    _same(a.k_hist[:, :, :n * G], b.k_hist[:, :, :n * G], "k_hist")
    _same(a.v_hist[:, :, :n * G], b.v_hist[:, :, :n * G], "v_hist")
    ra, rva = a.residual()
    rb, rvb = b.residual()
    assert rb.dtype == dtype
    assert torch.equal(ra, rb.float()) and torch.equal(rva, rvb.float())
    assert torch.equal(rb, kh[:, :, n * G:]) and torch.equal(rvb, vh[:, :, n * G:])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_ring16_rounds_wider_inputs(store_cls, dtype):
    """fp32 K/V fed to a 16-bit ring are rounded to the ring's type before
    anything is quantised, so the store equals one fed the rounded values
    (whether a token is quantised straight from the input or via the ring)."""
    B, H, D, G, R = 2, 2, 128, 32, 64
    k, v = make_kv(B, H, 200, D, seed=3)
    a = store_cls(B, H, D, G, R, "cuda:0", residual_dtype=dtype)
    b = store_cls(B, H, D, G, R, "cuda:0", residual_dtype=dtype)
    a.extend(k.cuda(), v.cuda(), flush_at=R)
    b.extend(k.to(dtype).cuda(), v.to(dtype).cuda(), flush_at=R)
    torch.cuda.synchronize()
    n = a.n_chunks
    assert n == b.n_chunks and n > 0
    for name in ("k_codes", "k_scale", "k_zero", "v_codes", "v_scale", "v_zero"):
        assert torch.equal(getattr(a, name)[:, :, :n], getattr(b, name)[:, :, :n]), name
    assert torch.equal(a.residual()[0], b.residual()[0])


def test_ring16_export_roundtrip(store_cls):
    """export_state keeps the ring's type and from_state restores it."""
    from intel_kivi_hybrid_amd.store import PackedKVStore
    B, H, D, G, R = 1, 2, 128, 32, 64
    k, v = make_kv(B, H, 150, D, seed=5)
    st = store_cls(B, H, D, G, R, "cuda:0", residual_dtype=torch.bfloat16)
    st.extend(k.to(torch.bfloat16).cuda(), v.to(torch.bfloat16).cuda(), flush_at=R)
    ex = st.export_state()
    assert ex["k_residual"].dtype == torch.bfloat16
    st2 = PackedKVStore.from_state(ex, G, R, "cuda:0")
    assert st2.residual_dtype == torch.bfloat16
    q = seeded_q(B, 8, D, seed=1).cuda()
    assert torch.equal(st.attention(q), st2.attention(q))
