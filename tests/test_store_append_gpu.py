"""GPU checks of the residual append: the one-launch append kernel, and the
attention launch that appends the step's new token itself
(kivi_packed_decode_attention_append, replacing the residual append of
src/kivi_sycl/cache/manager.py:226-231 together with the step's attention).

Bars: ring contents bit-exact; the fused launch's output bit-identical to a
separate append followed by attention, and within 1e-3 of float64 attention
over the oracle-dequantised history."""

import numpy as np
import pytest
import torch

from oracle.attention import decode_attention
from tests.kv_helpers import fill_store, make_kv, oracle_history, rel_err, seeded_q

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def store_cls(hip_device):
    from intel_kivi_hybrid_amd.store import PackedKVStore
    return PackedKVStore


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_append_kernel_writes_the_ring(store_cls, dtype):
    """Append 1..R tokens (strided views, wrapping the ring) and compare the
    window with the widened inputs."""
    B, H, D, G, R = 2, 3, 64, 32, 48
    st = store_cls(B, H, D, G, R, "cuda:0")
    k, v = make_kv(B, H, 300, D, seed=1)
    kb = k.transpose(1, 2).contiguous().transpose(1, 2).to(dtype).cuda()   # [B,H,T,D] view
    vb = v.transpose(1, 2).contiguous().transpose(1, 2).to(dtype).cuda()
    t = 0
    for n in (5, 1, 17, 3, 22):
        st.append(kb[:, :, t:t + n], vb[:, :, t:t + n])
        t += n
        if st.res_len >= 32:
            st.flush()
        rk, rv = st.residual()
        q0 = st.quantized_tokens
        assert torch.equal(rk.cpu(), kb[:, :, q0:t].float().cpu())
        assert torch.equal(rv.cpu(), vb[:, :, q0:t].float().cpu())


CASES = [
    # B, Hq, Hkv, D, G, Gv, R, T, splits
    (2, 8, 2, 128, 32, 32, 64, 300, 0),      # matrix-core kernel, one split
    (1, 8, 8, 128, 32, 128, 64, 1000, 4),    # several splits (partials + merge)
    (2, 8, 1, 64, 32, 32, 48, 200, 0),       # 8 query heads per kv head
    (1, 4, 2, 32, 16, 16, 32, 100, 0),       # plain code order: generic kernel
    (2, 4, 4, 64, 32, 32, 64, 64, 0),        # window of 32 tokens after the flush at T = R
]


@pytest.mark.parametrize("B,Hq,Hkv,D,G,Gv,R,T,splits", CASES)
def test_fused_append_attention(store_cls, B, Hq, Hkv, D, G, Gv, R, T, splits):
    print(f"[append] B={B} Hq={Hq} Hkv={Hkv} D={D} G={G} Gv={Gv} R={R} T={T} splits={splits}",
          flush=True)
    k, v = make_kv(B, Hkv, T + 3, D, seed=T + D)
    a = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    b = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    fill_store(a, k[:, :, :T], v[:, :, :T], R)
    fill_store(b, k[:, :, :T], v[:, :, :T], R)
    for step in range(3):
        kn = k[:, :, T + step:T + step + 1].cuda()
        vn = v[:, :, T + step:T + step + 1].cuda()
        q = seeded_q(B, Hq, D, seed=step).cuda()
        a.stage_token(kn, vn)                      # written by the attention launch
        oa = a.attention(q, num_splits=splits).clone()
        b.append(kn, vn)                           # separate append, then attention
        ob = b.attention(q, num_splits=splits).clone()
        assert torch.equal(oa, ob), f"step {step}"
        assert a._pending is None and a.res_len == b.res_len
        for x, y in zip(a.residual(), b.residual()):
            assert torch.equal(x, y)
        kh, vh = oracle_history(k, v, a.n_chunks, G, Gv)
        rk, rv = a.residual()
        ref = decode_attention(q.cpu().numpy(), kh, vh, rk.cpu().numpy(), rv.cpu().numpy())
        err = rel_err(oa.cpu().numpy(), ref)
        print(f"[append] step {step} rel_err={err:.2e}", flush=True)
        assert err <= 1e-3


def test_staged_token_is_committed_before_other_uses(store_cls):
    """A staged token counts at once; flushing, appending or reading the
    window before any attention writes it into the ring first."""
    B, H, D, G, R = 1, 2, 64, 32, 33
    k, v = make_kv(B, H, 40, D, seed=3)
    st = store_cls(B, H, D, G, R, "cuda:0")
    st.append(k[:, :, :32].cuda(), v[:, :, :32].cuda())
    st.stage_token(k[:, :, 32:33].cuda(), v[:, :, 32:33].cuda())
    assert st.res_len == 33 and st._pending is not None
    st.flush()                                     # reads tokens 0..31: commits token 32 first
    assert st._pending is None
    rk, rv = st.residual()
    assert torch.equal(rk.cpu(), k[:, :, 32:33]) and torch.equal(rv.cpu(), v[:, :, 32:33])
    st.stage_token(k[:, :, 33:34].cuda(), v[:, :, 33:34].cuda())
    st.append(k[:, :, 34:40].cuda(), v[:, :, 34:40].cuda())
    rk, _ = st.residual()
    assert torch.equal(rk.cpu(), k[:, :, 32:40])
    # non-fp32 or unaligned tokens take the separate append at once
    st.stage_token(k[:, :, 0:1].to(torch.bfloat16).cuda(), v[:, :, 0:1].to(torch.bfloat16).cuda())
    assert st._pending is None and st.res_len == 9


@pytest.mark.parametrize("ring,src", [(torch.float32, torch.float32),
                                      (torch.float32, torch.bfloat16),
                                      (torch.bfloat16, torch.bfloat16)])
def test_append_layers_matches_per_layer_appends(store_cls, ring, src):
    """One step's tokens for 20 layers (two launches of the multi-layer
    append: 16 + 4 layers), from strided views like a DynamicCache's, into
    rings at different positions, equal bit for bit the per-layer appends;
    a layer whose input has another type is appended on its own."""
    from intel_kivi_hybrid_amd.store import append_layers
    L, B, H, D, G, R = 20, 2, 3, 64, 32, 48
    print(f"[append] {L} layers, ring {ring}, new tokens {src}", flush=True)
    a = [store_cls(B, H, D, G, R, "cuda:0", residual_dtype=ring) for _ in range(L)]
    b = [store_cls(B, H, D, G, R, "cuda:0", residual_dtype=ring) for _ in range(L)]
    for i in range(L):                       # windows at different fill levels and starts
        k, v = make_kv(B, H, 20 + 3 * i, D, seed=i)
        for st in (a[i], b[i]):
            st.extend(k.to(ring).cuda(), v.to(ring).cuda(), flush_at=R)
    ks, vs = [], []
    for i in range(L):
        k, v = make_kv(B, H, 40, D, seed=100 + i)     # a cache of 40 tokens; the step's
        kc = k.transpose(1, 2).contiguous().transpose(1, 2).to(src).cuda()
        vc = v.transpose(1, 2).contiguous().transpose(1, 2).to(src).cuda()
        ks.append(kc[:, :, -1:])                      # newest token, a strided view
        vs.append(vc[:, :, -1:])
    ks[7] = ks[7].float() if src != torch.float32 else ks[7].half()   # not batchable:
    vs[7] = vs[7].float() if src != torch.float32 else vs[7].half()   # appended alone
    if ring != torch.float32:
        ks[7], vs[7] = ks[7].to(ring), vs[7].to(ring)
    append_layers(a, ks, vs)
    for st, k, v in zip(b, ks, vs):
        st.append(k, v)
    torch.cuda.synchronize()
    for i in range(L):
        assert (a[i].res_start, a[i].res_len) == (b[i].res_start, b[i].res_len)
        assert torch.equal(a[i].k_res, b[i].k_res) and torch.equal(a[i].v_res, b[i].v_res), i
