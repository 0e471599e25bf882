"""GPU parity of attention over the packed store for a left-padded batch:
sequence b attends to context positions kv_start[b] onward only (HF's
attention mask hides its leading pad positions), through
kivi_packed_attention's kv_start.  Against the float64 oracle with the same
kv_start (oracle.attention, pinned against SDPA with HF's boolean mask).
Bar: 1e-3 relative (max |o - o_ref| / max |o_ref| per row)."""

import pytest
import torch

from oracle.attention import decode_attention, prefix_attention
from tests.kv_helpers import fill_store, make_kv, oracle_history, rel_err

pytestmark = pytest.mark.gpu

ATTN_TOL = 1e-3


@pytest.fixture(scope="module")
def store_cls(hip_device):
    from intel_kivi_hybrid_amd.store import PackedKVStore
    return PackedKVStore


CASES = [
    # B, Hq, Hkv, D, G, Gv, R, T, L, splits, starts (as fractions of T, then clamped)
    (4, 8, 2, 128, 32, 32, 128, 900, 1, 0, (0, 31, 32, 850)),        # in a chunk, on a
    (4, 8, 2, 128, 32, 32, 128, 900, 3, 0, (5, 64, 200, 790)),       # boundary, in the window
    (3, 32, 8, 128, 32, 32, 128, 2000, 1, 7, (0, 1500, 1900)),       # splits, whole splits hidden
    (2, 4, 4, 64, 32, 32, 64, 700, 2, 0, (100, 660)),                # D=64, MHA
    (2, 16, 2, 128, 32, 128, 128, 3000, 1, 1, (2500, 17)),           # one split, Gv = D
    (2, 2, 2, 64, 16, 16, 32, 200, 1, 0, (7, 170)),                  # plain layout (generic)
    (2, 8, 2, 64, 16, 16, 32, 200, 4, 3, (0, 150)),                  # generic, multi-token, splits
    (2, 8, 2, 128, 32, 32, 128, 100, 1, 0, (0, 60)),                 # no chunk yet: window pass
    (2, 8, 2, 128, 32, 32, 128, 100, 3, 0, (5, 90)),                 # the same, 3 query tokens
]


@pytest.mark.parametrize("B,Hq,Hkv,D,G,Gv,R,T,L,splits,starts", CASES)
def test_padded_attention_matches_oracle(store_cls, B, Hq, Hkv, D, G, Gv, R, T, L, splits,
                                         starts):
    print(f"[padded] B={B} Hq={Hq} Hkv={Hkv} D={D} G={G} Gv={Gv} R={R} T={T} L={L} "
          f"splits={splits} starts={starts}", flush=True)
    k, v = make_kv(B, Hkv, T, D, seed=T + L + 1)
    st = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    fill_store(st, k, v, R)
    assert max(starts) <= T - L
    g = torch.Generator().manual_seed(D + L)
    q = torch.randn(B, Hq, L, D, generator=g) * D ** -0.5
    kh, vh = oracle_history(k, v, st.n_chunks, G, Gv)
    q0 = st.n_chunks * G
    kr, vr = k[:, :, q0:].numpy(), v[:, :, q0:].numpy()
    if L == 1:
        out = st.attention(q[:, :, 0].cuda(), num_splits=splits, kv_start=list(starts))
        ref = decode_attention(q[:, :, 0].numpy(), kh, vh, kr, vr, kv_start=starts)
    else:
        out = st.attention(q.cuda(), num_splits=splits, kv_start=list(starts))
        ref = prefix_attention(q.transpose(1, 2).numpy(), kh, vh, kr, vr, kv_start=starts)
    torch.cuda.synchronize()
    err = rel_err(out.cpu().numpy(), ref)
    print(f"[padded]   chunks={st.n_chunks} res={st.res_len} rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL
    # a device tensor of starts gives the same bits, and all-zero starts the unpadded result
    dev = torch.tensor(starts, dtype=torch.int32, device="cuda:0")
    qq = q[:, :, 0].cuda() if L == 1 else q.cuda()
    again = st.attention(qq, num_splits=splits, kv_start=dev)
    assert torch.equal(again, out)
    zero = st.attention(qq, num_splits=splits, kv_start=[0] * B)
    assert torch.equal(zero, st.attention(qq, num_splits=splits))


def test_padded_decode_after_staged_token(store_cls):
    """The staged decode token is committed before a padded launch (which
    goes through kivi_packed_attention rather than the fused append)."""
    B, Hq, Hkv, D, G, R, T = 2, 8, 2, 128, 32, 64, 300
    k, v = make_kv(B, Hkv, T + 1, D, seed=8)
    st = store_cls(B, Hkv, D, G, R, "cuda:0")
    fill_store(st, k[:, :, :T], v[:, :, :T], R)
    st.stage_token(k[:, :, T:].cuda(), v[:, :, T:].cuda())
    q = torch.randn(B, Hq, D, generator=torch.Generator().manual_seed(9)) * D ** -0.5
    out = st.attention(q.cuda(), kv_start=[40, 3])
    kh, vh = oracle_history(k, v, st.n_chunks, G, G)
    q0 = st.n_chunks * G
    ref = decode_attention(q.numpy(), kh, vh, k[:, :, q0:].numpy(), v[:, :, q0:].numpy(),
                           kv_start=(40, 3))
    assert rel_err(out.cpu().numpy(), ref) <= ATTN_TOL


def test_kv_start_checked_on_host(store_cls):
    B, Hkv, D, G, R = 2, 2, 64, 32, 64
    k, v = make_kv(B, Hkv, 100, D, seed=1)
    st = store_cls(B, Hkv, D, G, R, "cuda:0")
    fill_store(st, k, v, R)
    q = torch.randn(B, 4, D).cuda()
    with pytest.raises(RuntimeError, match="kv_start"):
        st.attention(q, kv_start=[0, 100])          # hides the whole context
    with pytest.raises(RuntimeError, match="kv_start"):
        st.attention(q, kv_start=[0])               # one start for two sequences
