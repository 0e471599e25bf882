"""GPU parity of attention for several query tokens per sequence over the
packed store (kivi_packed_attention through PackedKVStore.attention).

* Causal: the L queries are the residual window's last L tokens, and token i
  attends to the quantised history and to the window up to itself -- a
  forward of L tokens on a non-empty cache (chunked prefill, speculative
  verification), HF's causal mask over [cache ; new tokens].  Checked against
  oracle.attention.prefix_attention (float64).
* Non-causal: every query sees the whole cache, the reference's own
  attention check (q_len = 3 over a 32-token cache, B=1, H=2, D=64, G=32;
  tests/integration/test_attention_fix.py:19-43,91-115), against float64
  attention per query and the reference's cosine > 0.85 gate against fp32
  attention over the unquantised cache.

The shapes cover one launch with padding rows, several launches (q_len *
Hq/Hkv > 8 rows), forced splits, the long-context mode where one wave takes
the window, value groups of 128, the plain layout (generic kernel) and a
context held only in the window.  Bar: 1e-3 relative (max |o - o_ref| /
max |o_ref| per (batch, token, head)).
"""

import numpy as np
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
    # B, Hq, Hkv, D, G, Gv, R, T, L, splits
    (2, 8, 2, 128, 32, 32, 128, 600, 3, 0),      # GQA 4: 12 rows -> 2 launches
    (1, 4, 4, 64, 32, 32, 64, 300, 5, 0),        # MHA: 5 tokens in one launch, 3 padding rows
    (2, 16, 2, 128, 32, 32, 128, 900, 2, 3),     # GQA 8: one token per launch, 3 splits
    (1, 8, 2, 128, 32, 128, 128, 2200, 8, 1),    # one split: a wave takes the window, Gv = D
    (1, 2, 2, 64, 16, 16, 32, 100, 4, 0),        # plain layout: the generic kernel
    (2, 8, 2, 64, 32, 32, 64, 40, 3, 0),         # no chunk yet: the window pass alone
    (1, 4, 1, 128, 64, 64, 128, 1300, 6, 4),     # G = 64, GQA 4, 4 splits
    (1, 6, 2, 128, 32, 32, 128, 600, 3, 0),      # GQA 3: 2 tokens per launch, 2 padding rows
    (2, 24, 2, 64, 32, 32, 64, 300, 2, 2),       # GQA 12: head groups of 8 and 4, 2 splits
    (1, 14, 2, 64, 16, 16, 32, 100, 3, 0),       # GQA 7, plain layout: the generic kernel
    (1, 4, 2, 256, 64, 128, 128, 700, 3, 0),     # D=256, G=64, Gv=128: at most 4 rows per launch
]


@pytest.mark.parametrize("B,Hq,Hkv,D,G,Gv,R,T,L,splits", CASES)
def test_causal_queries_match_oracle(store_cls, B, Hq, Hkv, D, G, Gv, R, T, L, splits):
    print(f"[multi] B={B} Hq={Hq} Hkv={Hkv} D={D} G={G} Gv={Gv} R={R} T={T} L={L} "
          f"splits={splits}", flush=True)
    k, v = make_kv(B, Hkv, T, D, seed=T + L)
    st = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    fill_store(st, k, v, R)
    assert st.res_len >= L
    g = torch.Generator().manual_seed(L + D)
    q = torch.randn(B, Hq, L, D, generator=g) * D ** -0.5          # HF layout
    out = st.attention(q.cuda(), num_splits=splits)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (B, L, Hq, D)
    kh, vh = oracle_history(k, v, st.n_chunks, G, Gv)
    q0 = st.n_chunks * G
    ref = prefix_attention(q.transpose(1, 2).numpy(), kh, vh, k[:, :, q0:].numpy(),
                           v[:, :, q0:].numpy())
    err = rel_err(out.cpu().numpy(), ref)
    print(f"[multi]   chunks={st.n_chunks} res={st.res_len} rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL
    # the newest token sees everything: it equals a one-token decode of it
    last = st.attention(q[:, :, -1].contiguous().cuda(), num_splits=splits).cpu().numpy()
    assert rel_err(last, ref[:, -1]) <= ATTN_TOL


def test_reference_q3_geometry_noncausal(store_cls, kat):
    """The reference's attention check (test_attention_fix.py:19-115): B=1,
    H=2, three query tokens over a cache of 32 tokens (one group), D=64,
    G=32, seed 42; every query sees the whole cache.  Against float64
    attention over the oracle-dequantised cache (1e-3), and the reference's
    own gate: cosine > 0.85 against fp32 attention over the unquantised
    cache."""
    gate = kat["attention_cosine_gate"]
    B, H, T, D, G = gate["B"], gate["H"], gate["cache_len"], gate["D"], gate["G"]
    torch.manual_seed(42)
    q = torch.randn(B, H, 3, D)
    k = torch.randn(B, H, T, D)
    v = torch.randn(B, H, T, D)
    st = store_cls(B, H, D, G, G, "cuda:0")
    fill_store(st, k, v, G)
    assert st.n_chunks == 1 and st.res_len == 0
    out = st.attention(q.cuda(), causal=False).cpu().double()           # [B, 3, H, D]
    kh, vh = oracle_history(k, v, 1, G, G)
    ref = np.stack([decode_attention(q[:, :, i].numpy(), kh, vh, None, None) for i in range(3)],
                   axis=1)
    err = rel_err(out.numpy(), ref)
    fp32 = torch.softmax(q @ k.transpose(-2, -1) * D ** -0.5, dim=-1) @ v   # [B, H, 3, D]
    cos = torch.nn.functional.cosine_similarity(out.transpose(1, 2).reshape(1, -1),
                                                fp32.double().reshape(1, -1)).item()
    print(f"[multi] reference geometry: rel_err={err:.3e} cosine vs fp32 = {cos:.4f}", flush=True)
    assert err <= ATTN_TOL
    assert cos > gate["min_cosine"]


def test_multitoken_after_staged_token(store_cls):
    """A staged decode token (counted, not yet in the ring) is committed before
    a multi-token launch, which reads the ring only."""
    B, Hq, Hkv, D, G, R, T = 1, 8, 2, 128, 32, 64, 300
    k, v = make_kv(B, Hkv, T + 1, D, seed=5)
    st = store_cls(B, Hkv, D, G, R, "cuda:0")
    fill_store(st, k[:, :, :T], v[:, :, :T], R)
    st.stage_token(k[:, :, T:].cuda(), v[:, :, T:].cuda())
    q = torch.randn(B, Hq, 2, D, generator=torch.Generator().manual_seed(6)) * D ** -0.5
    out = st.attention(q.cuda())
    kh, vh = oracle_history(k, v, st.n_chunks, G, G)
    q0 = st.n_chunks * G
    ref = prefix_attention(q.transpose(1, 2).numpy(), kh, vh, k[:, :, q0:].numpy(),
                           v[:, :, q0:].numpy())
    assert rel_err(out.cpu().numpy(), ref) <= ATTN_TOL
