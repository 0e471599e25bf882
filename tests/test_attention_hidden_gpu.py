"""GPU parity of attention over the packed store for any key-padding pattern
(right padding, holes, hidden runs across splits): position p of sequence b
is hidden from every query token where HF's 2-D attention mask is 0,
through kivi_packed_attention_masked's hidden-position bits.  Against the
float64 oracle with the same visibility (oracle.attention, pinned against
SDPA with HF's boolean mask).  Bar: 1e-3 relative (max |o - o_ref| /
max |o_ref| per row); rows that see no position are zeros in both.

The reference hands any such mask to HF attention over the dequantised
cache (src/kivi_sycl/generation/generate.py:76,
src/kivi_sycl/cache/manager.py:251-290)."""

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


def _pattern(kind, B, T, L, seed):
    """Visibility [B, T] (True = attended); the L newest positions (the query
    tokens) stay visible except where a case hides one on purpose."""
    rng = np.random.default_rng(seed)
    vis = np.ones((B, T), bool)
    if kind == "holes":
        vis = rng.random((B, T)) > 0.3
    elif kind == "right":                      # pad positions between prompt and new tokens
        for b in range(B):
            lo = T // (b + 2)
            vis[b, lo:lo + (T - L - lo) * (b + 1) // (B + 1)] = False
    elif kind == "runs":                       # whole splits hidden, then a long run
        vis[0, :int(T * 0.7)] = False
        vis[1 % B, int(T * 0.2):int(T * 0.9)] = False
        vis[2 % B] = rng.random(T) > 0.5
    vis[:, T - L:] = True
    return vis


CASES = [
    # B, Hq, Hkv, D, G, Gv, R, T, L, splits, pattern
    (4, 8, 2, 128, 32, 32, 128, 900, 1, 0, "holes"),
    (4, 8, 2, 128, 32, 32, 128, 900, 3, 0, "right"),       # three causal query tokens
    (3, 32, 8, 128, 32, 32, 128, 2000, 1, 7, "runs"),      # splits, whole splits hidden
    (2, 4, 4, 64, 32, 32, 64, 700, 2, 0, "holes"),         # D=64, MHA
    (2, 16, 2, 128, 32, 128, 128, 3000, 1, 1, "right"),    # one split, Gv = D
    (2, 8, 2, 128, 64, 64, 128, 1500, 1, 0, "holes"),      # G=64: two words per chunk
    (2, 64, 8, 128, 32, 32, 128, 1200, 1, 0, "runs"),      # 8 query heads per kv head
    (2, 2, 2, 64, 16, 16, 32, 200, 1, 0, "holes"),         # plain layout (generic)
    (2, 8, 2, 64, 16, 16, 32, 200, 4, 3, "right"),         # generic, multi-token, splits
    (2, 8, 2, 128, 32, 32, 128, 100, 1, 0, "holes"),       # no chunk yet: window pass
    (2, 8, 2, 128, 32, 32, 128, 100, 3, 0, "right"),       # the same, 3 query tokens
    (1, 8, 2, 128, 32, 32, 128, 12300, 1, 1, "holes"),     # one split: > 64 chunks per wave
]


def _run(st, q, L, splits, key_mask=None, **kw):
    qq = q[:, :, 0].cuda() if L == 1 else q.cuda()
    return st.attention(qq, num_splits=splits, key_mask=key_mask, **kw)


def _ref(st, k, v, q, L, G, Gv, vis):
    kh, vh = oracle_history(k, v, st.n_chunks, G, Gv)
    q0 = st.n_chunks * G
    kr, vr = k[:, :, q0:].numpy(), v[:, :, q0:].numpy()
    if L == 1:
        return decode_attention(q[:, :, 0].numpy(), kh, vh, kr, vr, visible=vis)
    return prefix_attention(q.transpose(1, 2).numpy(), kh, vh, kr, vr, visible=vis)


@pytest.mark.parametrize("B,Hq,Hkv,D,G,Gv,R,T,L,splits,pattern", CASES)
def test_hidden_positions_match_oracle(store_cls, B, Hq, Hkv, D, G, Gv, R, T, L, splits,
                                       pattern):
    print(f"[hidden] B={B} Hq={Hq} Hkv={Hkv} D={D} G={G} Gv={Gv} R={R} T={T} L={L} "
          f"splits={splits} {pattern}", flush=True)
    k, v = make_kv(B, Hkv, T, D, seed=T + L + 3)
    st = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    fill_store(st, k, v, R)
    g = torch.Generator().manual_seed(D + L + 1)
    q = torch.randn(B, Hq, L, D, generator=g) * D ** -0.5
    vis = _pattern(pattern, B, T, L, seed=T)
    out = _run(st, q, L, splits, key_mask=torch.from_numpy(vis))
    torch.cuda.synchronize()
    ref = _ref(st, k, v, q, L, G, Gv, vis)
    err = rel_err(out.cpu().numpy(), ref)
    print(f"[hidden]   chunks={st.n_chunks} res={st.res_len} hidden={int((~vis).sum())} "
          f"rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL
    # packed words once for many calls give the same bits; all visible is
    # the unmasked launch
    from intel_kivi_hybrid_amd import _C
    words = _C.hidden_positions(torch.from_numpy(vis), "cuda:0")
    assert torch.equal(_run(st, q, L, splits, hidden=words), out)
    ones = torch.ones(B, T, dtype=torch.bool)
    assert torch.equal(_run(st, q, L, splits, key_mask=ones), _run(st, q, L, splits))


@pytest.mark.parametrize("L,splits", [(1, 0), (1, 5), (3, 0)])
def test_leading_run_equals_kv_start(store_cls, L, splits):
    """Hidden bits of a left-padded batch give the kv_start launch's bits."""
    B, Hq, Hkv, D, G, R, T = 3, 16, 4, 128, 32, 128, 1400
    print(f"[hidden] leading runs L={L} splits={splits}", flush=True)
    k, v = make_kv(B, Hkv, T, D, seed=5)
    st = store_cls(B, Hkv, D, G, R, "cuda:0")
    fill_store(st, k, v, R)
    q = torch.randn(B, Hq, L, D, generator=torch.Generator().manual_seed(6)) * D ** -0.5
    starts = [0, 333, T - R + 5]
    vis = np.arange(T)[None, :] >= np.array(starts)[:, None]
    a = _run(st, q, L, splits, key_mask=torch.from_numpy(vis))
    b = _run(st, q, L, splits, kv_start=starts)
    assert torch.equal(a, b)


@pytest.mark.parametrize("splits", [0, 4])
def test_fully_hidden_rows_are_zero(store_cls, splits):
    """A sequence with every position hidden gets zeros; the others are
    unaffected (bit for bit)."""
    B, Hq, Hkv, D, G, R, T = 3, 8, 2, 128, 32, 64, 700
    print(f"[hidden] fully hidden sequence, splits={splits}", flush=True)
    k, v = make_kv(B, Hkv, T, D, seed=7)
    st = store_cls(B, Hkv, D, G, R, "cuda:0")
    fill_store(st, k, v, R)
    q = (torch.randn(B, Hq, D, generator=torch.Generator().manual_seed(8)) * D ** -0.5).cuda()
    vis = torch.ones(B, T, dtype=torch.bool)
    vis[1] = False
    out = st.attention(q, num_splits=splits, key_mask=vis)
    assert torch.isfinite(out).all() and not out[1].any()
    plain = st.attention(q, num_splits=splits)
    assert torch.equal(out[0], plain[0]) and torch.equal(out[2], plain[2])


def test_hidden_positions_bf16_ring(store_cls):
    """The 16-bit-ring kernels apply the bits the same way."""
    B, Hq, Hkv, D, G, R, T = 2, 32, 8, 128, 32, 128, 1100
    print("[hidden] bf16 ring", flush=True)
    k, v = make_kv(B, Hkv, T, D, seed=9)
    k, v = k.bfloat16().float(), v.bfloat16().float()     # values the ring holds exactly
    st = store_cls(B, Hkv, D, G, R, "cuda:0", residual_dtype=torch.bfloat16)
    fill_store(st, k, v, R)
    q = torch.randn(B, Hq, 1, D, generator=torch.Generator().manual_seed(10)) * D ** -0.5
    vis = _pattern("holes", B, T, 1, seed=11)
    out = _run(st, q, 1, 0, key_mask=torch.from_numpy(vis))
    ref = _ref(st, k, v, q, 1, G, G, vis)
    err = rel_err(out.cpu().numpy(), ref)
    print(f"[hidden]   rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL


def test_hidden_positions_checked_on_host(store_cls):
    B, Hkv, D, G, R = 2, 2, 64, 32, 64
    k, v = make_kv(B, Hkv, 100, D, seed=1)
    st = store_cls(B, Hkv, D, G, R, "cuda:0")
    fill_store(st, k, v, R)
    q = torch.randn(B, 4, D).cuda()
    with pytest.raises(RuntimeError, match="key_mask"):
        st.attention(q, key_mask=torch.ones(B, 99, dtype=torch.bool))     # one position short
    with pytest.raises(RuntimeError, match="hidden"):
        st.attention(q, hidden=torch.zeros(B, 3, dtype=torch.int64, device="cuda:0"))
    with pytest.raises(RuntimeError, match="hidden"):
        st.attention(q, hidden=torch.zeros(B, 3, dtype=torch.int32, device="cuda:0")[:, :1])
