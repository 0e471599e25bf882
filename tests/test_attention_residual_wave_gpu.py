"""GPU parity of the matrix-core attention when one wave per workgroup takes
the whole residual window (long contexts: >= 16 chunks per wave), against
float64 attention over the oracle-dequantised cache plus the residual.

The launch plan (kivi_attention.hip, make_plan) picks this mode when the
store has a residual window and each wave has >= 16 chunks.  With a forced
split count S, a wave gets ceil(n_chunks / (4 S)) chunks.  The shapes below
are chosen so that it holds.
  * One split: the last wave takes every 16-token pass while the other three
    take extra chunks up front.
  * Four splits: the passes are spread over the splits' last waves, one
    split taking fewer, so the up-front chunks differ per split.
  * A window of one token, the fused append (bit-identical to a separate
    append), and GQA ratios 1, 4 and 8.
  * A decode that starts with the whole context in the window (generic
    kernel) and crosses its first flush onto the matrix-core kernel.
Bar: 1e-3 relative (max |o - o_ref| / max |o_ref| per (batch, head))."""

import pytest
import torch

from oracle.attention import decode_attention
from tests.kv_helpers import fill_store, make_kv, oracle_history, rel_err, seeded_q

pytestmark = pytest.mark.gpu

ATTN_TOL = 1e-3


@pytest.fixture(scope="module")
def store_cls(hip_device):
    from intel_kivi_hybrid_amd.store import PackedKVStore
    return PackedKVStore


def _chunks_per_wave(n_chunks, splits):
    return -(-n_chunks // (4 * splits))


def _check(st, k, v, q, out, G, Gv):
    kh, vh = oracle_history(k, v, st.n_chunks, G, Gv)
    rk, rv = st.residual()
    ref = decode_attention(q.cpu().numpy(), kh, vh, rk.float().cpu().numpy(),
                           rv.float().cpu().numpy())
    return rel_err(out.cpu().numpy(), ref)


CASES = [
    # B, Hq, Hkv, D, G, Gv, R, T, splits
    (1, 8, 2, 128, 32, 32, 128, 2200, 1),    # 65 chunks, window 120 (8 passes), one split
    (1, 4, 1, 128, 32, 32, 128, 8292, 4),    # 256 chunks, window 100 (7 passes) over 4 splits
    (1, 16, 2, 128, 32, 32, 128, 2200, 1),   # GQA 8
    (2, 2, 2, 128, 32, 32, 128, 2200, 1),    # MHA
    (1, 8, 2, 64, 32, 32, 64, 2300, 1),      # head_dim 64
    (1, 8, 2, 128, 32, 128, 32, 2049, 1),    # R = G: window of one token, Gv = D
]


@pytest.mark.parametrize("B,Hq,Hkv,D,G,Gv,R,T,splits", CASES)
def test_residual_wave_matches_oracle(store_cls, B, Hq, Hkv, D, G, Gv, R, T, splits):
    print(f"[reswave] B={B} Hq={Hq} Hkv={Hkv} D={D} G={G} Gv={Gv} R={R} T={T} splits={splits}",
          flush=True)
    k, v = make_kv(B, Hkv, T, D, seed=T + D)
    st = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    fill_store(st, k, v, R)
    assert st.res_len > 0 and _chunks_per_wave(st.n_chunks, splits) >= 16
    q = seeded_q(B, Hq, D, seed=T).cuda()
    out = st.attention(q, num_splits=splits)
    torch.cuda.synchronize()
    err = _check(st, k, v, q, out, G, Gv)
    print(f"[reswave]   chunks={st.n_chunks} res={st.res_len} rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL


@pytest.mark.parametrize("splits", [1, 4])
def test_residual_wave_decode_steps(store_cls, splits):
    """Decode steps in this mode: the fused append against a separate append
    (bit-identical) and against the oracle, across a flush."""
    B, Hq, Hkv, D, G, Gv, R = 1, 8, 2, 128, 32, 32, 128
    T = 8300 if splits == 4 else 2200
    steps = 24
    print(f"[reswave] decode steps splits={splits} T={T}", flush=True)
    k, v = make_kv(B, Hkv, T + steps, D, seed=splits + 5)
    a = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    b = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    fill_store(a, k[:, :, :T], v[:, :, :T], R)
    fill_store(b, k[:, :, :T], v[:, :, :T], R)
    flushes = 0
    for step in range(steps):
        t = T + step
        kn, vn = k[:, :, t:t + 1].cuda(), v[:, :, t:t + 1].cuda()
        q = seeded_q(B, Hq, D, seed=100 + step).cuda()
        assert _chunks_per_wave(a.n_chunks, splits) >= 16
        a.stage_token(kn, vn)
        oa = a.attention(q, num_splits=splits).clone()
        b.append(kn, vn)
        ob = b.attention(q, num_splits=splits).clone()
        assert torch.equal(oa, ob), f"step {step}: fused append differs"
        err = _check(a, k, v, q, oa, G, Gv)
        print(f"[reswave]   step {step} chunks={a.n_chunks} res={a.res_len} rel_err={err:.2e}",
              flush=True)
        assert err <= ATTN_TOL
        while a.res_len >= R:
            a.flush()
            b.flush()
            flushes += 1
    assert flushes >= 1


def test_residual_wave_16bit_ring(store_cls):
    """The 16-bit ring in this mode equals the fp32 ring fed the same values."""
    B, Hq, Hkv, D, G, Gv, R, T = 1, 8, 2, 128, 32, 32, 128, 2200
    k, v = make_kv(B, Hkv, T + 1, D, seed=77)
    kh, vh = k.to(torch.bfloat16).cuda(), v.to(torch.bfloat16).cuda()
    a = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    b = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv, residual_dtype=torch.bfloat16)
    a.extend(kh[:, :, :T], vh[:, :, :T], flush_at=R)
    b.extend(kh[:, :, :T], vh[:, :, :T], flush_at=R)
    assert _chunks_per_wave(a.n_chunks, 1) >= 16
    a.stage_token(kh[:, :, T:], vh[:, :, T:])
    b.stage_token(kh[:, :, T:], vh[:, :, T:])
    q = seeded_q(B, Hq, D, seed=9).cuda()
    assert torch.equal(a.attention(q, num_splits=1), b.attention(q, num_splits=1))


def test_decode_from_window_only_into_first_flush(store_cls):
    """A context held entirely in the residual window has no quantised chunk,
    so its launches take the generic kernel (the matrix-core kernel needs a
    chunk in every workgroup); the first flush moves the same decode onto the
    matrix-core kernel.  Each step: the fused append equals a separate append
    bit for bit, and the output matches the oracle."""
    B, Hq, Hkv, D, G, Gv, R = 2, 8, 2, 128, 32, 32, 64
    T, steps = 40, 40
    print(f"[reswave] window-only decode T={T} R={R} steps={steps}", flush=True)
    k, v = make_kv(B, Hkv, T + steps, D, seed=91)
    a = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    b = store_cls(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    fill_store(a, k[:, :, :T], v[:, :, :T], R)
    fill_store(b, k[:, :, :T], v[:, :, :T], R)
    assert a.n_chunks == 0
    seen_chunks = set()
    for step in range(steps):
        t = T + step
        kn, vn = k[:, :, t:t + 1].cuda(), v[:, :, t:t + 1].cuda()
        q = seeded_q(B, Hq, D, seed=300 + step).cuda()
        a.stage_token(kn, vn)
        oa = a.attention(q).clone()
        b.append(kn, vn)
        ob = b.attention(q).clone()
        assert torch.equal(oa, ob), f"step {step}: fused append differs"
        err = _check(a, k, v, q, oa, G, Gv)
        seen_chunks.add(a.n_chunks)
        assert err <= ATTN_TOL, f"step {step}: chunks={a.n_chunks} rel_err={err:.2e}"
        while a.res_len >= R:
            a.flush()
            b.flush()
    print(f"[reswave]   chunk counts seen: {sorted(seen_chunks)}", flush=True)
    assert 0 in seen_chunks and max(seen_chunks) >= 1
