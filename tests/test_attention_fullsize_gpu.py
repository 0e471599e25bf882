"""Attention parity at the sizes bench.py times: configs 3, 4 and 5 of the
benchmark brief, each store built exactly as bench.py builds it (the same
CPU-seeded K/V from ``bench.synth_kv``, one batched ``extend`` with the
KiviCache flush rule, then the residual tokens), checked against float64
attention over the oracle-dequantised history plus the fp32 residual
(oracle/attention.py; the math the reference states in
tests/integration/test_attention_fix.py:40-43).

* Config 3 (Llama-2-7B MHA): B=16, 32/32 heads, D=128, 4096 quantised +
  128 residual tokens.
* Config 4 (Llama-3-8B GQA decode loop): B=64, 32/8 heads, D=128, context
  8192 (8064 quantised + a full window of 128), then decode steps with the
  fused append across two flushes (src/kivi_sycl/cache/manager.py:242-249:
  flush the 32 oldest tokens while the window holds >= R); every flushed
  chunk bit-exact against the oracle codec.
* Config 5 (split-K): B=4, 32/8 heads, D=128, 131072 quantised tokens with
  value groups of 128, a full window of 128; the automatic split count (16)
  and the log-sum-exp merge; the decode step's flush.
* Eight query heads per kv head (Llama-3-70B-shaped GQA, not one of the
  benchmark configs): B=4, 64/8 heads, D=128, context 8192, at the automatic
  split count and at 1 and 2 splits, where each wave takes 32-63 chunks and
  so folds its value corrections into the output several times.

Bar: 1e-3 relative (max |o - o_ref| / max |o_ref| per (batch, head)) for
attention; bit-exact for codes, scales and zeros.
"""

import numpy as np
import pytest
import torch

import bench
from oracle.attention import decode_attention
from tests.kv_helpers import check_store_bit_exact, oracle_history, rel_err, seeded_q

pytestmark = pytest.mark.gpu

ATTN_TOL = 1e-3


def _say(*a):
    print(*a, flush=True)


def _oracle(q, kh, vh, k, v, Tq, T):
    """float64 attention over Tq dequantised tokens + residual [Tq, T)."""
    return decode_attention(q.numpy(), kh[:, :, :Tq], vh[:, :, :Tq],
                            k[:, :, Tq:T].numpy(), v[:, :, Tq:T].numpy())


def test_config3_mha_full_size(hip_device):
    B, H, D, R, G, Tq = 16, 32, 128, 128, 32, 4096
    _say(f"[full] config3 B={B} H={H} D={D} Tq={Tq} Tr={R}")
    k, v = bench.synth_kv(B, H, Tq + R, D, 1234 + 3)
    st = bench.make_store(k[:, :, :Tq + R - 1], v[:, :, :Tq + R - 1], G, G, R, hip_device)
    st.append(k[:, :, -1:].to(hip_device), v[:, :, -1:].to(hip_device))
    assert (st.quantized_tokens, st.res_len) == (Tq, R)
    q = seeded_q(B, H, D, seed=6)
    out = st.attention(q.to(hip_device)).cpu().numpy()
    _say("[full]   GPU done; oracle history")
    kh, vh = oracle_history(k, v, st.n_chunks, G, G)
    err = rel_err(out, _oracle(q, kh, vh, k, v, Tq, Tq + R))
    _say(f"[full]   config3 rel_err={err:.3e}")
    assert err <= ATTN_TOL


def test_config4_decode_loop_full_size(hip_device):
    B, Hq, Hkv, D, T, R, G = bench.CONFIG4
    Tq0 = T - R
    steps = 34                       # flushes at steps 0 and 32
    check_at = (0, 1, 31, 32, 33)
    _say(f"[full] config4 B={B} Hq={Hq} Hkv={Hkv} D={D} context {T}, {steps} decode steps")
    n_tok = Tq0 + (R - 1) + steps
    k, v = bench.synth_kv(B, Hkv, n_tok, D, 1234 + 4)
    st = bench.make_store(k[:, :, :Tq0 + R - 1], v[:, :, :Tq0 + R - 1], G, G, R, hip_device,
                          extra_chunks=4)
    assert (st.quantized_tokens, st.res_len) == (Tq0, R - 1)
    k_new = k[:, :, Tq0 + R - 1:].to(hip_device)
    v_new = v[:, :, Tq0 + R - 1:].to(hip_device)
    g = torch.Generator().manual_seed(5)
    qs = torch.randn(steps, B, Hq, D, generator=g) * D ** -0.5
    outs, states, flush_steps = {}, {}, []
    for i in range(steps):
        st.stage_token(k_new[:, :, i:i + 1], v_new[:, :, i:i + 1])
        o = st.attention(qs[i].to(hip_device))
        if i in check_at:
            outs[i] = o.cpu().numpy()
            states[i] = (st.quantized_tokens, st.quantized_tokens + st.res_len)
        while st.res_len >= R:
            st.flush()
            flush_steps.append(i)
    torch.cuda.synchronize()
    assert flush_steps == [0, 32]
    assert st.quantized_tokens == Tq0 + 2 * G
    _say("[full]   GPU done; checking the two decode-time flushes bit for bit")
    check_store_bit_exact(st, k, v, chunks=[Tq0 // G, Tq0 // G + 1])
    _say("[full]   oracle history")
    kh, vh = oracle_history(k, v, st.n_chunks, G, G)
    for i in check_at:
        Tq, Tend = states[i]
        err = rel_err(outs[i], _oracle(qs[i], kh, vh, k, v, Tq, Tend))
        _say(f"[full]   step {i}: Tq={Tq} Tr={Tend - Tq} rel_err={err:.3e}")
        assert err <= ATTN_TOL, f"step {i}"


def test_config5_split_k_full_size(hip_device):
    B, Hq, Hkv, D, R, G, Gv, Tq = 4, 32, 8, 128, 128, 32, 128, 131072
    _say(f"[full] config5 B={B} Hq={Hq} Hkv={Hkv} D={D} Tq={Tq} Gv={Gv}")
    k, v = bench.synth_kv(B, Hkv, Tq + R, D, 1234 + 5)
    st = bench.make_store(k[:, :, :Tq + R - 1], v[:, :, :Tq + R - 1], G, Gv, R, hip_device)
    assert (st.quantized_tokens, st.res_len) == (Tq, R - 1)
    # the decode step: the new token filed by the attention launch itself
    st.stage_token(k[:, :, -1:].to(hip_device), v[:, :, -1:].to(hip_device))
    ws = st.workspace_bytes(Hq)
    splits = ws // (B * Hq * (D + 2) * 4)
    _say(f"[full]   automatic split count {splits}")
    assert splits >= 8, "the long context must be split across workgroups"
    q = seeded_q(B, Hq, D, seed=7).to(hip_device)
    out_fused = st.attention(q).cpu().numpy()
    # the bench's timed call: the token now read from the ring
    out_ring = st.attention(q).cpu().numpy()
    assert np.array_equal(out_fused.view(np.uint32), out_ring.view(np.uint32))
    st.flush()
    assert (st.quantized_tokens, st.res_len) == (Tq + G, R - G)
    check_store_bit_exact(st, k, v, chunks=[Tq // G])
    _say("[full]   GPU done; oracle history")
    kh, vh = oracle_history(k, v, Tq // G, G, Gv)
    err = rel_err(out_fused, _oracle(q.cpu(), kh, vh, k, v, Tq, Tq + R))
    _say(f"[full]   config5 rel_err={err:.3e}")
    assert err <= ATTN_TOL
    # after the flush, other split counts agree with the oracle too (1 = no merge)
    del kh, vh
    kh, vh = oracle_history(k, v, st.n_chunks, G, Gv)
    ref = _oracle(q.cpu(), kh, vh, k, v, Tq + G, Tq + R)
    for s in (1, 3, 32):
        o = st.attention(q, num_splits=s).cpu().numpy()
        e = rel_err(o, ref)
        _say(f"[full]   after the flush, {s} splits: rel_err={e:.3e}")
        assert e <= ATTN_TOL


def test_gqa8_long_context(hip_device):
    B, Hq, Hkv, D, R, G, T = 4, 64, 8, 128, 128, 32, 8192
    Tq = T - R
    _say(f"[full] gqa8 B={B} Hq={Hq} Hkv={Hkv} D={D} Tq={Tq} Tr={R}")
    k, v = bench.synth_kv(B, Hkv, T, D, 1234 + 8)
    st = bench.make_store(k[:, :, :T - 1], v[:, :, :T - 1], G, G, R, hip_device)
    st.append(k[:, :, -1:].to(hip_device), v[:, :, -1:].to(hip_device))
    assert (st.quantized_tokens, st.res_len) == (Tq, R)
    q = seeded_q(B, Hq, D, seed=8)
    outs = {s: st.attention(q.to(hip_device), num_splits=s).cpu().numpy() for s in (0, 1, 2)}
    _say("[full]   GPU done; oracle history")
    kh, vh = oracle_history(k, v, st.n_chunks, G, G)
    ref = _oracle(q, kh, vh, k, v, Tq, T)
    for s, o in outs.items():
        err = rel_err(o, ref)
        _say(f"[full]   gqa8 splits={s} rel_err={err:.3e}")
        assert err <= ATTN_TOL, f"splits={s}"
