"""Pins the float64 attention oracle (oracle/attention.py) on the CPU.

The reference has no attention kernel; the math it states is
``softmax(Q K^T * D^-0.5) V`` over the dequantised cache
(tests/integration/test_attention_fix.py:40-43,91-93), run by the HF model
with GQA ``repeat_kv`` (query head h reads kv head h // (Hq / Hkv)).  The
oracle is checked here against:
  * torch's scaled_dot_product_attention in float64 (an independent library
    routine), with K/V repeated per query head, on shapes with and without a
    quantised history and a residual window;
  * closed forms: identical keys or a zero query give the mean of V, a
    one-token context gives that token's V, a two-token context the
    two-term softmax written out by hand;
  * mutants: each plausible mistake planted in a copy of the oracle's own
    source (wrong scale, wrong head map, a dropped history or residual, V
    swapped for K, normalisation over the wrong axis) must fail the library
    comparison, so the comparison above pins those parts.
The padding arguments are pinned the same way: ``kv_start`` and ``visible``
(any key-padding pattern) against SDPA with the boolean mask HF builds,
special cases (all visible, a leading run equal to kv_start, one visible
position, none) and their own mutants.
It also pins the vectorised history builder of the GPU tests against the
per-chunk oracle quantise + dequantise.
"""

import os
import types

import numpy as np
import pytest
import torch

from oracle import attention as oracle_attention
from oracle.attention import decode_attention
from tests.kv_helpers import make_kv, oracle_chunk, oracle_history

SHAPES = [
    # B, Hq, Hkv, D, Tq, Tr
    (2, 8, 2, 64, 96, 17),     # GQA 4, history + residual
    (1, 4, 4, 128, 0, 40),     # MHA, residual only (no flush yet)
    (2, 6, 3, 32, 64, 0),      # GQA 2, residual empty right after a flush
    (1, 8, 1, 16, 32, 1),      # GQA 8, one residual token
]


def _inputs(B, Hq, Hkv, D, Tq, Tr, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, D, generator=g, dtype=torch.float64)
    kh = torch.randn(B, Hkv, Tq, D, generator=g, dtype=torch.float64)
    vh = torch.randn(B, Hkv, Tq, D, generator=g, dtype=torch.float64)
    kr = torch.randn(B, Hkv, Tr, D, generator=g, dtype=torch.float64)
    vr = torch.randn(B, Hkv, Tr, D, generator=g, dtype=torch.float64)
    kh[..., 3] *= 10.0                          # a channel outlier
    return q, kh, vh, kr, vr


def _sdpa(q, kh, vh, kr, vr):
    """torch float64 SDPA over [history ; residual], K/V repeated per query head."""
    Hq, Hkv = q.shape[1], kh.shape[1]
    K = torch.cat([kh, kr], dim=2).repeat_interleave(Hq // Hkv, dim=1)
    V = torch.cat([vh, vr], dim=2).repeat_interleave(Hq // Hkv, dim=1)
    o = torch.nn.functional.scaled_dot_product_attention(q[:, :, None], K, V)
    return o[:, :, 0]


def _max_err(fn, shape, seed):
    q, kh, vh, kr, vr = _inputs(*shape, seed=seed)
    out = fn(q.numpy(), kh.numpy(), vh.numpy(), kr.numpy(), vr.numpy())
    return float(np.abs(out - _sdpa(q, kh, vh, kr, vr).numpy()).max())


@pytest.mark.parametrize("shape", SHAPES)
def test_oracle_matches_sdpa_float64(shape):
    assert _max_err(decode_attention, shape, seed=sum(shape)) < 1e-12


def test_closed_forms():
    rng = np.random.default_rng(3)
    B, Hq, Hkv, D, T = 2, 8, 2, 32, 20
    q = rng.standard_normal((B, Hq, D))
    v = rng.standard_normal((B, Hkv, T, D))
    # identical keys: uniform weights, the mean of V
    k = np.broadcast_to(rng.standard_normal((B, Hkv, 1, D)), (B, Hkv, T, D))
    mean_v = np.repeat(v.mean(axis=2), Hq // Hkv, axis=1)
    o = decode_attention(q, k[:, :, :12], v[:, :, :12], k[:, :, 12:], v[:, :, 12:])
    assert np.allclose(o, mean_v, rtol=0, atol=1e-13)
    # zero query: uniform weights whatever the keys
    kk = rng.standard_normal((B, Hkv, T, D))
    o = decode_attention(np.zeros_like(q), kk[:, :, :5], v[:, :, :5], kk[:, :, 5:], v[:, :, 5:])
    assert np.allclose(o, mean_v, rtol=0, atol=1e-13)
    # one-token context (history only, or residual only): that token's V
    v1 = np.repeat(v[:, :, :1], Hq // Hkv, axis=1)[:, :, 0]
    o = decode_attention(q, kk[:, :, :1], v[:, :, :1], None, None)
    assert np.array_equal(o, v1)
    o = decode_attention(q, None, None, kk[:, :, :1], v[:, :, :1])
    assert np.array_equal(o, v1)
    # two tokens, written out: o = (e^s0 v0 + e^s1 v1) / (e^s0 + e^s1),
    # s = q.k / sqrt(D), query head h on kv head h // 4
    o = decode_attention(q, kk[:, :, :1], v[:, :, :1], kk[:, :, 1:2], v[:, :, 1:2])
    for b in range(B):
        for h in range(Hq):
            j = h // (Hq // Hkv)
            s0 = q[b, h] @ kk[b, j, 0] / np.sqrt(D)
            s1 = q[b, h] @ kk[b, j, 1] / np.sqrt(D)
            w0, w1 = np.exp(s0), np.exp(s1)
            ref = (w0 * v[b, j, 0] + w1 * v[b, j, 1]) / (w0 + w1)
            assert np.allclose(o[b, h], ref, rtol=1e-13, atol=1e-13)


MUTANTS = {
    "softmax scale": ("D ** -0.5", "D ** -1.0"),
    "head map": ("kh * g:(kh + 1) * g]", "kh::Hkv]"),
    "history dropped": ("if k_hist is not None and k_hist.shape[2]:", "if False:"),
    "residual dropped": ("if k_res is not None and k_res.shape[2]:", "if False:"),
    "V swapped for K": ("p @ V", "p @ K"),
    "normalised over heads": ("p.sum(axis=1, keepdims=True)", "p.sum(axis=0, keepdims=True)"),
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_mistakes_fail_the_library_comparison(name):
    """A mistake planted in a copy of the oracle's source fails the SDPA
    comparison on at least one shape (so that comparison pins the part the
    mistake touches)."""
    old, new = MUTANTS[name]
    path = os.path.abspath(oracle_attention.__file__)
    with open(path) as f:
        src = f.read()
    assert old in src, f"mutation site for '{name}' not found"
    mutant = types.ModuleType(f"oracle_attention_mutant_{name.replace(' ', '_')}")
    exec(compile(src.replace(old, new), path, "exec"), mutant.__dict__)
    worst = 0.0
    for shape in SHAPES:
        try:
            worst = max(worst, _max_err(mutant.decode_attention, shape, seed=sum(shape)))
        except (ValueError, IndexError):
            worst = np.inf                # the mutant cannot even run this shape
    assert worst > 1e-6, f"mutant '{name}' passes the comparison (max err {worst:.2e})"


@pytest.mark.parametrize("B,H,D,G,Gv,n", [(2, 3, 64, 32, 32, 5), (1, 2, 128, 32, 128, 3),
                                          (2, 2, 8, 4, 4, 6), (1, 4, 64, 64, 16, 2)])
def test_vectorised_history_matches_per_chunk_oracle(B, H, D, G, Gv, n):
    """The GPU tests' one-call history builder equals quantise + dequantise
    chunk by chunk (the store's definition of a chunk), bit for bit."""
    k, v = make_kv(B, H, n * G + 5, D, seed=D + n)
    kh, vh = oracle_history(k, v, n, G, Gv)
    assert kh.shape == (B, H, n * G, D) and vh.shape == (B, H, n * G, D)
    for c in range(n):
        o = oracle_chunk(k[:, :, c * G:(c + 1) * G], v[:, :, c * G:(c + 1) * G], G, Gv)
        assert np.array_equal(o["k_deq"].view(np.uint32), kh[:, :, c * G:(c + 1) * G].view(np.uint32))
        assert np.array_equal(o["v_deq"].view(np.uint32), vh[:, :, c * G:(c + 1) * G].view(np.uint32))
    kh0, vh0 = oracle_history(k, v, 0, G, Gv)
    assert kh0.shape == (B, H, 0, D) and vh0.shape == (B, H, 0, D)


# ---- multi-token queries (causal over the window's newest tokens) ----------
PREFIX_SHAPES = [
    # B, L (q_len), Hq, Hkv, D, Tq, Tr
    (2, 3, 8, 2, 64, 96, 17),     # the reference's q_len=3, GQA 4
    (1, 8, 4, 4, 32, 0, 8),       # the whole window is new tokens, no history
    (2, 2, 6, 3, 16, 64, 40),
    (1, 5, 8, 1, 32, 32, 9),
]


def _sdpa_prefix(q, kh, vh, kr, vr):
    B, L, Hq, D = q.shape
    Hkv = kr.shape[1]
    K = torch.cat([kh, kr], dim=2).repeat_interleave(Hq // Hkv, dim=1)
    V = torch.cat([vh, vr], dim=2).repeat_interleave(Hq // Hkv, dim=1)
    T = K.shape[2]
    mask = torch.arange(T)[None, :] <= (T - L + torch.arange(L))[:, None]     # [L, T]
    o = torch.nn.functional.scaled_dot_product_attention(q.transpose(1, 2), K, V,
                                                         attn_mask=mask)
    return o.transpose(1, 2)                                                 # [B, L, Hq, D]


def _prefix_err(fn, shape, seed):
    B, L, Hq, Hkv, D, Tq, Tr = shape
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, L, Hq, D, generator=g, dtype=torch.float64)
    kh, vh = (torch.randn(B, Hkv, Tq, D, generator=g, dtype=torch.float64) for _ in range(2))
    kr, vr = (torch.randn(B, Hkv, Tr, D, generator=g, dtype=torch.float64) for _ in range(2))
    out = fn(q.numpy(), kh.numpy(), vh.numpy(), kr.numpy(), vr.numpy())
    return float(np.abs(out - _sdpa_prefix(q, kh, vh, kr, vr).numpy()).max())


@pytest.mark.parametrize("shape", PREFIX_SHAPES)
def test_prefix_oracle_matches_sdpa_float64(shape):
    assert _prefix_err(oracle_attention.prefix_attention, shape, seed=sum(shape)) < 1e-12


def test_prefix_oracle_reduces_to_decode():
    """q_len = 1 is the decode case; the last of q_len tokens sees the whole
    cache, so it equals decode attention of that token alone."""
    B, L, Hq, Hkv, D, Tq, Tr = 2, 4, 8, 2, 32, 64, 11
    rng = np.random.default_rng(5)
    q = rng.standard_normal((B, L, Hq, D))
    kh, vh = rng.standard_normal((2, B, Hkv, Tq, D))
    kr, vr = rng.standard_normal((2, B, Hkv, Tr, D))
    o = oracle_attention.prefix_attention(q, kh, vh, kr, vr)
    assert np.array_equal(o[:, -1], decode_attention(q[:, -1], kh, vh, kr, vr))
    o1 = oracle_attention.prefix_attention(q[:, :1], kh, vh, kr[:, :, :Tr - L + 1],
                                           vr[:, :, :Tr - L + 1])
    assert np.array_equal(o1[:, 0], o[:, 0])


PREFIX_MUTANTS = {
    "mask off by one": ("n = T - L + i + 1", "n = T - L + i + 2"),
    "mask reversed": ("n = T - L + i + 1", "n = T - i"),
    "head map": ("q[b, i, kh * g:(kh + 1) * g]", "q[b, i, kh::Hkv]"),
}


@pytest.mark.parametrize("name", sorted(PREFIX_MUTANTS))
def test_prefix_planted_mistakes_fail(name):
    old, new = PREFIX_MUTANTS[name]
    path = os.path.abspath(oracle_attention.__file__)
    with open(path) as f:
        src = f.read()
    assert src.count(old) >= 1, f"mutation site for '{name}' not found"
    mutant = types.ModuleType("oracle_prefix_mutant")
    exec(compile(src.replace(old, new), path, "exec"), mutant.__dict__)
    worst = 0.0
    for shape in PREFIX_SHAPES:
        try:
            worst = max(worst, _prefix_err(mutant.prefix_attention, shape, seed=sum(shape)))
        except (ValueError, IndexError):
            worst = np.inf
    assert worst > 1e-6, f"mutant '{name}' passes (max err {worst:.2e})"


# ---- left-padded batches: each sequence hides its first kv_start[b] positions
PAD_SHAPES = [
    # B, L, Hq, Hkv, D, Tq, Tr, kv_start
    (3, 1, 8, 2, 32, 64, 17, (0, 5, 70)),        # start in the history, in the window
    (2, 3, 4, 4, 16, 32, 9, (31, 32)),            # the last history token, the first window one
    (2, 4, 6, 3, 16, 0, 12, (0, 7)),              # no history
]


def _sdpa_padded(q, kh, vh, kr, vr, kv_start):
    B, L, Hq, D = q.shape
    Hkv = kr.shape[1]
    K = torch.cat([kh, kr], dim=2).repeat_interleave(Hq // Hkv, dim=1)
    V = torch.cat([vh, vr], dim=2).repeat_interleave(Hq // Hkv, dim=1)
    T = K.shape[2]
    t = torch.arange(T)
    causal = t[None, :] <= (T - L + torch.arange(L))[:, None]                     # [L, T]
    pad = t[None, :] >= torch.tensor(kv_start)[:, None]                          # [B, T]
    mask = causal[None, None] & pad[:, None, None]                               # [B, 1, L, T]
    o = torch.nn.functional.scaled_dot_product_attention(q.transpose(1, 2), K, V,
                                                         attn_mask=mask)
    return o.transpose(1, 2)


def _padded_err(mod, shape, seed):
    B, L, Hq, Hkv, D, Tq, Tr, kv_start = shape
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, L, Hq, D, generator=g, dtype=torch.float64)
    kh, vh = (torch.randn(B, Hkv, Tq, D, generator=g, dtype=torch.float64) for _ in range(2))
    kr, vr = (torch.randn(B, Hkv, Tr, D, generator=g, dtype=torch.float64) for _ in range(2))
    ref = _sdpa_padded(q, kh, vh, kr, vr, kv_start).numpy()
    args = (kh.numpy(), vh.numpy(), kr.numpy(), vr.numpy())
    if L == 1:
        out = mod.decode_attention(q[:, 0].numpy(), *args, kv_start=kv_start)[:, None]
    else:
        out = mod.prefix_attention(q.numpy(), *args, kv_start=kv_start)
    return float(np.abs(out - ref).max())


@pytest.mark.parametrize("shape", PAD_SHAPES)
def test_padded_oracle_matches_sdpa_float64(shape):
    """kv_start against SDPA with HF's boolean mask of a left-padded batch
    (padding positions hidden, causal among the new tokens)."""
    assert _padded_err(oracle_attention, shape, seed=len(shape)) < 1e-12


PAD_MUTANTS = {
    "decode start ignored": ("seen = np.arange(K.shape[0]) >= s0",
                             "seen = np.arange(K.shape[0]) >= 0"),
    "decode start off by one": ("seen = np.arange(K.shape[0]) >= s0",
                                "seen = np.arange(K.shape[0]) > s0"),
    "prefix start ignored": ("seen = (t >= s0) & (t < n)", "seen = t < n"),
}


@pytest.mark.parametrize("name", sorted(PAD_MUTANTS))
def test_padded_planted_mistakes_fail(name):
    old, new = PAD_MUTANTS[name]
    path = os.path.abspath(oracle_attention.__file__)
    with open(path) as f:
        src = f.read()
    assert src.count(old) == 1, f"mutation site for '{name}' not found"
    mutant = types.ModuleType("oracle_pad_mutant")
    exec(compile(src.replace(old, new), path, "exec"), mutant.__dict__)
    worst = 0.0
    for shape in PAD_SHAPES:
        try:
            worst = max(worst, _padded_err(mutant, shape, seed=len(shape)))
        except (ValueError, IndexError):
            worst = np.inf
    assert worst > 1e-6, f"mutant '{name}' passes (max err {worst:.2e})"


# ---- any key-padding pattern: position t of sequence b hidden unless visible[b, t]
VIS_SHAPES = [
    # B, L, Hq, Hkv, D, Tq, Tr
    (3, 1, 8, 2, 32, 64, 17),      # decode, GQA 4
    (2, 3, 4, 4, 16, 32, 9),       # three causal query tokens, MHA
    (2, 4, 6, 3, 16, 0, 12),       # no history
]


def _visibility(B, T, seed):
    """Holes, right padding and a run hidden across the history/window edge;
    the last position (the newest query token) always visible."""
    rng = np.random.default_rng(seed)
    vis = rng.random((B, T)) > 0.3
    vis[0, T // 2:T - 1] = False                   # right padding before the new token
    vis[-1, :T // 3] = False                        # a left-padding run
    vis[:, T - 1] = True
    return vis


def _sdpa_visible(q, kh, vh, kr, vr, vis):
    B, L, Hq, D = q.shape
    Hkv = kr.shape[1]
    K = torch.cat([kh, kr], dim=2).repeat_interleave(Hq // Hkv, dim=1)
    V = torch.cat([vh, vr], dim=2).repeat_interleave(Hq // Hkv, dim=1)
    T = K.shape[2]
    t = torch.arange(T)
    causal = t[None, :] <= (T - L + torch.arange(L))[:, None]                     # [L, T]
    mask = causal[None, None] & torch.from_numpy(vis)[:, None, None]              # [B, 1, L, T]
    o = torch.nn.functional.scaled_dot_product_attention(q.transpose(1, 2), K, V,
                                                         attn_mask=mask)
    return o.transpose(1, 2), mask[:, 0].any(-1)                                  # [B, L] rows seen


def _visible_err(mod, shape, seed):
    B, L, Hq, Hkv, D, Tq, Tr = shape
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, L, Hq, D, generator=g, dtype=torch.float64)
    kh, vh = (torch.randn(B, Hkv, Tq, D, generator=g, dtype=torch.float64) for _ in range(2))
    kr, vr = (torch.randn(B, Hkv, Tr, D, generator=g, dtype=torch.float64) for _ in range(2))
    vis = _visibility(B, Tq + Tr, seed)
    ref, seen = _sdpa_visible(q, kh, vh, kr, vr, vis)
    args = (kh.numpy(), vh.numpy(), kr.numpy(), vr.numpy())
    if L == 1:
        out = mod.decode_attention(q[:, 0].numpy(), *args, visible=vis)[:, None]
    else:
        out = mod.prefix_attention(q.numpy(), *args, visible=vis)
    rows = seen.numpy()
    assert rows.any()
    return float(np.abs(out[rows] - ref.numpy()[rows]).max())


@pytest.mark.parametrize("shape", VIS_SHAPES)
def test_visible_oracle_matches_sdpa_float64(shape):
    """``visible`` against SDPA with the boolean mask (visible positions,
    causal among the new tokens), on the rows that see a position."""
    assert _visible_err(oracle_attention, shape, seed=len(shape) + shape[1]) < 1e-12


def test_visible_special_cases():
    """All visible is the unmasked result, a leading hidden run is kv_start,
    one visible position gives that position's V row, none gives zeros."""
    B, L, Hq, Hkv, D, Tq, Tr = 2, 3, 8, 2, 16, 32, 10
    T = Tq + Tr
    rng = np.random.default_rng(11)
    q = rng.standard_normal((B, L, Hq, D))
    kh, vh = rng.standard_normal((2, B, Hkv, Tq, D))
    kr, vr = rng.standard_normal((2, B, Hkv, Tr, D))
    for fn, qq in ((decode_attention, q[:, -1]), (oracle_attention.prefix_attention, q)):
        full = fn(qq, kh, vh, kr, vr)
        assert np.array_equal(fn(qq, kh, vh, kr, vr, visible=np.ones((B, T), bool)), full)
        starts = (5, 33)
        lead = np.arange(T)[None, :] >= np.array(starts)[:, None]
        assert np.array_equal(fn(qq, kh, vh, kr, vr, visible=lead),
                              fn(qq, kh, vh, kr, vr, kv_start=starts))
    one = np.zeros((B, T), bool)
    one[0, 7] = True                     # a history position
    one[1, Tq + 2] = True                # a window position
    o = decode_attention(q[:, -1], kh, vh, kr, vr, visible=one)
    assert np.allclose(o[0], np.repeat(vh[0, :, 7], Hq // Hkv, axis=0), rtol=0, atol=1e-15)
    assert np.allclose(o[1], np.repeat(vr[1, :, 2], Hq // Hkv, axis=0), rtol=0, atol=1e-15)
    none = np.zeros((B, T), bool)
    assert not decode_attention(q[:, -1], kh, vh, kr, vr, visible=none).any()
    # the first query token sees positions up to T - L only: hiding exactly
    # those leaves its row empty (zeros) and the later rows not
    early = np.ones((B, T), bool)
    early[:, :T - L + 1] = False
    o = oracle_attention.prefix_attention(q, kh, vh, kr, vr, visible=early)
    assert not o[:, 0].any() and o[:, 1:].all()


VIS_MUTANTS = {
    "decode visible ignored": ("                seen &= np.asarray(visible[b], dtype=bool)\n"
                               "            qh", "                pass\n            qh"),
    "prefix visible ignored": ("                    seen &= np.asarray(visible[b], dtype=bool)",
                               "                    pass"),
    "visible shifted by one": ("np.asarray(visible[b], dtype=bool)",
                               "np.roll(np.asarray(visible[b], dtype=bool), 1)"),
    "visible inverted": ("seen &= np.asarray(visible[b], dtype=bool)",
                         "seen &= ~np.asarray(visible[b], dtype=bool)"),
}


@pytest.mark.parametrize("name", sorted(VIS_MUTANTS))
def test_visible_planted_mistakes_fail(name):
    old, new = VIS_MUTANTS[name]
    path = os.path.abspath(oracle_attention.__file__)
    with open(path) as f:
        src = f.read()
    assert old in src, f"mutation site for '{name}' not found"
    mutant = types.ModuleType("oracle_visible_mutant")
    exec(compile(src.replace(old, new), path, "exec"), mutant.__dict__)
    worst = 0.0
    for shape in VIS_SHAPES:
        try:
            worst = max(worst, _visible_err(mutant, shape, seed=len(shape) + shape[1]))
        except (ValueError, IndexError, AssertionError):
            worst = np.inf
    assert worst > 1e-6, f"mutant '{name}' passes (max err {worst:.2e})"
