"""Test infrastructure only: float64 decode attention over a KIVI cache.

The reference has no attention kernel.  Its attention semantics are what its
test states explicitly -- ``softmax(Q K^T * D^-0.5) V`` over the dequantised
keys/values (tests/integration/test_attention_fix.py:40-43,91-93) -- and what
the HF model computes over ``get_full_cache()`` (dequantised history followed
by the fp32 residual window, src/kivi_sycl/cache/manager.py:263-288).  Query
head ``h`` reads kv head ``h // (Hq // Hkv)`` (HF ``repeat_kv``).
"""

from __future__ import annotations

import numpy as np


def _attend(qh, K, V, scale, seen):
    """softmax(qh K^T * scale) V over the positions ``seen`` (bool [T]);
    zeros when none is seen."""
    if not seen.any():
        return np.zeros((qh.shape[0], V.shape[1]))
    K, V = K[seen], V[seen]
    s = (qh @ K.T) * scale                       # [g, n]
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return p @ V


def decode_attention(q, k_hist, v_hist, k_res, v_res, softmax_scale=None, kv_start=None,
                     visible=None):
    """q: [B, Hq, D]; k_hist/v_hist: [B, Hkv, Tq, D] dequantised history;
    k_res/v_res: [B, Hkv, Tr, D] fp32 residual.  Returns o [B, Hq, D] float64.

    ``kv_start`` (B ints, optional): sequence b attends to context positions
    kv_start[b] .. Tq+Tr-1 only -- a left-padded batch, whose HF attention
    mask hides each sequence's leading pad positions.  ``visible`` (bool
    [B, Tq+Tr], optional): any key-padding pattern, position t of sequence b
    attended only where visible[b, t] (HF's 2-D attention mask); a sequence
    that sees no position gets zeros.

    Works one (batch, kv-head) at a time so that long contexts fit in memory.
    """
    q = np.asarray(q, dtype=np.float64)
    B, Hq, D = q.shape
    Hkv = k_hist.shape[1] if k_hist is not None else k_res.shape[1]
    if Hq % Hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    g = Hq // Hkv
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    out = np.empty((B, Hq, D), dtype=np.float64)
    for b in range(B):
        for kh in range(Hkv):
            parts_k, parts_v = [], []
            if k_hist is not None and k_hist.shape[2]:
                parts_k.append(np.asarray(k_hist[b, kh], dtype=np.float64))
                parts_v.append(np.asarray(v_hist[b, kh], dtype=np.float64))
            if k_res is not None and k_res.shape[2]:
                parts_k.append(np.asarray(k_res[b, kh], dtype=np.float64))
                parts_v.append(np.asarray(v_res[b, kh], dtype=np.float64))
            K = np.concatenate(parts_k, axis=0)          # [T, D]
            V = np.concatenate(parts_v, axis=0)
            s0 = 0 if kv_start is None else int(kv_start[b])
            seen = np.arange(K.shape[0]) >= s0
            if visible is not None:
                seen &= np.asarray(visible[b], dtype=bool)
            qh = q[b, kh * g:(kh + 1) * g]               # [g, D]
            out[b, kh * g:(kh + 1) * g] = _attend(qh, K, V, scale, seen)
    return out


def prefix_attention(q, k_hist, v_hist, k_res, v_res, softmax_scale=None, kv_start=None,
                     visible=None):
    """Causal attention of the window's last ``q_len`` tokens.

    q: [B, q_len, Hq, D] -- the queries of the ``q_len`` newest tokens, which
    are the last ``q_len`` tokens of the residual window (k_res/v_res
    [B, Hkv, Tr, D], Tr >= q_len) after the dequantised history
    k_hist/v_hist [B, Hkv, Tq, D].  Query token i (0-based) sits at position
    Tq + Tr - q_len + i and attends to positions 0 .. Tq + Tr - q_len + i:
    the HF model's causal mask over [cache ; new tokens] in a forward of
    ``q_len`` tokens on a non-empty cache (the reference's own attention check
    uses q_len=3, tests/integration/test_attention_fix.py:19-36,91-93).
    GQA, ``kv_start`` and ``visible`` (hidden positions on top of the causal
    rule; a query row that sees no position gets zeros) as in
    decode_attention.  Returns o [B, q_len, Hq, D] float64.
    """
    q = np.asarray(q, dtype=np.float64)
    B, L, Hq, D = q.shape
    Hkv = k_res.shape[1]
    if Hq % Hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    if k_res.shape[2] < L:
        raise ValueError("the residual window must hold the q_len new tokens")
    g = Hq // Hkv
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    out = np.empty((B, L, Hq, D), dtype=np.float64)
    for b in range(B):
        for kh in range(Hkv):
            parts_k, parts_v = [], []
            if k_hist is not None and k_hist.shape[2]:
                parts_k.append(np.asarray(k_hist[b, kh], dtype=np.float64))
                parts_v.append(np.asarray(v_hist[b, kh], dtype=np.float64))
            parts_k.append(np.asarray(k_res[b, kh], dtype=np.float64))
            parts_v.append(np.asarray(v_res[b, kh], dtype=np.float64))
            K = np.concatenate(parts_k, axis=0)          # [T, D]
            V = np.concatenate(parts_v, axis=0)
            T = K.shape[0]
            s0 = 0 if kv_start is None else int(kv_start[b])
            t = np.arange(T)
            for i in range(L):
                n = T - L + i + 1                        # visible tokens of query i
                seen = (t >= s0) & (t < n)
                if visible is not None:
                    seen &= np.asarray(visible[b], dtype=bool)
                qh = q[b, i, kh * g:(kh + 1) * g]        # [g, D]
                out[b, i, kh * g:(kh + 1) * g] = _attend(qh, K, V, scale, seen)
    return out
