"""Test-side helpers: build packed stores from seeded K/V and the matching
oracle views (dequantised history, expected store bytes)."""

import numpy as np
import torch

from oracle import codec
from tests.conftest import seeded_kv


def make_kv(B, H, T, D, seed):
    k = seeded_kv((B, H, T, D), seed=seed, kind="key")
    v = seeded_kv((B, H, T, D), seed=seed + 1, kind="value")
    return k, v


def oracle_chunk(k_chunk, v_chunk, G, Gv):
    """Oracle quantisation of one chunk [B,H,G,D] in the store's byte order.

    Keys: quantize_keys on the [B,H,D,G] transpose (per channel along tokens),
    then codes re-packed token-major ([G][D/4], channel 4i+k at bits 2k).
    Values: quantize_values on [B,H,G,D] rows, codes re-packed channel-major
    ([D][G/4], token 4j+k at bits 2k)."""
    B, H, _, D = k_chunk.shape
    kt = k_chunk.transpose(2, 3).contiguous().numpy()             # [B,H,D,G]
    kp, ks, kz = codec.quantize_groups(kt, G)
    kcodes = codec.unpack_codes(kp, G).reshape(B, H, D, G).transpose(0, 1, 3, 2)   # [B,H,G,D]
    k_bytes = pack_last(kcodes)                                    # [B,H,G,D/4]
    vp, vs, vz = codec.quantize_groups(v_chunk.contiguous().numpy(), Gv)
    vcodes = codec.unpack_codes(vp, Gv).reshape(B, H, G, D).transpose(0, 1, 3, 2)  # [B,H,D,G]
    v_bytes = pack_last(vcodes)                                    # [B,H,D,G/4]
    k_deq = codec.dequantize_groups(kp, ks, kz, G).reshape(B, H, D, G).transpose(0, 1, 3, 2)
    v_deq = codec.dequantize_groups(vp, vs, vz, Gv).reshape(B, H, G, D)
    return {
        "k_codes": k_bytes, "k_scale": ks.reshape(B, H, D), "k_zero": kz.reshape(B, H, D),
        "v_codes": v_bytes, "v_scale": vs.reshape(B, H, G, D // Gv),
        "v_zero": vz.reshape(B, H, G, D // Gv),
        "k_deq": np.ascontiguousarray(k_deq), "v_deq": v_deq,
    }


def pack_last(codes):
    """codes [..., N] (N % 4 == 0) -> bytes [..., N/4], element 4j+k at bits 2k."""
    c = codes.astype(np.uint8).reshape(*codes.shape[:-1], codes.shape[-1] // 4, 4)
    return (c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)).astype(np.uint8)


def fill_store(store, k, v, R):
    """Feed tokens [B,H,T,D] one group at a time as KiviCache would (flush
    while residual >= R)."""
    T = k.shape[2]
    dev = store.device
    t = 0
    step = store.G
    while t < T:
        n = min(step, T - t, store.R - store.res_len)
        store.append(k[:, :, t:t + n].to(dev), v[:, :, t:t + n].to(dev))
        t += n
        while store.res_len >= R:
            store.flush()


def oracle_history(k, v, n_chunks, G, Gv):
    """Dequantised history [B,H,n_chunks*G,D] for keys and values.

    One oracle round-trip call per tensor over the whole history (the
    round-trip is pinned bit-identical to quantise + dequantise): keys as
    [B,H,n,D,G] (each channel of each chunk one group of G tokens), values as
    [B,H,n*G,D] (each token's channels in groups of Gv)."""
    B, H, _, D = k.shape
    T = n_chunks * G
    if T == 0:
        return np.zeros((B, H, 0, D), np.float32), np.zeros((B, H, 0, D), np.float32)
    k, v = torch.as_tensor(k), torch.as_tensor(v)
    # layout changes in torch (threaded copies), the arithmetic in the oracle
    kt = k[:, :, :T].reshape(B, H, n_chunks, G, D).transpose(3, 4).contiguous()
    k_deq = torch.from_numpy(codec.roundtrip_groups(kt.numpy(), G)).reshape(B, H, n_chunks, D, G)
    del kt
    k_deq = k_deq.transpose(3, 4).contiguous().reshape(B, H, T, D).numpy()
    v_deq = codec.roundtrip_groups(v[:, :, :T].contiguous().numpy(), Gv).reshape(B, H, T, D)
    return k_deq, v_deq


def _u32(t):
    return t.detach().cpu().numpy().view(np.uint32)


def check_store_bit_exact(st, k, v, chunks=None):
    """Every flushed chunk of store ``st`` (or those listed in ``chunks``:
    codes through the documented byte transposes, scales, zeros and, if
    kept, the dequantised history) equals the oracle's quantisation of
    tokens [c*G, (c+1)*G) of ``k``/``v`` ([B,H,T,D] fp32, CPU), and the
    residual window holds the tokens after the last chunk (up to T)."""
    G, Gv = st.G, st.Gv
    for c in (range(st.n_chunks) if chunks is None else chunks):
        assert 0 <= c < st.n_chunks, f"chunk {c} not flushed ({st.n_chunks} chunks)"
        o = oracle_chunk(k[:, :, c * G:(c + 1) * G], v[:, :, c * G:(c + 1) * G], G, Gv)
        assert np.array_equal(st.unpermuted_k_codes(c).cpu().numpy(), o["k_codes"]), \
            f"k codes chunk {c}"
        assert np.array_equal(_u32(st.k_scale[:, :, c]), o["k_scale"].view(np.uint32))
        assert np.array_equal(_u32(st.k_zero[:, :, c]), o["k_zero"].view(np.uint32))
        assert np.array_equal(st.unpermuted_v_codes(c).cpu().numpy(), o["v_codes"]), \
            f"v codes chunk {c}"
        assert np.array_equal(_u32(st.chunk_v_scale(c).contiguous()), o["v_scale"].view(np.uint32))
        assert np.array_equal(_u32(st.chunk_v_zero(c).contiguous()), o["v_zero"].view(np.uint32))
        if st.k_hist is not None:
            kh = st.k_hist[:, :, c * G:(c + 1) * G]
            vh = st.v_hist[:, :, c * G:(c + 1) * G]
            assert np.array_equal(_u32(kh), o["k_deq"].view(np.uint32)), f"k history chunk {c}"
            assert np.array_equal(_u32(vh), o["v_deq"].view(np.uint32)), f"v history chunk {c}"
    rk, rv = st.residual()
    q0 = st.n_chunks * G
    q1 = q0 + st.res_len
    assert torch.equal(rk.cpu(), k[:, :, q0:q1]) and torch.equal(rv.cpu(), v[:, :, q0:q1])


def rel_err(out, ref):
    """max |out - ref| / max |ref| per (b, head) row, worst row."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    num = np.abs(out - ref).max(axis=-1)
    den = np.abs(ref).max(axis=-1)
    return float((num / den).max())


def seeded_q(B, Hq, D, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, Hq, D, generator=g) * (D ** -0.5)
