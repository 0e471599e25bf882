"""GPU test of kivi_packed_decode_attention_noalloc, the allocation-free
variant of kivi_packed_decode_attention (no reference counterpart: it is for
callers that cannot allocate device memory).  Called through the C ABI
(ctypes) against the existing entry point with a caller workspace, on two
calls in a row, the second with a smaller input: outputs bit-identical
(same kernels and plan; the split partials live in the library's static
device array instead of the workspace), and within 1e-3 of float64
attention over the oracle-dequantised cache (oracle/attention.py)."""

import ctypes

import numpy as np
import pytest
import torch

from oracle.attention import decode_attention
from tests.kv_helpers import make_kv, oracle_history, rel_err, seeded_q

pytestmark = pytest.mark.gpu

KIVI_NOALLOC_SCRATCH_BYTES = 8 << 20


def _vp(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _common(st, q, out, splits):
    """Arguments shared by both entry points, split around the workspace."""
    Hq = q.shape[1]
    head = [_vp(q), _vp(st.k_codes), _vp(st.k_scale), _vp(st.k_zero), _vp(st.v_codes),
            _vp(st.v_scale), _vp(st.v_zero), _vp(st.k_res), _vp(st.v_res), st.res_dtype_code,
            _vp(out)]
    tail = [st.B, Hq, st.H, st.D, st.G, st.Gv, st.capacity, st.n_chunks, st.R, st.res_start,
            st.res_len, float(st.D ** -0.5), splits,
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)]
    return head, tail


def _case(lib, B, Hq, Hkv, D, G, Gv, R, T, splits, seed):
    from intel_kivi_hybrid_amd import _native
    from intel_kivi_hybrid_amd.store import PackedKVStore
    print(f"[noalloc] B={B} Hq={Hq} Hkv={Hkv} D={D} G={G} Gv={Gv} R={R} T={T} splits={splits}",
          flush=True)
    k, v = make_kv(B, Hkv, T, D, seed=seed)
    st = PackedKVStore(B, Hkv, D, G, R, "cuda:0", group_size_v=Gv)
    st.extend(k.cuda(), v.cuda(), flush_at=R)
    q = seeded_q(B, Hq, D, seed=seed + 1).cuda()
    need = st.workspace_bytes(Hq, splits)
    assert need <= KIVI_NOALLOC_SCRATCH_BYTES
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda:0")
    out_ws = torch.full_like(q, float("nan"))
    out_na = torch.full_like(q, float("nan"))
    head, tail = _common(st, q, out_ws, splits)
    _native.check(lib.kivi_packed_decode_attention(*head, _vp(ws), need, *tail),
                  "kivi_packed_decode_attention")
    head, tail = _common(st, q, out_na, splits)
    _native.check(lib.kivi_packed_decode_attention_noalloc(*head, *tail),
                  "kivi_packed_decode_attention_noalloc")
    torch.cuda.synchronize()
    a, b = out_ws.cpu().numpy(), out_na.cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "noalloc output differs"
    kh, vh = oracle_history(k, v, st.n_chunks, G, Gv)
    q0 = st.n_chunks * G
    err = rel_err(b, decode_attention(q.cpu().numpy(), kh, vh, k[:, :, q0:].numpy(),
                                      v[:, :, q0:].numpy()))
    print(f"[noalloc]   chunks={st.n_chunks} res={st.res_len} partials={need} B "
          f"rel_err={err:.3e}", flush=True)
    assert err <= 1e-3
    return need


def test_noalloc_matches_workspace_entry_point(hip_device):
    from intel_kivi_hybrid_amd import _native
    lib = _native.load()
    # first call: split partials in the scratch array (7 splits, 2 rows of 8 heads)
    need1 = _case(lib, 2, 8, 2, 128, 32, 32, 64, 2000, splits=7, seed=11)
    # second call, smaller: fewer rows, fewer splits, head_dim 64
    need2 = _case(lib, 1, 4, 1, 64, 32, 32, 32, 700, splits=3, seed=12)
    assert 0 < need2 < need1
    # a single split needs no partials at all
    assert _case(lib, 1, 8, 2, 128, 32, 32, 64, 500, splits=1, seed=13) == 0


def test_noalloc_plain_layout_and_wide_head_groups(hip_device):
    """The generic kernel (a plain-layout store: G = 16) and more than 8
    query heads per kv head (12: launches over head groups of 8 and 4, each
    leaving its partials in the same scratch array before its merge), split,
    against the workspace entry point bit for bit."""
    from intel_kivi_hybrid_amd import _native
    lib = _native.load()
    _case(lib, 2, 4, 2, 64, 16, 16, 32, 600, splits=5, seed=14)
    _case(lib, 2, 24, 2, 128, 32, 32, 64, 1500, splits=3, seed=15)
