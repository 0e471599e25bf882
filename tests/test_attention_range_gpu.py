"""Dynamic range of the matrix-core decode attention.

The kernel forms its products in units of 2^-64: each 2-bit code is read in
place as the bf16 value c * 2^(2k-133) (k its operand position), and the
scales it multiplies carry 2^(69-2k).  That bounds the factors the kernel
takes: key scales and the key products q * ks * softmax_scale * log2(e)
below 2^59, value scales below 2^51; value codes' products below ~2^-38
lose relative precision (fp32 subnormals).  The reference has no such
window (fp32 attention over the dequantised history,
src/kivi_sycl/cache/manager.py:251-290), so the window is checked here at
its edges, with the 1e-3 bar of the benchmark brief against float64
attention over the oracle-dequantised history plus the fp32 residual (the
math of tests/integration/test_attention_fix.py:40-43):

* keys x 2^50 (scales ~2^52, products kept moderate by a query x 2^-50);
* values x 2^45 (scales ~2^47, token outliers ~2^50);
* keys and values x 2^-30 (query x 2^30);
* values x 2^-30 alone (outputs ~2^-30).
"""

import numpy as np
import pytest

import bench
from oracle.attention import decode_attention
from tests.kv_helpers import oracle_history, rel_err, seeded_q

pytestmark = pytest.mark.gpu

ATTN_TOL = 1e-3
# B, Hq, Hkv, D, R, G, T: config 4's per-sequence shape at batch 2
SHAPE = (2, 32, 8, 128, 128, 32, 2048 + 128)
CASES = {                       # (key exponent, value exponent)
    "keys_2^50": (50, 0),
    "values_2^45": (0, 45),
    "both_2^-30": (-30, -30),
    "values_2^-30": (0, -30),
}


@pytest.fixture(scope="module")
def base_kv():
    B, HQ, HKV, D, R, G, T = SHAPE
    return bench.synth_kv(B, HKV, T, D, 1234 + 7)


@pytest.mark.parametrize("case", list(CASES))
def test_scaled_inputs(base_kv, hip_device, case):
    B, HQ, HKV, D, R, G, T = SHAPE
    ek, ev = CASES[case]
    print(f"[range] {case}: keys x 2^{ek}, values x 2^{ev}", flush=True)
    k0, v0 = base_kv
    k, v = k0 * 2.0 ** ek, v0 * 2.0 ** ev
    st = bench.make_store(k[:, :, :T - 1], v[:, :, :T - 1], G, G, R, hip_device)
    st.append(k[:, :, -1:].to(hip_device), v[:, :, -1:].to(hip_device))
    Tq = T - R
    assert (st.quantized_tokens, st.res_len) == (Tq, R)
    kh, vh = oracle_history(k, v, st.n_chunks, G, G)
    q = seeded_q(B, HQ, D, seed=9) * 2.0 ** -ek
    out = st.attention(q.to(hip_device)).cpu().numpy()
    assert np.isfinite(out).all()
    ref = decode_attention(q.numpy(), kh, vh, k[:, :, Tq:].numpy(), v[:, :, Tq:].numpy())
    err = rel_err(out, ref)
    print(f"[range]   rel_err={err:.3e}", flush=True)
    assert err <= ATTN_TOL
