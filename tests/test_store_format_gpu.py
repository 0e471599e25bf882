"""GPU checks of the packed-store format: a store's export in the reference's
quantize_keys / quantize_values layouts equals the oracle codec run over the
whole quantised history (bit-exact), re-imports into an identical store, and
a saved KiviPackedCache reloads into a cache that decodes identically."""

import numpy as np
import pytest
import torch

from oracle import codec
from tests.kv_helpers import make_kv, seeded_q

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def store_cls(hip_device):
    from intel_kivi_hybrid_amd.store import PackedKVStore
    return PackedKVStore


SHAPES = [
    (2, 4, 128, 32, 32, 64, 300),    # matrix-core code order
    (1, 3, 128, 32, 128, 64, 170),   # Gv = D
    (1, 2, 8, 4, 4, 8, 30),          # plain code order (reference test geometry)
    (2, 2, 64, 64, 32, 128, 260),    # G = 64
]


def _filled(store_cls, B, H, D, G, Gv, R, T, seed, history=False):
    k, v = make_kv(B, H, T, D, seed=seed)
    st = store_cls(B, H, D, G, R, "cuda:0", group_size_v=Gv, keep_history=history)
    st.extend(k.cuda(), v.cuda(), flush_at=R)
    return st, k, v


@pytest.mark.parametrize("B,H,D,G,Gv,R,T", SHAPES)
def test_export_is_reference_layout(store_cls, B, H, D, G, Gv, R, T):
    print(f"[format] export B={B} H={H} D={D} G={G} Gv={Gv} R={R} T={T}", flush=True)
    st, k, v = _filled(store_cls, B, H, D, G, Gv, R, T, seed=T)
    n = st.n_chunks
    Tq = n * G
    ex = {name: t.cpu() for name, t in st.export_state().items()}
    kt = k[:, :, :Tq].transpose(2, 3).contiguous().numpy()          # [B,H,D,Tq]
    kp, ks, kz = codec.quantize_groups(kt, G)
    assert np.array_equal(ex["k_codes"].numpy().reshape(-1), kp)
    assert np.array_equal(ex["k_scale"].numpy().reshape(-1).view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(ex["k_zero"].numpy().reshape(-1).view(np.uint32), kz.view(np.uint32))
    vp, vs, vz = codec.quantize_groups(v[:, :, :Tq].contiguous().numpy(), Gv)
    assert np.array_equal(ex["v_codes"].numpy().reshape(-1), vp)
    assert np.array_equal(ex["v_scale"].numpy().reshape(-1).view(np.uint32), vs.view(np.uint32))
    assert np.array_equal(ex["v_zero"].numpy().reshape(-1).view(np.uint32), vz.view(np.uint32))
    assert ex["k_codes"].shape == (B, H, D, Tq // 4) and ex["v_codes"].shape == (B, H, Tq, D // 4)
    assert torch.equal(ex["k_residual"], k[:, :, Tq:]) and torch.equal(ex["v_residual"], v[:, :, Tq:])


@pytest.mark.parametrize("B,H,D,G,Gv,R,T", SHAPES)
def test_import_restores_the_store(store_cls, B, H, D, G, Gv, R, T):
    st, _, _ = _filled(store_cls, B, H, D, G, Gv, R, T, seed=T + 1)
    back = store_cls.from_state(st.export_state(), G, R, "cuda:0", group_size_v=Gv)
    n = st.n_chunks
    assert (back.n_chunks, back.res_len) == (n, st.res_len)
    for name in ("k_codes", "k_scale", "k_zero", "v_codes", "v_scale", "v_zero"):
        assert torch.equal(getattr(back, name)[:, :, :n], getattr(st, name)[:, :, :n]), name
    for a, b in zip(back.residual(), st.residual()):
        assert torch.equal(a, b)
    if D % 16 == 0 and G % 16 == 0:
        q = seeded_q(B, 2 * H, D, seed=3).cuda()
        assert torch.equal(back.attention(q), st.attention(q))


def test_export_dequantises_with_the_reference_ops(store_cls):
    """The exported codes in the _C layouts dequantise (with the _C ops)
    to exactly the history the flush kernel served."""
    from intel_kivi_hybrid_amd import _C
    B, H, D, G, Gv, R, T = 2, 4, 128, 32, 32, 64, 250
    st, _, _ = _filled(store_cls, B, H, D, G, Gv, R, T, seed=9, history=True)
    ex = st.export_state()
    Tq = st.quantized_tokens
    kd = torch.empty(B, H, D, Tq, device="cuda:0")
    _C.dequantize_keys(ex["k_codes"].contiguous(), ex["k_scale"].contiguous(),
                       ex["k_zero"].contiguous(), kd, G)
    vd = torch.empty(B, H, Tq, D, device="cuda:0")
    _C.dequantize_values(ex["v_codes"].contiguous(), ex["v_scale"].contiguous(),
                         ex["v_zero"].contiguous(), vd, D, Gv)
    assert torch.equal(kd.transpose(2, 3), st.k_hist[:, :, :Tq])
    assert torch.equal(vd, st.v_hist[:, :, :Tq])


def test_import_rejects_inconsistent_state(store_cls):
    st, _, _ = _filled(store_cls, 1, 2, 64, 32, 32, 32, 100, seed=4)
    ex = st.export_state()
    bad = dict(ex)
    bad["v_codes"] = ex["v_codes"][:, :, :-1]
    with pytest.raises(ValueError, match="v_codes"):
        store_cls.from_state(bad, 32, 32, "cuda:0")
    with pytest.raises(ValueError, match="exceeds capacity"):
        store_cls.from_state(ex, 32, 2, "cuda:0")
    with pytest.raises(ValueError, match="lacks"):
        store_cls.from_state({"k_codes": ex["k_codes"]}, 32, 32, "cuda:0")


def test_saved_cache_resumes_decoding(hip_device, tmp_path):
    """Save a KiviPackedCache mid-generation, load it, and continue: the next
    forward passes produce bit-identical logits to the uninterrupted cache."""
    from transformers import GPT2Config, GPT2LMHeadModel
    from intel_kivi_hybrid_amd.cache.packed_cache import KiviPackedCache, packed_attention
    torch.manual_seed(5)
    model = GPT2LMHeadModel(GPT2Config(n_layer=3, n_head=4, n_embd=256)).eval().to(hip_device)
    ids = torch.randint(0, model.config.vocab_size, (2, 70), generator=torch.Generator().manual_seed(1))
    a = KiviPackedCache.from_model(model, device="cuda:0", group_size=32, residual_length=32)
    with torch.no_grad(), packed_attention(model):
        out = model(ids.to(hip_device), past_key_values=a, use_cache=True)
        nxt = out.logits[:, -1:].argmax(-1)
        for _ in range(13):
            out = model(nxt, past_key_values=a, use_cache=True)
            nxt = out.logits[:, -1:].argmax(-1)
        path = str(tmp_path / "cache.safetensors")
        a.save(path)
        b = KiviPackedCache.load(path, device="cuda:0")
        assert b.get_seq_length() == a.get_seq_length() == 83
        assert b.total_flushes == a.total_flushes
        for key in ("total_tokens", "quantized_tokens", "residual_tokens", "kivi_bytes"):
            assert b.get_stats(1)[key] == a.get_stats(1)[key]
        na = nb = nxt
        for _ in range(40):
            oa = model(na, past_key_values=a, use_cache=True)
            ob = model(nb, past_key_values=b, use_cache=True)
            assert torch.equal(oa.logits, ob.logits)
            na = oa.logits[:, -1:].argmax(-1)
            nb = ob.logits[:, -1:].argmax(-1)


def test_save_leaves_a_pending_step_croppable(hip_device, tmp_path):
    """A multi-token step takes the window past R and leaves its flushes to
    the next update.  save() writes the settled state (the file's windows
    hold fewer than R tokens, and the loaded cache decodes as the settled
    one) without settling the live cache, so a crop() of that step's
    tokens still works after the save and the cache then continues exactly
    as a twin that was never saved."""
    from transformers import GPT2Config, GPT2LMHeadModel
    from intel_kivi_hybrid_amd.cache.packed_cache import KiviPackedCache, packed_attention
    torch.manual_seed(6)
    model = GPT2LMHeadModel(GPT2Config(n_layer=2, n_head=4, n_embd=256)).eval().to(hip_device)
    gen = torch.Generator().manual_seed(2)
    ids = torch.randint(0, model.config.vocab_size, (1, 60), generator=gen).to(hip_device)
    draft = torch.randint(0, model.config.vocab_size, (1, 7), generator=gen).to(hip_device)
    G, R = 32, 32
    a = KiviPackedCache.from_model(model, device="cuda:0", group_size=G, residual_length=R)
    twin = KiviPackedCache.from_model(model, device="cuda:0", group_size=G, residual_length=R)
    with torch.no_grad(), packed_attention(model):
        for c in (a, twin):
            model(ids, past_key_values=c, use_cache=True)
            model(draft, past_key_values=c, use_cache=True)
        res_before = a.store(0).res_len
        assert res_before >= R                      # the step's flushes are still owed
        path = str(tmp_path / "pending.safetensors")
        a.save(path)
        assert a.store(0).res_len == res_before     # the live cache is untouched
        b = KiviPackedCache.load(path, device="cuda:0")
        assert b.store(0).res_len < R and b.get_seq_length() == a.get_seq_length()
        owed = (res_before - R) // G + 1              # per layer, as settle() does them
        assert b.total_flushes == a.total_flushes + model.config.n_layer * owed
        # the settled file decodes as the unsaved cache does after its update
        nxt = draft[:, -1:]
        ob = model(nxt, past_key_values=b, use_cache=True)
        ot = model(nxt, past_key_values=twin, use_cache=True)
        assert torch.equal(ob.logits, ot.logits)
        # the saved cache can still drop the step's rejected tokens
        a.crop(-5)
        twin2 = KiviPackedCache.from_model(model, device="cuda:0", group_size=G,
                                           residual_length=R)
        model(ids, past_key_values=twin2, use_cache=True)
        model(draft, past_key_values=twin2, use_cache=True)
        twin2.crop(-5)
        n = draft[:, 1:2]
        for _ in range(20):
            oa = model(n, past_key_values=a, use_cache=True)
            o2 = model(n, past_key_values=twin2, use_cache=True)
            assert torch.equal(oa.logits, o2.logits)
            n = oa.logits[:, -1:].argmax(-1)
