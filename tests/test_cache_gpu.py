"""GPU parity of the HBM-resident KiviCache and generate() against the CPU
restatement of the reference's KiviCache (oracle/kivi_cache.py).

Bars: the served cache (get_full_cache) is bit-identical to the oracle's at
every decode step, flush counts and get_stats match exactly, the packed store
holds exactly the oracle codec's codes/scales/zeros, fused attention through
the cache is within 1e-3 relative of float64 attention over the served K/V,
and greedy generation on a seeded GPT-2-shaped model yields the same tokens
as the reference control flow (100 % match).
"""

import numpy as np
import pytest
import torch

from oracle.attention import decode_attention
from oracle.kivi_cache import KiviCacheOracle, closed_form_stats, iter_kv_layers
from tests.conftest import seeded_kv
from tests.fake_model import FakeModel, iter_layers
from tests.kv_helpers import oracle_chunk, rel_err, seeded_q

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def KiviCache(hip_device):
    from intel_kivi_hybrid_amd import KiviCache as cls
    return cls


def _served_equal(ours, ref, where):
    a, b = iter_layers(ours), iter_layers(ref)
    assert len(a) == len(b), where
    for i, ((ka, va), (kb, vb)) in enumerate(zip(a, b)):
        assert ka.shape == kb.shape, f"{where} layer {i}: {tuple(ka.shape)} vs {tuple(kb.shape)}"
        assert torch.equal(ka.cpu(), kb.cpu()), f"{where} layer {i}: keys differ"
        assert torch.equal(va.cpu(), vb.cpu()), f"{where} layer {i}: values differ"


def _lockstep(KiviCache, mode, layers, B, H, D, G, R, prefill, steps, model_device="cpu"):
    print(f"[cache] mode={mode} layers={layers} B={B} H={H} D={D} G={G} R={R} "
          f"prefill={prefill} steps={steps} model_device={model_device}", flush=True)
    ours = KiviCache(layers, D, H, device="cuda:0", group_size=G, residual_length=R)
    ref = KiviCacheOracle(layers, D, H, G, R)
    m_ours = FakeModel(layers, H, D, mode, batch=B, seed=11, device=model_device)
    m_ref = FakeModel(layers, H, D, mode, batch=B, seed=11)
    ours.add_tokens(m_ours.forward(prefill))
    ref.add_tokens(m_ref.forward(prefill))
    for step in range(steps):
        p_ours, p_ref = ours.get_full_cache(), ref.get_full_cache()
        _served_equal(p_ours, p_ref, f"step {step}")
        for k, _ in iter_layers(p_ours):
            assert k.device.type == torch.device(model_device).type
        ours.add_tokens(m_ours.forward(1, p_ours))
        ref.add_tokens(m_ref.forward(1, p_ref))
    _served_equal(ours.get_full_cache(), ref.get_full_cache(), "final")
    assert ours.total_flushes == ref.total_flushes
    for i in range(layers):
        assert ours.get_stats(i) == ref.get_stats(i)
    return ours, ref


@pytest.mark.parametrize("mode", ["in_place", "legacy_tuple"])
def test_reference_scenario_geometry(KiviCache, mode):
    """tests/unit/test_manager_bookkeeping.py:147-196 geometry: G=4, R=8, D=8,
    2 layers, 2 heads, prefill 6, 24 steps."""
    ours, _ = _lockstep(KiviCache, mode, 2, 1, 2, 8, 4, 8, 6, 24)
    assert ours.total_flushes > 0


@pytest.mark.parametrize("mode,B,H,D,G,R,prefill,steps,dev", [
    ("in_place", 2, 4, 64, 32, 64, 100, 70, "cpu"),       # prefill flushes several groups
    ("legacy_tuple", 2, 4, 64, 32, 48, 5, 90, "cpu"),     # R not a multiple of G: ring wrap
    ("in_place", 3, 2, 128, 16, 16, 40, 40, "cuda:0"),    # model on the GPU, R == G
    ("legacy_tuple", 1, 3, 32, 8, 24, 1, 60, "cuda:0"),
])
def test_lockstep_shapes(KiviCache, mode, B, H, D, G, R, prefill, steps, dev):
    _lockstep(KiviCache, mode, 2, B, H, D, G, R, prefill, steps, model_device=dev)


def test_desync_and_batch_change_raise(KiviCache):
    c = KiviCache(1, 8, 2, device="cuda:0", group_size=4, residual_length=8)
    m = FakeModel(1, 2, 8, "in_place")
    out = m.forward(5)
    c.add_tokens(out)
    with pytest.raises(AssertionError, match="desync"):
        c.add_tokens(out)
    with pytest.raises(AssertionError, match="batch size changed"):
        c.add_tokens(FakeModel(1, 2, 8, "in_place", batch=3).forward(9))


def test_failed_check_keeps_earlier_layers_tokens(KiviCache):
    """A step whose third layer fails its check (no new token) still files
    the token of the two layers before it, as per-layer appends did; the
    other layers' tokens stay out."""
    from transformers import DynamicCache
    L, B, H, D = 4, 1, 2, 8
    c = KiviCache(L, D, H, device="cuda:0", group_size=4, residual_length=8)
    g = torch.Generator().manual_seed(3)
    k0 = [torch.randn(B, H, 5, D, generator=g).cuda() for _ in range(L)]
    v0 = [torch.randn(B, H, 5, D, generator=g).cuda() for _ in range(L)]
    first = DynamicCache()
    for i in range(L):
        first.update(k0[i], v0[i], i)
    c.add_tokens(first)
    step = DynamicCache()
    for i in range(L):
        n = 5 if i == 2 else 6                      # layer 2 brings no new token
        kx = torch.cat([k0[i], torch.randn(B, H, 1, D, generator=g).cuda()], 2)[:, :, :n]
        vx = torch.cat([v0[i], torch.randn(B, H, 1, D, generator=g).cuda()], 2)[:, :, :n]
        step.update(kx, vx, i)
    with pytest.raises(AssertionError, match="no tokens beyond"):
        c.add_tokens(step)
    assert [c.store(i).res_len for i in range(L)] == [6, 6, 5, 5]
    for i in (0, 1):
        kr, vr = c.store(i).residual()
        assert torch.equal(kr, step.layers[i].keys) and torch.equal(vr, step.layers[i].values)


def test_reset_and_reuse_with_new_batch(KiviCache):
    c = KiviCache(2, 16, 2, device="cuda:0", group_size=4, residual_length=8)
    ref = KiviCacheOracle(2, 16, 2, 4, 8)
    for batch, seed in ((2, 1), (2, 2), (3, 3)):
        c.reset()
        ref.reset()
        m1 = FakeModel(2, 2, 16, "in_place", batch=batch, seed=seed)
        m2 = FakeModel(2, 2, 16, "in_place", batch=batch, seed=seed)
        c.add_tokens(m1.forward(7))
        ref.add_tokens(m2.forward(7))
        for _ in range(20):
            pa, pb = c.get_full_cache(), ref.get_full_cache()
            c.add_tokens(m1.forward(1, pa))
            ref.add_tokens(m2.forward(1, pb))
        _served_equal(c.get_full_cache(), ref.get_full_cache(), f"batch {batch}")
        assert c.get_stats(1) == ref.get_stats(1)


def test_explicit_flush_group(KiviCache):
    c = KiviCache(1, 8, 2, device="cuda:0", group_size=4, residual_length=8)
    c.add_tokens(FakeModel(1, 2, 8, "in_place").forward(5))
    assert c.get_stats(0)["residual_tokens"] == 5
    c._flush_group(0)
    assert c.get_stats(0)["residual_tokens"] == 1 and c.total_flushes == 1
    with pytest.raises(AssertionError, match="Cannot flush 4 tokens"):
        c._flush_group(0)


def test_config1_cache_full_size(KiviCache):
    """Benchmark config 1: GPT-2-small-shaped cache, 12 layers, B=1, H=12,
    D=64, R=G=32, 200 decode steps of seeded K/V with channel/token
    outliers.  Served K/V, packed bytes, scales/zeros and accounting."""
    layers, B, H, D, G, R, T = 12, 1, 12, 64, 32, 32, 200
    print("[cache] config1", flush=True)
    k_all = seeded_kv((B, H, T, D), seed=1235, kind="key")
    v_all = seeded_kv((B, H, T, D), seed=1236, kind="value")
    ours = KiviCache(layers, D, None, device="cuda:0", group_size=G, residual_length=R)
    ref = KiviCacheOracle(layers, D, None, G, R)
    for t in range(T):
        pkv = tuple((k_all[:, :, :t + 1], v_all[:, :, :t + 1]) for _ in range(layers))
        ours.add_tokens(pkv)
        ref.add_tokens(pkv)
    _served_equal(ours.get_full_cache(), ref.get_full_cache(), "config1")
    for i in range(layers):
        s = ours.get_stats(i)
        assert s == ref.get_stats(i) == closed_form_stats(B, H, D, G, R, T)
        assert s["kivi_bytes"] == 196608 and s["fp32_bytes"] == 1228800
    st = ours.store(0)
    assert st.n_chunks == 6 and st.res_len == 8
    for c in range(st.n_chunks):
        o = oracle_chunk(k_all[:, :, c * G:(c + 1) * G], v_all[:, :, c * G:(c + 1) * G], G, G)
        assert np.array_equal(st.unpermuted_k_codes(c).cpu().numpy(), o["k_codes"])
        assert np.array_equal(st.unpermuted_v_codes(c).cpu().numpy(), o["v_codes"])
        got = {"k_scale": st.k_scale[:, :, c], "k_zero": st.k_zero[:, :, c],
               "v_scale": st.chunk_v_scale(c), "v_zero": st.chunk_v_zero(c)}
        for name, t in got.items():
            bits = t.contiguous().cpu().numpy().view(np.uint32)
            assert np.array_equal(bits, o[name].view(np.uint32)), f"{name} chunk {c}"


@pytest.mark.parametrize("Hq", [12, 24])
def test_fused_attention_through_cache(KiviCache, Hq):
    layers, B, H, D, G, R = 2, 2, 12, 64, 32, 64
    ours = KiviCache(layers, D, H, device="cuda:0", group_size=G, residual_length=R)
    m = FakeModel(layers, H, D, "in_place", batch=B, seed=4, jitter=1.0)
    ours.add_tokens(m.forward(150))
    for _ in range(17):
        ours.add_tokens(m.forward(1, ours.get_full_cache()))
    q = seeded_q(B, Hq, D, seed=8)
    for layer in range(layers):
        out = ours.attention(layer, q.cuda())
        torch.cuda.synchronize()
        k, v = iter_layers(ours.get_full_cache())[layer]
        ref = decode_attention(q.numpy(), k.cpu().numpy(), v.cpu().numpy(), None, None)
        err = rel_err(out.cpu().numpy(), ref)
        print(f"[cache] fused attention layer {layer} Hq={Hq} rel_err={err:.2e}", flush=True)
        assert err <= 1e-3
        # a padded batch: holes and right padding over the served context
        T = k.shape[2]
        vis = torch.rand(B, T, generator=torch.Generator().manual_seed(layer)) > 0.25
        vis[1, 60:T - 1] = False
        vis[:, T - 1] = True
        out = ours.attention(layer, q.cuda(), key_mask=vis)
        ref = decode_attention(q.numpy(), k.cpu().numpy(), v.cpu().numpy(), None, None,
                               visible=vis.numpy())
        assert rel_err(out.cpu().numpy(), ref) <= 1e-3


class _FakeTokenizer:
    """Prompt -> fixed ids; decode -> space-joined ids (no vocabulary needed)."""
    eos_token_id = None

    def __init__(self, vocab):
        self.vocab = vocab

    def __call__(self, prompt, return_tensors="pt"):
        ids = torch.tensor([[(ord(c) * 131 + 7 * i) % self.vocab for i, c in enumerate(prompt)]])
        return type("Enc", (), {"input_ids": ids})()

    def decode(self, ids, skip_special_tokens=True):
        return " ".join(str(int(t)) for t in ids)


class _OracleCacheShim(KiviCacheOracle):
    """The reference control flow (oracle) behind KiviCache.from_model."""

    @classmethod
    def from_model(cls, model, device="cuda", group_size=32, residual_length=128):
        from intel_kivi_hybrid_amd.config import detect_model_config
        cfg = detect_model_config(model)
        return cls(cfg["num_layers"], cfg["head_dim"], cfg["num_kv_heads"], group_size,
                   residual_length)


@pytest.mark.parametrize("R,max_new", [(32, 200), (64, 200)])
def test_greedy_tokens_match_reference_flow(hip_device, monkeypatch, R, max_new):
    """generate() on a seeded random GPT-2-shaped model (12 layers, 12 heads,
    D=64), model on the CPU in both arms as in the reference: the HBM cache
    and the reference's control flow must pick the same greedy tokens."""
    import importlib
    from transformers import GPT2Config, GPT2LMHeadModel
    gen_mod = importlib.import_module("intel_kivi_hybrid_amd.generation.generate")
    torch.manual_seed(0)
    model = GPT2LMHeadModel(GPT2Config(n_layer=12, n_head=12, n_embd=768)).eval()
    tok = _FakeTokenizer(model.config.vocab_size)
    prompt = "The quick brown fox jumps over the lazy dog and"
    print(f"[greedy] R={R} max_new={max_new}", flush=True)
    ours = gen_mod.generate(model, tok, prompt, max_new_tokens=max_new, group_size=32,
                            residual_length=R, device="cuda:0")
    monkeypatch.setattr(gen_mod, "KiviCache", _OracleCacheShim)
    ref = gen_mod.generate(model, tok, prompt, max_new_tokens=max_new, group_size=32,
                           residual_length=R, device="cuda:0")
    a, b = ours.split(), ref.split()
    match = sum(x == y for x, y in zip(a, b)) / max(len(a), len(b))
    print(f"[greedy] {len(a)} ids, token match {100 * match:.1f} %", flush=True)
    assert a == b


def test_generate_with_model_on_gpu(hip_device):
    from transformers import GPT2Config, GPT2LMHeadModel
    from intel_kivi_hybrid_amd import generate
    torch.manual_seed(1)
    model = GPT2LMHeadModel(GPT2Config(n_layer=4, n_head=4, n_embd=256)).eval().to("cuda:0")
    tok = _FakeTokenizer(model.config.vocab_size)
    text = generate(model, tok, "hello there", max_new_tokens=80, group_size=32,
                    residual_length=32, device="cuda:0")
    assert len(text.split()) == len("hello there") + 80
