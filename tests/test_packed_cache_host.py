"""Host checks of KiviPackedCache, the transformers.Cache whose decode attention
reads the packed store.  The GPU store is replaced by a CPU stand-in built on
the oracle (tests/cpu_store.py), so these tests exercise the cache's control
flow -- when tokens are appended, attended and flushed -- against the
reference's generate()/KiviCache flow (oracle restatement of
src/kivi_sycl/generation/generate.py:13-89 and cache/manager.py:162-374)."""

import importlib

import pytest
import torch
from transformers import GPT2Config, GPT2LMHeadModel, LlamaConfig, LlamaForCausalLM
from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS

from oracle.kivi_cache import KiviCacheOracle, closed_form_stats
from tests.cpu_store import CpuPackedStore

pc = importlib.import_module("intel_kivi_hybrid_amd.cache.packed_cache")
gen_mod = importlib.import_module("intel_kivi_hybrid_amd.generation.generate")


class _Tok:
    eos_token_id = None

    def __init__(self, vocab):
        self.vocab = vocab

    def __call__(self, prompt, return_tensors="pt"):
        ids = torch.tensor([[(ord(c) * 131 + 7 * i) % self.vocab for i, c in enumerate(prompt)]])
        return type("Enc", (), {"input_ids": ids})()

    def decode(self, ids, skip_special_tokens=True):
        return " ".join(str(int(t)) for t in ids)


class _OracleShim(KiviCacheOracle):
    @classmethod
    def from_model(cls, model, device="cuda", group_size=32, residual_length=128):
        from intel_kivi_hybrid_amd.config import detect_model_config
        cfg = detect_model_config(model)
        return cls(cfg["num_layers"], cfg["head_dim"], cfg["num_kv_heads"], group_size,
                   residual_length)


@pytest.fixture
def cpu_store(monkeypatch):
    monkeypatch.setattr(pc, "_STORE_CLASS", CpuPackedStore)
    monkeypatch.setattr(pc, "_resolve_device", lambda d: torch.device("cpu"))


def _gpt2(layers=4, heads=4, embd=256, seed=0):
    torch.manual_seed(seed)
    return GPT2LMHeadModel(GPT2Config(n_layer=layers, n_head=heads, n_embd=embd)).eval()


def test_registered_with_transformers():
    pc.register_packed_attention()
    assert ALL_ATTENTION_FUNCTIONS[pc.KIVI_ATTENTION] is pc.kivi_packed_attention_forward
    assert pc.KIVI_ATTENTION in ALL_MASK_ATTENTION_FUNCTIONS
    model = _gpt2(2, 2, 64)
    with pc.packed_attention(model):
        assert model.config._attn_implementation == pc.KIVI_ATTENTION
    assert model.config._attn_implementation == "sdpa"


def test_signature_matches_generate():
    import inspect
    a = inspect.signature(gen_mod.generate).parameters
    b = inspect.signature(gen_mod.generate_packed).parameters
    assert list(a) == list(b)
    assert all(a[n].default == b[n].default for n in a)


@pytest.mark.parametrize("R,prompt_len,max_new", [(32, 9, 90), (64, 70, 80), (32, 32, 40)])
def test_generate_packed_follows_reference_flow(cpu_store, monkeypatch, R, prompt_len, max_new):
    """Token for token, generate_packed (model-driven cache updates, attention
    from the store, flush after the step's attention) picks what the
    reference's generate() picks with its served fp32 cache."""
    model = _gpt2()
    tok = _Tok(model.config.vocab_size)
    prompt = ("The quick brown fox jumps over the lazy dog " * 4)[:prompt_len]
    ours = gen_mod.generate_packed(model, tok, prompt, max_new_tokens=max_new, group_size=32,
                                   residual_length=R, device="cuda")
    monkeypatch.setattr(gen_mod, "KiviCache", _OracleShim)
    ref = gen_mod.generate(model, tok, prompt, max_new_tokens=max_new, group_size=32,
                           residual_length=R, device="cuda")
    assert ours.split() == ref.split()


def test_cache_state_matches_reference_after_each_step(cpu_store):
    """After every forward pass the packed cache holds what the reference's
    KiviCache holds after add_tokens(): the same quantised/residual split in
    every layer, and in layer 0 (whose K/V depend only on the tokens) the
    same dequantised history and residual, bit for bit.  Deeper layers see
    K/V computed from attention outputs, which differ in the last bits
    between the float64 oracle attention and the reference flow's fp32 SDPA."""
    model = _gpt2(3, 4, 128, seed=3)
    G, R = 32, 64
    ours = pc.KiviPackedCache.from_model(model, group_size=G, residual_length=R)
    ref = _OracleShim.from_model(model, group_size=G, residual_length=R)
    ids = torch.randint(0, model.config.vocab_size, (2, 75), generator=torch.Generator().manual_seed(5))
    with torch.no_grad(), pc.packed_attention(model):
        out = model(ids, past_key_values=ours, use_cache=True)
    with torch.no_grad():
        ref_out = model(ids, use_cache=True)
    ref.add_tokens(ref_out.past_key_values)
    nxt = out.logits[:, -1:].argmax(-1)
    for step in range(70):
        for i in range(3):
            st = ours.store(i)
            k, v = list(ref.get_full_cache().layers)[i].keys, list(ref.get_full_cache().layers)[i].values
            n_hist = st.quantized_tokens
            assert st.res_len == k.shape[2] - n_hist
            if i:
                continue
            assert torch.equal(st.hist_k, k[:, :, :n_hist]) and torch.equal(st.hist_v, v[:, :, :n_hist])
            assert torch.equal(st.res_k, k[:, :, n_hist:]) and torch.equal(st.res_v, v[:, :, n_hist:])
        s_ours, s_ref = ours.get_stats(0), ref.get_stats(0)
        for key in ("total_tokens", "quantized_tokens", "residual_tokens", "kivi_bytes",
                    "fp32_bytes"):
            assert s_ours[key] == s_ref[key], key
        with torch.no_grad(), pc.packed_attention(model):
            out = model(nxt, past_key_values=ours, use_cache=True)
        with torch.no_grad():
            ref_out = model(nxt, past_key_values=ref.get_full_cache(), use_cache=True)
        ref.add_tokens(ref_out.past_key_values)
        nxt = out.logits[:, -1:].argmax(-1)
    assert ours.total_flushes == ref.total_flushes
    assert ours.get_seq_length() == 75 + 70


def test_stats_closed_form(cpu_store):
    """get_stats byte counts follow the flush formula (manager.py:350-356)."""
    B, H, D, G, R = 1, 12, 64, 32, 32
    cache = pc.KiviPackedCache(12, D, H, group_size=G, residual_length=R)
    for t in range(200):
        for i in range(12):
            k = torch.randn(B, H, 1, D)
            cache.update(k, k.clone(), i)
            cache.layers[i]._awaiting_attention = False
            cache.layers[i].settle()
    s = cache.get_stats(0)
    expect = closed_form_stats(B, H, D, G, R, 200)
    for key in ("total_tokens", "quantized_tokens", "residual_tokens", "kivi_bytes",
                "fp32_bytes"):
        assert s[key] == expect[key], key
    assert s["compression"] == pytest.approx(6.25)
    assert cache.total_flushes == 12 * 6


def test_wrong_attention_is_detected(cpu_store):
    """A decode step run with another attention implementation sees only the
    new token; the cache refuses the next update instead of going on."""
    model = _gpt2(2, 2, 64)
    cache = pc.KiviPackedCache.from_model(model, group_size=32, residual_length=32)
    ids = torch.tensor([[1, 2, 3, 4]])
    with torch.no_grad():
        with pc.packed_attention(model):
            model(ids, past_key_values=cache, use_cache=True)
        model(torch.tensor([[5]]), past_key_values=cache, use_cache=True)   # plain sdpa
        with pytest.raises(RuntimeError, match="did not run"):
            model(torch.tensor([[6]]), past_key_values=cache, use_cache=True)


def test_unsupported_inputs_raise(cpu_store):
    model = _gpt2(2, 2, 64)
    cache = pc.KiviPackedCache.from_model(model, group_size=32, residual_length=32)
    with torch.no_grad(), pc.packed_attention(model):
        with pytest.raises(RuntimeError, match="KiviPackedCache"):
            model(torch.tensor([[1, 2, 3]]), use_cache=False)
    with pytest.raises(ValueError, match="head_dim"):
        bad = pc.KiviPackedCache(2, 64, 2, group_size=32, residual_length=32)
        bad.update(torch.zeros(1, 2, 3, 48), torch.zeros(1, 2, 3, 48), 0)


def test_hole_mask_follows_reference_flow(cpu_store):
    """A mask with holes (positions hidden inside the context) reaches the
    store as hidden-position words, and the logits are the reference flow's
    (HF SDPA with the same mask over get_full_cache())."""
    model = _gpt2(2, 2, 64, seed=3)
    G, R = 32, 32
    cache = pc.KiviPackedCache.from_model(model, group_size=G, residual_length=R)
    ref = _OracleShim.from_model(model, group_size=G, residual_length=R)
    gen = torch.Generator().manual_seed(4)
    ids = torch.randint(1, model.config.vocab_size, (2, 40), generator=gen)
    mask = torch.ones(2, 40, dtype=torch.long)
    mask[0, 3:9] = 0
    mask[1, 20:39] = 0                      # right padding before the last prompt token
    with torch.no_grad(), pc.packed_attention(model):
        model(ids, past_key_values=cache, use_cache=True, attention_mask=mask)
    with torch.no_grad():
        ref.add_tokens(model(ids, use_cache=True, attention_mask=mask).past_key_values)
    for n in (1, 1, 3, 1, 1):
        new = torch.randint(1, model.config.vocab_size, (2, n), generator=gen)
        mask = torch.cat([mask, torch.ones(2, n, dtype=torch.long)], dim=1)
        with torch.no_grad(), pc.packed_attention(model):
            lo = model(new, past_key_values=cache, use_cache=True, attention_mask=mask).logits
        with torch.no_grad():
            out = model(new, past_key_values=ref.get_full_cache(), use_cache=True,
                        attention_mask=mask)
        ref.add_tokens(out.past_key_values)
        err = ((lo - out.logits).abs().max() / out.logits.abs().max()).item()
        assert err <= 1e-4, (n, err)
        for lay in cache.layers:
            lay.settle()
    assert cache._mask_memo[1][1] is not None       # hidden words, not kv_start


def _hf_mask(attend):
    return attend[:, None]                            # [B, 1, q_len, kv_len]


def test_mask_plan_paths():
    """HF masks as the packed kernels take them: a leading hidden run is
    kv_start, any other key-padding pattern hidden words (bit p % 32 of word
    p // 32), a 0 / lowest-value float mask the same as the boolean one; an
    additive bias or a per-query pattern other than causal is refused."""
    class Owner:
        _mask_memo = None
    B, L, T = 3, 2, 70
    t = torch.arange(T)
    causal = t[None, :] <= (T - L + torch.arange(L))[:, None]
    lead = t[None, :] >= torch.tensor([0, 5, 40])[:, None]
    kv_start, hidden = pc._mask_plan(Owner(), _hf_mask(lead[:, None] & causal), L, T, "cpu")
    assert hidden is None and kv_start.tolist() == [0, 5, 40]
    vis = lead.clone()
    vis[0, 33] = False                                # a hole in the second word
    vis[2, 64:68] = False                             # right padding before the new tokens
    kv_start, hidden = pc._mask_plan(Owner(), _hf_mask(vis[:, None] & causal), L, T, "cpu")
    assert kv_start is None and hidden.dtype == torch.int32 and hidden.shape == (B, 3)
    w = hidden.numpy().astype("uint32")
    for b in range(B):
        for p in range(T):
            assert bool((w[b, p // 32] >> (p % 32)) & 1) == (not bool(vis[b, p])), (b, p)
    low = torch.finfo(torch.float32).min
    fm = torch.where(vis[:, None] & causal, 0.0, low)[:, None]
    kv2, hidden2 = pc._mask_plan(Owner(), fm, L, T, "cpu")
    assert kv2 is None and torch.equal(hidden2, hidden)
    with pytest.raises(NotImplementedError, match="padded batch"):
        pc._mask_plan(Owner(), torch.where(vis[:, None] & causal, 0.5, low)[:, None], L, T, "cpu")
    odd = (vis[:, None] & causal).clone()
    odd[1, 0, 10] = False                             # the first query hides one more position
    with pytest.raises(NotImplementedError, match="padded batch"):
        pc._mask_plan(Owner(), _hf_mask(odd), L, T, "cpu")


def test_hf_generate_uses_the_cache(cpu_store):
    """transformers' own generate() drives the cache: greedy output equals
    generate_packed's for the same prompt."""
    model = _gpt2(3, 4, 128, seed=7)
    tok = _Tok(model.config.vocab_size)
    prompt = "hello packed world"
    ours = gen_mod.generate_packed(model, tok, prompt, max_new_tokens=50, group_size=32,
                                   residual_length=32)
    ids = tok(prompt).input_ids
    cache = pc.KiviPackedCache.from_model(model, group_size=32, residual_length=32)
    with pc.packed_attention(model):
        hf = model.generate(ids, past_key_values=cache, max_new_tokens=50, do_sample=False,
                            attention_mask=torch.ones_like(ids), pad_token_id=0)
    assert tok.decode(hf[0]).split() == ours.split()
    assert cache.get_seq_length() == ids.shape[1] + 49


def test_gqa_model(cpu_store, monkeypatch):
    """A grouped-query Llama (8 query heads over 2 kv heads) through the
    packed cache picks the reference flow's tokens."""
    torch.manual_seed(11)
    cfg = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2,
                      max_position_embeddings=512)
    model = LlamaForCausalLM(cfg).eval()
    tok = _Tok(cfg.vocab_size)
    ours = gen_mod.generate_packed(model, tok, "grouped query heads", max_new_tokens=60,
                                   group_size=32, residual_length=32)
    monkeypatch.setattr(gen_mod, "KiviCache", _OracleShim)
    ref = gen_mod.generate(model, tok, "grouped query heads", max_new_tokens=60,
                           group_size=32, residual_length=32)
    assert ours.split() == ref.split()


def test_unsupported_geometry_refused_up_front(cpu_store):
    """Geometries the decode kernel cannot run are refused when the cache is
    built, not at the first decode step after the prompt has been stored."""
    from intel_kivi_hybrid_amd.store import decode_geometry_error
    with pytest.raises(ValueError, match="group_size_k 8"):
        pc.KiviPackedCache(2, 64, 2, group_size=8, residual_length=32)
    with pytest.raises(ValueError, match="head_dim 72"):
        pc.KiviPackedCache(2, 72, 2, group_size=8, residual_length=32)
    with pytest.raises(ValueError, match="head_dim 512"):
        pc.KiviPackedCache(2, 512, 2, group_size=32, residual_length=32)
    assert decode_geometry_error(8, 2, 128, 32, 32) is None
    assert decode_geometry_error(4, 4, 64, 32, 64) is None
    assert decode_geometry_error(6, 2, 64, 32, 32) is None         # any head ratio
    assert decode_geometry_error(40, 1, 128, 32, 32) is None
    assert "multiple of kv_heads" in decode_geometry_error(6, 4, 64, 32, 32)
    assert "needs" in decode_geometry_error(8, 1, 256, 64, 32)     # LDS beyond the device's


def _ref_step(model, ref, ids):
    with torch.no_grad():
        out = model(ids, past_key_values=ref.get_full_cache(), use_cache=True)
    ref.add_tokens(out.past_key_values)
    return out.logits


def _check_layer0(ours, ref):
    """Layer 0's store equals the reference's KiviCache bit for bit once the
    flushes a multi-token step leaves to the next update are done."""
    lay = ours.layers[0]
    lay.settle()
    st = ours.store(0)
    k, v = list(ref.get_full_cache().layers)[0].keys, list(ref.get_full_cache().layers)[0].values
    n_hist = st.quantized_tokens
    assert st.res_len == k.shape[2] - n_hist
    assert torch.equal(st.hist_k, k[:, :, :n_hist]) and torch.equal(st.hist_v, v[:, :, :n_hist])
    assert torch.equal(st.res_k, k[:, :, n_hist:]) and torch.equal(st.res_v, v[:, :, n_hist:])


@pytest.mark.parametrize("steps", [[5, 1, 3, 8, 1, 1, 17, 2, 1, 30, 4], [64, 1, 63, 2]])
def test_multitoken_steps_follow_reference_flow(cpu_store, steps):
    """Forwards of several tokens on a non-empty cache (chunked prefill)
    attend causally over [history ; window ; new tokens] like the reference
    flow's forward over get_full_cache(), and leave the same store once its
    flushes are done: logits agree to float rounding (the stand-in attends in
    float64, the reference flow in fp32 SDPA) and layer 0's history and
    window bit for bit."""
    model = _gpt2(3, 4, 128, seed=9)
    G, R = 32, 64
    ours = pc.KiviPackedCache.from_model(model, group_size=G, residual_length=R)
    ref = _OracleShim.from_model(model, group_size=G, residual_length=R)
    gen = torch.Generator().manual_seed(10)
    ids = torch.randint(0, model.config.vocab_size, (2, 40), generator=gen)
    with torch.no_grad(), pc.packed_attention(model):
        model(ids, past_key_values=ours, use_cache=True)
    _ref_step(model, ref, ids)
    total = 40
    for n in steps:
        chunk = torch.randint(0, model.config.vocab_size, (2, n), generator=gen)
        with torch.no_grad(), pc.packed_attention(model):
            lo = model(chunk, past_key_values=ours, use_cache=True).logits
        lr = _ref_step(model, ref, chunk)
        total += n
        assert lo.shape == lr.shape
        torch.testing.assert_close(lo, lr, rtol=1e-4, atol=1e-4)
        assert ours.get_seq_length() == total
        _check_layer0(ours, ref)
    assert ours.total_flushes == ref.total_flushes


def test_crop_drops_a_steps_rejected_tokens(cpu_store):
    """crop() after a multi-token step (assisted decoding's verification
    pass) drops its rejected tokens: the cache then continues exactly as if
    only the accepted tokens had been fed, here across a flush boundary
    (the step takes the window past R, the crop brings it back)."""
    model = _gpt2(2, 4, 128, seed=12)
    G, R = 32, 64
    ours = pc.KiviPackedCache.from_model(model, group_size=G, residual_length=R)
    ref = _OracleShim.from_model(model, group_size=G, residual_length=R)
    gen = torch.Generator().manual_seed(13)
    ids = torch.randint(0, model.config.vocab_size, (1, 60), generator=gen)
    with torch.no_grad(), pc.packed_attention(model):
        model(ids, past_key_values=ours, use_cache=True)
    _ref_step(model, ref, ids)
    res0 = ours.store(0).res_len
    draft = torch.randint(0, model.config.vocab_size, (1, 7), generator=gen)
    with torch.no_grad(), pc.packed_attention(model):
        model(draft, past_key_values=ours, use_cache=True)
    assert ours.store(0).res_len == res0 + 7          # flushes wait for the next update
    ours.crop(-5)                                     # two drafts accepted
    assert ours.get_seq_length() == 62
    _ref_step(model, ref, draft[:, :2])
    nxt = torch.randint(0, model.config.vocab_size, (1, 1), generator=gen)
    for step in range(40):
        with torch.no_grad(), pc.packed_attention(model):
            lo = model(nxt, past_key_values=ours, use_cache=True).logits
        lr = _ref_step(model, ref, nxt)
        torch.testing.assert_close(lo, lr, rtol=1e-4, atol=1e-4)
        _check_layer0(ours, ref)
        nxt = lo[:, -1:].argmax(-1)
    # the legacy positive form keeps that many tokens
    ours.crop(ours.get_seq_length() - 1)
    assert ours.get_seq_length() == 60 + 2 + 40 - 1
    # quantised tokens cannot be dropped
    with pytest.raises(ValueError, match="cannot roll back"):
        ours.crop(-(ours.store(0).res_len + 1))


def test_hf_assisted_generation(cpu_store):
    """transformers' assisted generation (a 1-layer draft proposing 3 tokens
    per step) drives the cache with verification passes of several tokens and
    crop() of the rejected drafts; greedy output equals plain greedy
    generation with the same cache type."""
    model = _gpt2(3, 4, 128, seed=7)
    draft = _gpt2(1, 4, 128, seed=7)
    draft.generation_config.num_assistant_tokens = 3
    draft.generation_config.num_assistant_tokens_schedule = "constant"
    draft.generation_config.assistant_confidence_threshold = 0.0
    ids = torch.randint(0, model.config.vocab_size, (1, 20),
                        generator=torch.Generator().manual_seed(1))
    sizes, crops = [], []
    update, crop = pc.KiviPackedLayer.update, pc.KiviPackedLayer.crop

    def spy_update(self, k, v, *a, **kw):
        if self.index == 0:
            sizes.append(k.shape[2])
        return update(self, k, v, *a, **kw)

    def spy_crop(self, n):
        if self.index == 0:
            crops.append(int(n))
        return crop(self, n)

    outs = []
    for assistant in (None, draft):
        sizes.clear()
        crops.clear()
        cache = pc.KiviPackedCache.from_model(model, group_size=32, residual_length=32)
        kw = {} if assistant is None else {"assistant_model": assistant}
        pc.KiviPackedLayer.update, pc.KiviPackedLayer.crop = spy_update, spy_crop
        try:
            with pc.packed_attention(model):
                outs.append(model.generate(ids, past_key_values=cache, max_new_tokens=60,
                                           do_sample=False, attention_mask=torch.ones_like(ids),
                                           pad_token_id=0, **kw))
        finally:
            pc.KiviPackedLayer.update, pc.KiviPackedLayer.crop = update, crop
        assert cache.get_seq_length() == ids.shape[1] + 59
    assert max(sizes[1:]) > 2 and any(c < 0 for c in crops)
    assert torch.equal(outs[0], outs[1])


def _padded_batch(vocab, lengths, gen):
    """Left-padded prompts: ids [B, T] (pad id 0), attention mask, positions
    as transformers' generate() makes them (cumsum of the mask - 1)."""
    T = max(lengths)
    ids = torch.zeros(len(lengths), T, dtype=torch.long)
    mask = torch.zeros(len(lengths), T, dtype=torch.long)
    for b, n in enumerate(lengths):
        ids[b, T - n:] = torch.randint(1, vocab, (n,), generator=gen)
        mask[b, T - n:] = 1
    return ids, mask


def _positions(mask, n):
    pos = mask.cumsum(-1) - 1
    return pos.clamp(min=0)[:, -n:]


@pytest.mark.parametrize("steps", [[1] * 40, [1, 3, 1, 1, 9, 1, 2, 1, 1, 1, 30, 1]])
def test_left_padded_batch_follows_reference_flow(cpu_store, steps):
    """A left-padded batch (prompts of 50, 37 and 12 tokens): every forward
    after the prompt hides each sequence's pad positions through HF's
    boolean mask, which the packed attention turns into a per-sequence first
    visible position.  Logits equal the reference flow's (HF SDPA with the
    same mask over get_full_cache()) to float rounding, and layer 0's store
    (pad tokens included, as the reference's add_tokens stores them) bit for
    bit, over one-token and multi-token steps across several flushes."""
    model = _gpt2(3, 4, 128, seed=21)
    G, R = 32, 64
    ours = pc.KiviPackedCache.from_model(model, group_size=G, residual_length=R)
    ref = _OracleShim.from_model(model, group_size=G, residual_length=R)
    gen = torch.Generator().manual_seed(22)
    ids, mask = _padded_batch(model.config.vocab_size, [50, 37, 12], gen)
    kw = dict(attention_mask=mask, position_ids=_positions(mask, ids.shape[1]), use_cache=True)
    with torch.no_grad(), pc.packed_attention(model):
        lo = model(ids, past_key_values=ours, **kw).logits
    with torch.no_grad():
        out = model(ids, **kw)
    ref.add_tokens(out.past_key_values)
    torch.testing.assert_close(lo, out.logits, rtol=1e-5, atol=1e-5)
    for n in steps:
        new = torch.randint(1, model.config.vocab_size, (3, n), generator=gen)
        mask = torch.cat([mask, torch.ones(3, n, dtype=torch.long)], dim=1)
        kw = dict(attention_mask=mask, position_ids=_positions(mask, n), use_cache=True)
        with torch.no_grad(), pc.packed_attention(model):
            lo = model(new, past_key_values=ours, **kw).logits
        with torch.no_grad():
            out = model(new, past_key_values=ref.get_full_cache(), **kw)
        ref.add_tokens(out.past_key_values)
        torch.testing.assert_close(lo, out.logits, rtol=1e-4, atol=1e-4)
        _check_layer0(ours, ref)
    assert ours.total_flushes == ref.total_flushes > 0


def test_hf_generate_left_padded_batch(cpu_store):
    """transformers' generate() on a left-padded batch of prompts drives the
    packed cache (padding mask on every step) to the tokens of a greedy loop
    over the reference flow with the same masks and positions."""
    model = _gpt2(3, 4, 128, seed=31)
    G, R = 32, 32
    gen = torch.Generator().manual_seed(32)
    ids, mask = _padded_batch(model.config.vocab_size, [23, 9], gen)
    new_tokens = 40
    cache = pc.KiviPackedCache.from_model(model, group_size=G, residual_length=R)
    with pc.packed_attention(model):
        hf = model.generate(ids, attention_mask=mask, past_key_values=cache,
                            max_new_tokens=new_tokens, do_sample=False, pad_token_id=0)
    # the reference flow, step by step
    ref = _OracleShim.from_model(model, group_size=G, residual_length=R)
    kw = dict(attention_mask=mask, position_ids=_positions(mask, ids.shape[1]), use_cache=True)
    with torch.no_grad():
        out = model(ids, **kw)
    ref.add_tokens(out.past_key_values)
    toks = [out.logits[:, -1:].argmax(-1)]
    for _ in range(new_tokens - 1):
        mask = torch.cat([mask, torch.ones(2, 1, dtype=torch.long)], dim=1)
        kw = dict(attention_mask=mask, position_ids=_positions(mask, 1), use_cache=True)
        with torch.no_grad():
            out = model(toks[-1], past_key_values=ref.get_full_cache(), **kw)
        ref.add_tokens(out.past_key_values)
        toks.append(out.logits[:, -1:].argmax(-1))
    assert torch.equal(hf[:, ids.shape[1]:], torch.cat(toks, dim=1))
    assert cache.total_flushes == ref.total_flushes > 0
