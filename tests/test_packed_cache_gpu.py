"""GPU parity of KiviPackedCache + the "kivi_packed" attention (the model's
attention reads the 2-bit HBM store through the fused HIP kernel).

Greedy decoding must pick the tokens the reference's generate() picks with
its served fp32 cache (src/kivi_sycl/generation/generate.py:13-89,
cache/manager.py:162-374), here restated by the CPU oracle, and the tokens of
this package's served-cache generate()."""

import importlib

import pytest
import torch

from oracle.kivi_cache import KiviCacheOracle

pytestmark = pytest.mark.gpu

gen_mod = importlib.import_module("intel_kivi_hybrid_amd.generation.generate")
pc = importlib.import_module("intel_kivi_hybrid_amd.cache.packed_cache")


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


def _match(a, b):
    n = sum(x == y for x, y in zip(a, b))
    return n, max(len(a), len(b))


@torch.no_grad()
def _served_step_logits(model, tok, prompt, tokens, step, R, G=32):
    """Logits of the served-cache flow (this package's generate(), the
    reference's control flow) at generated step ``step``, replaying the first
    ``step`` generated tokens of ``tokens`` (prompt + completion, as ids)."""
    from intel_kivi_hybrid_amd import KiviCache
    dev = next(model.parameters()).device
    ids = tok(prompt).input_ids.to(dev)
    n_prompt = ids.shape[1]
    cache = KiviCache.from_model(model, device="cuda:0", group_size=G, residual_length=R)
    out = model(ids, use_cache=True)
    cache.add_tokens(out.past_key_values)
    for j in range(step):
        nxt = torch.tensor([[int(tokens[n_prompt + j])]], device=dev)
        out = model(nxt, past_key_values=cache.get_full_cache(), use_cache=True)
        cache.add_tokens(out.past_key_values)
    return out.logits[0, -1].float()


def _assert_greedy_agrees(model, tok, prompt, ours, ref, R, tol=1e-3):
    """Greedy token lists ``ours`` and ``ref`` (prompt + completion) agree,
    or first differ at a step where the reference flow's two best logits lie
    within ``tol`` (relative to the largest |logit|, the logits bar this file
    holds the packed path to) and ours picked the other of the two: a near
    tie that fp32 rounding of either attention may break either way, after
    which the sequences follow different contexts."""
    if ours == ref:
        return
    assert len(ours) == len(ref)
    i = next(j for j, (x, y) in enumerate(zip(ours, ref)) if x != y)
    n_prompt = tok(prompt).input_ids.shape[1]
    logits = _served_step_logits(model, tok, prompt, ref, i - n_prompt, R)
    top2 = torch.topk(logits, 2)
    gap = ((top2.values[0] - top2.values[1]) / logits.abs().max()).item()
    print(f"[greedy] first difference at token {i}: ref {ref[i]} ours {ours[i]}, "
          f"reference top-2 gap {gap:.2e} (relative)", flush=True)
    assert int(ref[i]) == int(top2.indices[0])
    assert int(ours[i]) == int(top2.indices[1]) and gap <= tol, "not a near tie"


@pytest.mark.parametrize("R,max_new", [(32, 200), (64, 200)])
def test_packed_generate_matches_reference_flow(hip_device, monkeypatch, R, max_new):
    """12-layer GPT-2 shape (12 heads, D=64), model on the CPU in both arms as
    in the reference; the packed arm's decode attention runs on the GPU."""
    from transformers import GPT2Config, GPT2LMHeadModel
    torch.manual_seed(0)
    model = GPT2LMHeadModel(GPT2Config(n_layer=12, n_head=12, n_embd=768)).eval()
    tok = _Tok(model.config.vocab_size)
    prompt = "The quick brown fox jumps over the lazy dog and"
    print(f"[packed-greedy] R={R} max_new={max_new}", flush=True)
    ours = gen_mod.generate_packed(model, tok, prompt, max_new_tokens=max_new, group_size=32,
                                   residual_length=R, device="cuda:0")
    monkeypatch.setattr(gen_mod, "KiviCache", _OracleShim)
    ref = gen_mod.generate(model, tok, prompt, max_new_tokens=max_new, group_size=32,
                           residual_length=R, device="cuda:0")
    n, tot = _match(ours.split(), ref.split())
    print(f"[packed-greedy] token match {n}/{tot}", flush=True)
    assert ours.split() == ref.split()


def test_packed_generate_model_on_gpu(hip_device):
    """Model on the GPU: generate_packed picks the tokens of the served-cache
    generate() (the same model forward, attention over the store vs SDPA
    over the served fp32 history)."""
    from transformers import GPT2Config, GPT2LMHeadModel
    torch.manual_seed(1)
    model = GPT2LMHeadModel(GPT2Config(n_layer=6, n_head=12, n_embd=768)).eval().to(hip_device)
    tok = _Tok(model.config.vocab_size)
    prompt = "hello there, packed cache"
    a = gen_mod.generate_packed(model, tok, prompt, max_new_tokens=150, group_size=32,
                                residual_length=64, device="cuda:0").split()
    b = gen_mod.generate(model, tok, prompt, max_new_tokens=150, group_size=32,
                         residual_length=64, device="cuda:0").split()
    n, tot = _match(a, b)
    print(f"[packed-gpu] token match {n}/{tot}", flush=True)
    assert a == b


def test_hf_generate_with_packed_cache(hip_device):
    """transformers' generate() with a KiviPackedCache equals generate_packed."""
    from transformers import GPT2Config, GPT2LMHeadModel
    torch.manual_seed(2)
    model = GPT2LMHeadModel(GPT2Config(n_layer=4, n_head=4, n_embd=256)).eval().to(hip_device)
    tok = _Tok(model.config.vocab_size)
    prompt = "transformers drives the cache"
    ours = gen_mod.generate_packed(model, tok, prompt, max_new_tokens=100, group_size=32,
                                   residual_length=32, device="cuda:0").split()
    ids = tok(prompt).input_ids.to(hip_device)
    cache = pc.KiviPackedCache.from_model(model, device="cuda:0", group_size=32,
                                          residual_length=32)
    with pc.packed_attention(model):
        hf = model.generate(ids, past_key_values=cache, max_new_tokens=100, do_sample=False,
                            attention_mask=torch.ones_like(ids), pad_token_id=0)
    assert tok.decode(hf[0].cpu()).split() == ours
    st = cache.get_stats(0)
    assert st["total_tokens"] == ids.shape[1] + 99
    assert cache.total_flushes == 4 * ((st["total_tokens"] - 32) // 32 + 1)


@pytest.mark.parametrize("heads,kv_heads", [(14, 2), (16, 1)])
def test_any_head_ratio_llama_logits(hip_device, heads, kv_heads):
    """Llama layers with 7 query heads per kv head (the Qwen2-7B grouping)
    and with one kv head (multi-query), model on the GPU in fp32: fed the
    same tokens, the packed cache's logits (fused decode kernel) match the
    served cache's (HF attention over the dequantised history) at every
    step, across several flushes.  Logits rather than greedy tokens, so a
    near-tie in a random model cannot decide the outcome."""
    from transformers import LlamaConfig, LlamaForCausalLM
    from intel_kivi_hybrid_amd.cache.manager import KiviCache
    torch.manual_seed(4)
    cfg = LlamaConfig(vocab_size=512, hidden_size=64 * heads, intermediate_size=1024,
                      num_hidden_layers=2, num_attention_heads=heads,
                      num_key_value_heads=kv_heads, max_position_embeddings=512)
    model = LlamaForCausalLM(cfg).eval().to(hip_device)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, cfg.vocab_size, (1, 160), generator=g).to(hip_device)
    n_prompt, R = 40, 32
    print(f"[packed-ratio] heads={heads} kv_heads={kv_heads}", flush=True)
    packed = pc.KiviPackedCache.from_model(model, device="cuda:0", group_size=32,
                                           residual_length=R)
    served = KiviCache.from_model(model, device="cuda:0", group_size=32, residual_length=R)
    worst = 0.0
    with torch.no_grad():
        out = model(ids[:, :n_prompt], use_cache=True)
        served.add_tokens(out.past_key_values)
        with pc.packed_attention(model):
            model(ids[:, :n_prompt], past_key_values=packed, use_cache=True)
        for s in range(n_prompt, ids.shape[1]):
            ref = model(ids[:, s:s + 1], past_key_values=served.get_full_cache(),
                        use_cache=True)
            served.add_tokens(ref.past_key_values)
            with pc.packed_attention(model):
                ours = model(ids[:, s:s + 1], past_key_values=packed, use_cache=True)
            a, b = ours.logits[0, -1].float(), ref.logits[0, -1].float()
            worst = max(worst, ((a - b).abs().max() / b.abs().max()).item())
    print(f"[packed-ratio]   worst logits rel diff {worst:.3e} over "
          f"{ids.shape[1] - n_prompt} steps", flush=True)
    assert packed.get_stats(0)["total_tokens"] == ids.shape[1]
    assert worst <= 1e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gqa_llama_packed_vs_served(hip_device, dtype):
    """Grouped-query Llama (8 query heads over 2 kv heads, D=128), model on
    the GPU: packed vs served cache pick the same tokens in fp32.  In bf16
    (which the reference's fp32 served cache cannot feed) both paths run end
    to end -- the served cache takes the model's dtype -- and their
    agreement with the fp32 tokens is printed."""
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(3)
    cfg = LlamaConfig(vocab_size=1024, hidden_size=1024, intermediate_size=2048,
                      num_hidden_layers=4, num_attention_heads=8, num_key_value_heads=2,
                      max_position_embeddings=1024)
    model = LlamaForCausalLM(cfg).eval().to(hip_device)
    tok = _Tok(cfg.vocab_size)
    prompt = "grouped query attention over a packed cache"
    a = gen_mod.generate_packed(model, tok, prompt, max_new_tokens=120, group_size=32,
                                residual_length=64, device="cuda:0").split()
    if dtype == torch.float32:
        b = gen_mod.generate(model, tok, prompt, max_new_tokens=120, group_size=32,
                             residual_length=64, device="cuda:0").split()
        n, tot = _match(a, b)
        print(f"[packed-gqa] token match {n}/{tot}", flush=True)
        _assert_greedy_agrees(model, tok, prompt, a, b, R=64)
    else:
        model = model.to(dtype)
        c = gen_mod.generate_packed(model, tok, prompt, max_new_tokens=120, group_size=32,
                                    residual_length=64, device="cuda:0").split()
        d = gen_mod.generate(model, tok, prompt, max_new_tokens=120, group_size=32,
                             residual_length=64, device="cuda:0").split()
        n, tot = _match(a, c)
        n2, _ = _match(a, d)
        n3, _ = _match(c, d)
        print(f"[packed-gqa] bf16 packed vs fp32 {n}/{tot}, bf16 served vs fp32 {n2}/{tot}, "
              f"bf16 packed vs served {n3}/{tot}", flush=True)
        assert len(c) == len(a) == len(d)


def test_attention_output_matches_oracle(hip_device):
    """One decode step of the packed attention function against the float64
    oracle over the same store contents (1e-3 relative)."""
    from oracle.attention import decode_attention
    B, Hq, Hkv, D, G, R = 3, 8, 2, 128, 32, 64
    cache = pc.KiviPackedCache(1, D, Hkv, device="cuda:0", group_size=G, residual_length=R)
    g = torch.Generator().manual_seed(9)
    k = torch.randn(B, Hkv, 150, D, generator=g)
    v = torch.randn(B, Hkv, 150, D, generator=g)
    cache.update(k.cuda(), v.cuda(), 0)                      # prompt: 150 tokens
    k1, v1 = torch.randn(B, Hkv, 1, D, generator=g), torch.randn(B, Hkv, 1, D, generator=g)
    kt, _ = cache.update(k1.cuda(), v1.cuda(), 0)
    st = cache.store(0)
    n = st.n_chunks
    # dequantised history in token order, from the store's own codes
    kh, vh = [], []
    for c in range(n):
        kc = st.unpermuted_k_codes(c).cpu().numpy()                  # [B,H,G,D/4] token-major
        ks, kz = st.k_scale[:, :, c].cpu().numpy(), st.k_zero[:, :, c].cpu().numpy()
        codes = torch.from_numpy(kc)
        kd = torch.stack([(codes.to(torch.int32) >> (2 * j)) & 3 for j in range(4)], -1)
        kd = kd.reshape(B, Hkv, G, D).float()
        kh.append(kd * torch.from_numpy(ks)[:, :, None, :] + torch.from_numpy(kz)[:, :, None, :])
        vc = torch.from_numpy(st.unpermuted_v_codes(c).cpu().numpy())   # [B,H,D,G/4]
        vd = torch.stack([(vc.to(torch.int32) >> (2 * j)) & 3 for j in range(4)], -1)
        vd = vd.reshape(B, Hkv, D, G).transpose(2, 3).float()
        vs = st.chunk_v_scale(c).cpu()                                 # [B,H,G,D/Gv]
        vz = st.chunk_v_zero(c).cpu()
        vh.append(vd * vs.repeat_interleave(st.Gv, -1) + vz.repeat_interleave(st.Gv, -1))
    kr, vr = st.residual()
    q = torch.randn(B, Hq, 1, D, generator=g)

    class _M(torch.nn.Module):
        is_causal = True
    out, w = pc.kivi_packed_attention_forward(_M(), q.cuda(), kt, kt, None, scaling=D ** -0.5)
    ref = decode_attention(q[:, :, 0].numpy(), torch.cat(kh, 2).numpy(), torch.cat(vh, 2).numpy(),
                           kr.cpu().numpy(), vr.cpu().numpy())
    got = out[:, 0].cpu().double().numpy()
    err = abs(got - ref).max() / abs(ref).max()
    print(f"[packed-attn] chunks={n} res={kr.shape[2]} rel_err={err:.2e}", flush=True)
    assert w is None and out.shape == (B, 1, Hq, D)
    assert err <= 1e-3
    assert st.res_len == 150 - n * G + 1


def _ref_step(model, ref, ids):
    with torch.no_grad():
        out = model(ids, past_key_values=ref.get_full_cache(), use_cache=True)
    ref.add_tokens(out.past_key_values)
    return out.logits


def test_multitoken_steps_follow_reference_flow(hip_device):
    """Forwards of several tokens on a non-empty cache (chunked prefill) run
    the multi-token kernel causally over [history ; window ; new tokens]:
    logits agree with the reference flow's forward over get_full_cache()
    (fp32 SDPA over the oracle's served history) and the stores split the
    context the same way after each step's flushes.  Model on the CPU in both
    arms, attention of the packed arm on the GPU."""
    from transformers import GPT2Config, GPT2LMHeadModel
    torch.manual_seed(4)
    model = GPT2LMHeadModel(GPT2Config(n_layer=4, n_head=4, n_embd=256)).eval()
    G, R = 32, 64
    ours = pc.KiviPackedCache.from_model(model, device="cuda:0", group_size=G,
                                         residual_length=R)
    ref = _OracleShim.from_model(model, group_size=G, residual_length=R)
    gen = torch.Generator().manual_seed(5)
    ids = torch.randint(0, model.config.vocab_size, (2, 90), generator=gen)
    with torch.no_grad(), pc.packed_attention(model):
        model(ids, past_key_values=ours, use_cache=True)
    _ref_step(model, ref, ids)
    worst = 0.0
    for n in [5, 1, 3, 8, 1, 17, 2, 64, 1, 40, 7]:
        chunk = torch.randint(0, model.config.vocab_size, (2, n), generator=gen)
        print(f"[packed-multi] step of {n} tokens", flush=True)
        with torch.no_grad(), pc.packed_attention(model):
            lo = model(chunk, past_key_values=ours, use_cache=True).logits
        lr = _ref_step(model, ref, chunk)
        err = ((lo - lr).abs().max() / lr.abs().max()).item()
        worst = max(worst, err)
        assert err <= 1e-3, err
        assert torch.equal(lo.argmax(-1), lr.argmax(-1))
        for lay in ours.layers:
            lay.settle()
        st = ours.store(0)
        assert st.quantized_tokens == ref.get_stats(0)["quantized_tokens"]
        assert st.res_len == ref.get_stats(0)["residual_tokens"]
    print(f"[packed-multi] worst logits rel err {worst:.2e}", flush=True)
    assert ours.total_flushes == ref.total_flushes


def test_hf_assisted_generation(hip_device):
    """transformers' assisted generation drives the cache: verification
    passes of several tokens, then crop() of the rejected drafts.  Greedy
    output equals plain greedy generation with the same cache type, and both
    kinds of steps did occur."""
    from transformers import GPT2Config, GPT2LMHeadModel
    torch.manual_seed(6)
    model = GPT2LMHeadModel(GPT2Config(n_layer=4, n_head=4, n_embd=256)).eval().to(hip_device)
    torch.manual_seed(6)
    draft = GPT2LMHeadModel(GPT2Config(n_layer=1, n_head=4, n_embd=256)).eval().to(hip_device)
    draft.generation_config.num_assistant_tokens = 3
    draft.generation_config.num_assistant_tokens_schedule = "constant"
    draft.generation_config.assistant_confidence_threshold = 0.0
    ids = torch.randint(0, model.config.vocab_size, (1, 40),
                        generator=torch.Generator().manual_seed(7)).to(hip_device)
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
        cache = pc.KiviPackedCache.from_model(model, device="cuda:0", group_size=32,
                                              residual_length=32)
        kw = {} if assistant is None else {"assistant_model": assistant}
        pc.KiviPackedLayer.update, pc.KiviPackedLayer.crop = spy_update, spy_crop
        try:
            with pc.packed_attention(model):
                outs.append(model.generate(ids, past_key_values=cache, max_new_tokens=120,
                                           do_sample=False, attention_mask=torch.ones_like(ids),
                                           pad_token_id=0, **kw).cpu())
        finally:
            pc.KiviPackedLayer.update, pc.KiviPackedLayer.crop = update, crop
        assert cache.get_seq_length() == ids.shape[1] + 119
    n, tot = _match(outs[0][0].tolist(), outs[1][0].tolist())
    print(f"[packed-assisted] token match {n}/{tot}; steps {sizes[-12:]}, crops {crops[-12:]}",
          flush=True)
    assert max(sizes[1:]) > 2 and any(c < 0 for c in crops)
    assert torch.equal(outs[0], outs[1])


def test_left_padded_batch_follows_reference_flow(hip_device):
    """A left-padded batch of three prompts (50, 37 and 12 tokens) decoded
    with one-token and multi-token steps: the packed attention on the GPU
    hides each sequence's pad positions from HF's mask, and the logits agree
    with the reference flow's (HF SDPA with the same mask over
    get_full_cache()); the stores split the context the same way.  Model on
    the CPU in both arms."""
    from transformers import GPT2Config, GPT2LMHeadModel
    torch.manual_seed(21)
    model = GPT2LMHeadModel(GPT2Config(n_layer=3, n_head=4, n_embd=256)).eval()
    G, R = 32, 64
    ours = pc.KiviPackedCache.from_model(model, device="cuda:0", group_size=G,
                                         residual_length=R)
    ref = _OracleShim.from_model(model, group_size=G, residual_length=R)
    gen = torch.Generator().manual_seed(22)
    lengths = [50, 37, 12]
    T = max(lengths)
    ids = torch.zeros(3, T, dtype=torch.long)
    mask = torch.zeros(3, T, dtype=torch.long)
    for b, n in enumerate(lengths):
        ids[b, T - n:] = torch.randint(1, model.config.vocab_size, (n,), generator=gen)
        mask[b, T - n:] = 1

    def kw(n):
        return dict(attention_mask=mask, position_ids=(mask.cumsum(-1) - 1).clamp(min=0)[:, -n:],
                    use_cache=True)
    with torch.no_grad(), pc.packed_attention(model):
        model(ids, past_key_values=ours, **kw(T))
    _ref_step_kw = lambda x, n: model(x, past_key_values=ref.get_full_cache(), **kw(n))  # noqa: E731
    with torch.no_grad():
        ref.add_tokens(model(ids, **kw(T)).past_key_values)
    worst = 0.0
    for n in [1, 1, 3, 1, 9, 1, 1, 30, 1, 2] + [1] * 20:
        new = torch.randint(1, model.config.vocab_size, (3, n), generator=gen)
        mask = torch.cat([mask, torch.ones(3, n, dtype=torch.long)], dim=1)
        with torch.no_grad(), pc.packed_attention(model):
            lo = model(new, past_key_values=ours, **kw(n)).logits
        with torch.no_grad():
            out = _ref_step_kw(new, n)
        ref.add_tokens(out.past_key_values)
        err = ((lo - out.logits).abs().max() / out.logits.abs().max()).item()
        worst = max(worst, err)
        assert err <= 1e-3, (n, err)
        for lay in ours.layers:
            lay.settle()
        assert ours.store(0).quantized_tokens == ref.get_stats(0)["quantized_tokens"]
    print(f"[packed-padded] worst logits rel err {worst:.2e}", flush=True)
    assert ours.total_flushes == ref.total_flushes > 0


def test_hf_generate_left_padded_batch(hip_device):
    """transformers' generate() on a left-padded batch (prompts of 23 and 9
    tokens) with the packed cache on the GPU picks the tokens of a greedy loop
    over the reference flow with the same masks and positions (model on the
    CPU in both arms)."""
    from transformers import GPT2Config, GPT2LMHeadModel
    torch.manual_seed(31)
    model = GPT2LMHeadModel(GPT2Config(n_layer=4, n_head=4, n_embd=256)).eval()
    G, R = 32, 32
    gen = torch.Generator().manual_seed(32)
    lengths, T = [23, 9], 23
    ids = torch.zeros(2, T, dtype=torch.long)
    mask = torch.zeros(2, T, dtype=torch.long)
    for b, n in enumerate(lengths):
        ids[b, T - n:] = torch.randint(1, model.config.vocab_size, (n,), generator=gen)
        mask[b, T - n:] = 1
    new_tokens = 60
    cache = pc.KiviPackedCache.from_model(model, device="cuda:0", group_size=G,
                                          residual_length=R)
    with pc.packed_attention(model):
        hf = model.generate(ids, attention_mask=mask, past_key_values=cache,
                            max_new_tokens=new_tokens, do_sample=False, pad_token_id=0)
    ref = _OracleShim.from_model(model, group_size=G, residual_length=R)

    def kw(m, n):
        return dict(attention_mask=m, position_ids=(m.cumsum(-1) - 1).clamp(min=0)[:, -n:],
                    use_cache=True)
    with torch.no_grad():
        out = model(ids, **kw(mask, T))
    ref.add_tokens(out.past_key_values)
    toks = [out.logits[:, -1:].argmax(-1)]
    for _ in range(new_tokens - 1):
        mask = torch.cat([mask, torch.ones(2, 1, dtype=torch.long)], dim=1)
        with torch.no_grad():
            out = model(toks[-1], past_key_values=ref.get_full_cache(), **kw(mask, 1))
        ref.add_tokens(out.past_key_values)
        toks.append(out.logits[:, -1:].argmax(-1))
    ours = hf[:, T:]
    want = torch.cat(toks, dim=1)
    n, tot = _match(ours.reshape(-1).tolist(), want.reshape(-1).tolist())
    print(f"[packed-padded-generate] token match {n}/{tot}", flush=True)
    assert torch.equal(ours, want)


@pytest.mark.parametrize("kind", ["right", "holes"])
def test_padded_batch_any_pattern_follows_reference_flow(hip_device, kind):
    """A right-padded batch (pad positions between each prompt and its new
    tokens) or one with holes inside the prompts, decoded with one-token and
    multi-token steps: the packed attention applies HF's mask through
    hidden-position bits, and the logits agree with the reference flow's (HF
    SDPA with the same mask over get_full_cache()).  Model on the CPU in both
    arms."""
    from transformers import GPT2Config, GPT2LMHeadModel
    torch.manual_seed(41)
    model = GPT2LMHeadModel(GPT2Config(n_layer=3, n_head=4, n_embd=256)).eval()
    G, R = 32, 64
    ours = pc.KiviPackedCache.from_model(model, device="cuda:0", group_size=G,
                                         residual_length=R)
    ref = _OracleShim.from_model(model, group_size=G, residual_length=R)
    gen = torch.Generator().manual_seed(42)
    lengths = [50, 37, 12]
    T = max(lengths)
    ids = torch.randint(1, model.config.vocab_size, (3, T), generator=gen)
    mask = torch.zeros(3, T, dtype=torch.long)
    for b, n in enumerate(lengths):
        mask[b, :n] = 1
        if kind == "holes":
            mask[b, :n - 1] = (torch.rand(n - 1, generator=gen) > 0.3).long()
    ids = ids * mask

    def kw(n):
        return dict(attention_mask=mask, position_ids=(mask.cumsum(-1) - 1).clamp(min=0)[:, -n:],
                    use_cache=True)
    with torch.no_grad(), pc.packed_attention(model):
        model(ids, past_key_values=ours, **kw(T))
    with torch.no_grad():
        ref.add_tokens(model(ids, **kw(T)).past_key_values)
    worst = 0.0
    for n in [1, 1, 3, 1, 9, 1, 1, 30, 1, 2] + [1] * 20:
        new = torch.randint(1, model.config.vocab_size, (3, n), generator=gen)
        mask = torch.cat([mask, torch.ones(3, n, dtype=torch.long)], dim=1)
        with torch.no_grad(), pc.packed_attention(model):
            lo = model(new, past_key_values=ours, **kw(n)).logits
        with torch.no_grad():
            out = model(new, past_key_values=ref.get_full_cache(), **kw(n))
        ref.add_tokens(out.past_key_values)
        err = ((lo - out.logits).abs().max() / out.logits.abs().max()).item()
        worst = max(worst, err)
        assert err <= 1e-3, (n, err)
        for lay in ours.layers:
            lay.settle()
    plan = ours._mask_memo[1]
    assert plan[0] is None and plan[1] is not None      # the hidden-bits path ran
    print(f"[packed-{kind}] worst logits rel err {worst:.2e}", flush=True)
    assert ours.total_flushes == ref.total_flushes > 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@torch.no_grad()
def test_half_precision_logits_match_served_cache(hip_device, dtype):
    """A half-precision Llama (GQA 4:1, head_dim 128) decodes the same
    seeded tokens over a 1K-token prompt with the packed cache (2-bit store,
    16-bit residual ring, the fused kernel) and with KiviCache driven as the
    reference's generate() drives it (the same quantisation, served to SDPA
    as a dequantised cache of the model's dtype): the final logits agree to
    within the served cache's 16-bit rounding (cosine >= 0.999, max
    difference <= 5 % of the largest logit)."""
    from transformers import LlamaConfig, LlamaForCausalLM
    from intel_kivi_hybrid_amd import KiviCache, KiviPackedCache
    torch.manual_seed(4)
    cfg = LlamaConfig(vocab_size=2048, hidden_size=1024, intermediate_size=2048,
                      num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2,
                      max_position_embeddings=2048)
    model = LlamaForCausalLM(cfg).eval().to(hip_device, dtype)
    B, T, steps, G, R = 2, 1000, 40, 32, 64
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(5))
    dec = torch.randint(0, cfg.vocab_size, (B, steps), generator=torch.Generator().manual_seed(6))
    ids, dec = ids.to(hip_device), dec.to(hip_device)
    pos = torch.arange(T + steps, device=hip_device)

    packed = KiviPackedCache.from_model(model, device="cuda:0", group_size=G, residual_length=R)
    with pc.packed_attention(model):
        model(ids, past_key_values=packed, use_cache=True, cache_position=pos[:T])
        for i in range(steps):
            a = model(dec[:, i:i + 1], past_key_values=packed, use_cache=True,
                      cache_position=pos[T + i:T + i + 1]).logits[:, -1].float()

    served = KiviCache.from_model(model, device="cuda:0", group_size=G, residual_length=R)
    out = model(ids, use_cache=True, cache_position=pos[:T])
    served.add_tokens(out.past_key_values)
    for i in range(steps):
        out = model(dec[:, i:i + 1], past_key_values=served.get_full_cache(), use_cache=True,
                    cache_position=pos[T + i:T + i + 1])
        served.add_tokens(out.past_key_values)
    b = out.logits[:, -1].float()
    assert packed.total_flushes == served.total_flushes > 0
    cos = torch.nn.functional.cosine_similarity(a, b, dim=-1).min().item()
    rel = ((a - b).abs().max() / b.abs().max()).item()
    print(f"[packed-half] {dtype}: cosine {cos:.6f}, max diff {rel:.3e} of the largest logit",
          flush=True)
    assert cos >= 0.999 and rel <= 5e-2
