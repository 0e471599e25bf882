"""CPU tests of the host-side API: KiviCache construction rules and
assertion messages (src/kivi_sycl/cache/manager.py:82-90), model-config
detection (src/kivi_sycl/config/model_config.py:6-59), token sampling
(src/kivi_sycl/generation/sampling.py:10-25) and the public signatures.
Nothing here launches device work."""

import inspect
from types import SimpleNamespace

import pytest
import torch
from transformers import GPT2Config, LlamaConfig, MistralConfig

from intel_kivi_hybrid_amd import KiviCache, generate
from intel_kivi_hybrid_amd.cache.manager import _iter_kv_layers, flush_bytes
from intel_kivi_hybrid_amd.config import detect_model_config
from intel_kivi_hybrid_amd.generation import sample_token


def test_constructor_rules():
    with pytest.raises(AssertionError, match=r"head_dim \(60\) must be divisible by group_size \(32\)"):
        KiviCache(2, 60, group_size=32)
    with pytest.raises(AssertionError, match=r"group_size \(6\) must be >= 4 and divisible by 4"):
        KiviCache(2, 12, group_size=6)
    with pytest.raises(AssertionError, match=r"must not exceed residual_length"):
        KiviCache(2, 64, group_size=64, residual_length=32)
    c = KiviCache(12, 64, num_kv_heads=12, group_size=32, residual_length=64)
    assert repr(c) == "KiviCache(layers=12, head_dim=64, G=32, R=64, device='cuda')"
    assert c.total_flushes == 0
    assert c.get_stats(0) == {"total_tokens": 0, "quantized_tokens": 0, "residual_tokens": 0,
                              "kivi_bytes": 0, "fp32_bytes": 0, "compression": 0}


def test_device_rules():
    assert KiviCache(1, 8, group_size=4, residual_length=8, device="xpu").device == torch.device("cuda")
    assert KiviCache(1, 8, group_size=4, residual_length=8, device="xpu:1").device == torch.device("cuda:1")
    with pytest.raises(ValueError, match="HIP device"):
        KiviCache(1, 8, group_size=4, residual_length=8, device="cpu")
    # the reference's own unit tests build a CPU cache behind a stubbed _C
    # (tests/unit/test_manager_bookkeeping.py:72-80); the error names that use
    with pytest.raises(ValueError, match="stubbed _C"):
        KiviCache(1, 8, group_size=4, residual_length=8, device="cpu")


def test_signatures_match_reference():
    params = lambda f: list(inspect.signature(f).parameters)       # noqa: E731
    assert params(KiviCache.__init__) == ["self", "num_layers", "head_dim", "num_kv_heads",
                                          "device", "group_size", "residual_length"]
    assert params(KiviCache.from_model) == ["model", "device", "group_size", "residual_length"]
    assert params(generate) == ["model", "tokenizer", "prompt", "max_new_tokens", "group_size",
                                "residual_length", "device", "temperature", "top_k",
                                "do_sample", "verbose"]
    d = inspect.signature(generate).parameters
    assert (d["max_new_tokens"].default, d["group_size"].default,
            d["residual_length"].default) == (200, 32, 128)
    for name in ("add_tokens", "get_full_cache", "reset", "get_stats", "_flush_group"):
        assert callable(getattr(KiviCache, name))


@pytest.mark.parametrize("cfg,expect", [
    (GPT2Config(n_layer=12, n_head=12, n_embd=768), (12, 12, 64)),
    (LlamaConfig(num_hidden_layers=32, num_attention_heads=32, num_key_value_heads=8,
                 hidden_size=4096), (32, 8, 128)),
    (MistralConfig(num_hidden_layers=4, num_attention_heads=8, num_key_value_heads=2,
                   hidden_size=512, head_dim=96), (4, 2, 96)),
])
def test_detect_model_config(cfg, expect):
    got = detect_model_config(SimpleNamespace(config=cfg))
    assert (got["num_layers"], got["num_kv_heads"], got["head_dim"]) == expect
    c = KiviCache.from_model(SimpleNamespace(config=cfg), group_size=32, residual_length=64)
    assert (c.num_layers, c.num_kv_heads, c.head_dim) == expect


def test_detect_model_config_errors():
    with pytest.raises(ValueError, match="Cannot detect num_layers"):
        detect_model_config(SimpleNamespace(config=SimpleNamespace(n_head=2)))
    with pytest.raises(ValueError, match="Cannot detect num_heads"):
        detect_model_config(SimpleNamespace(config=SimpleNamespace(n_layer=2)))
    with pytest.raises(ValueError, match="Cannot detect head_dim"):
        detect_model_config(SimpleNamespace(config=SimpleNamespace(n_layer=2, num_kv_heads=2)))
    # a None GQA field falls through to the query-head count
    got = detect_model_config(SimpleNamespace(config=SimpleNamespace(
        num_layers=3, num_key_value_heads=None, num_attention_heads=4, hidden_size=64)))
    assert got == {"num_layers": 3, "num_kv_heads": 4, "head_dim": 16}


def test_sample_token():
    logits = torch.tensor([[0.1, 3.0, -1.0, 2.9], [5.0, 0.0, 0.0, 0.0]])
    assert sample_token(logits, 1.0, None, False).tolist() == [[1], [0]]
    torch.manual_seed(0)
    for _ in range(50):
        ids = sample_token(logits.clone(), 0.7, 2, True)
        assert ids.shape == (2, 1)
        assert ids[0, 0].item() in (1, 3) and ids[1, 0].item() in (0, 1, 2, 3)
    # sampling does not modify the caller's logits
    before = logits.clone()
    sample_token(logits, 0.5, 1, True)
    assert torch.equal(before, logits)
    # top_k=1 is greedy
    assert sample_token(logits, 0.3, 1, True)[:, 0].tolist() == [1, 0]


def test_iter_kv_layers_surfaces():
    from transformers.cache_utils import DynamicCache
    k = torch.zeros(1, 2, 3, 4)
    v = torch.ones(1, 2, 3, 4)
    dc = DynamicCache()
    dc.update(k, v, 0)
    legacy = SimpleNamespace(key_cache=[k], value_cache=[v])
    for surface in (dc, legacy, ((k, v),)):
        (kk, vv), = list(_iter_kv_layers(surface))
        assert torch.equal(kk, k) and torch.equal(vv, v)


def test_flush_bytes_formula():
    # manager.py:350-356 at the GPT-2 geometry: 24,576 B per flush per layer
    assert flush_bytes(1, 12, 64, 32) == 24576
