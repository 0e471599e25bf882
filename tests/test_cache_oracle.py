"""CPU tests: pin the KiviCache oracle (oracle/kivi_cache.py) to the
reference's own cache scenarios (tests/unit/test_manager_bookkeeping.py:147-209)
and to the README's published accounting (README.md:17-18).

The oracle is then the checker for the HBM-resident KiviCache on the GPU.
"""

import numpy as np
import pytest
import torch

from oracle import codec
from oracle.kivi_cache import KiviCacheOracle, closed_form_stats, iter_kv_layers
from tests.conftest import seeded_kv
from tests.fake_model import FakeModel, run_generation


def _identity(t, group_size):
    return t.detach().to("cpu", torch.float32).clone()


def _mirror(t, group_size):
    return codec.mirror_roundtrip(t.detach().to("cpu", torch.float32).contiguous(), group_size)


GEOM = dict(G=4, R=8, D=8, layers=2, heads=2, prefill=6, steps=24)   # the reference's


def _run(mode, roundtrip_fn=None, **kw):
    g = dict(GEOM, **kw)
    cache = KiviCacheOracle(g["layers"], g["D"], g["heads"], g["G"], g["R"],
                            roundtrip_fn=roundtrip_fn)
    model = FakeModel(g["layers"], g["heads"], g["D"], mode, seed=3)
    run_generation(cache, model, g["steps"], g["prefill"])
    return cache, model


@pytest.mark.parametrize("mode", ["in_place", "legacy_tuple"])
def test_identity_roundtrip_serves_ground_truth(mode):
    cache, model = _run(mode, _identity)
    for i, (k, v) in enumerate(iter_kv_layers(cache.get_full_cache())):
        assert torch.equal(k, model.truth_k[i]) and torch.equal(v, model.truth_v[i])
        assert k.shape[2] == model.total_tokens


@pytest.mark.parametrize("mode", ["in_place", "legacy_tuple"])
@pytest.mark.parametrize("use_mirror", [False, True])
def test_flushed_chunks_match_per_chunk_roundtrip(mode, use_mirror):
    G = GEOM["G"]
    cache, model = _run(mode, _mirror if use_mirror else None)
    for i, (k, v) in enumerate(iter_kv_layers(cache.get_full_cache())):
        n_hist = cache._quant_token_count[i]
        assert n_hist > 0
        assert torch.equal(k[:, :, n_hist:], model.truth_k[i][:, :, n_hist:])
        assert torch.equal(v[:, :, n_hist:], model.truth_v[i][:, :, n_hist:])
        for c0 in range(0, n_hist, G):
            kt = model.truth_k[i][:, :, c0:c0 + G].transpose(2, 3).contiguous()
            vt = model.truth_v[i][:, :, c0:c0 + G].contiguous()
            assert codec.count_ties(kt.numpy(), G) == 0 and codec.count_ties(vt.numpy(), G) == 0
            # the reference's torch mirror and the C codec agree on tie-free chunks
            exp_k = _mirror(kt, G).transpose(2, 3)
            exp_v = _mirror(vt, G)
            assert torch.equal(k[:, :, c0:c0 + G], exp_k), f"layer {i} key chunk {c0}"
            assert torch.equal(v[:, :, c0:c0 + G], exp_v), f"layer {i} value chunk {c0}"


def test_double_add_tokens_raises_desync():
    cache = KiviCacheOracle(1, 8, 2, 4, 8)
    model = FakeModel(1, 2, 8, "in_place")
    out = model.forward(5)
    cache.add_tokens(out)
    with pytest.raises(AssertionError, match="desync"):
        cache.add_tokens(out)


def test_batch_change_raises():
    cache = KiviCacheOracle(1, 8, 2, 4, 8)
    cache.add_tokens(FakeModel(1, 2, 8, "in_place", batch=1).forward(3))
    with pytest.raises(AssertionError, match="batch size changed"):
        cache.add_tokens(FakeModel(1, 2, 8, "in_place", batch=2).forward(4))


def _feed_seeded(cache, layers, B, H, D, steps, seed, prefill=0):
    """Config-1 style feeding: seeded N(0,1) K/V with outliers, one token per
    step, through a legacy-tuple model contract (full history each step)."""
    k_all = seeded_kv((B, H, prefill + steps, D), seed=seed, kind="key")
    v_all = seeded_kv((B, H, prefill + steps, D), seed=seed + 1, kind="value")
    first = prefill if prefill else 1
    cache.add_tokens(tuple((k_all[:, :, :first], v_all[:, :, :first]) for _ in range(layers)))
    for t in range(first, prefill + steps):
        cache.add_tokens(tuple((k_all[:, :, :t + 1], v_all[:, :, :t + 1]) for _ in range(layers)))
    return k_all, v_all


def test_readme_accounting_replayed():
    """README.md:17-18 (examples/benchmark.py:74-118): GPT-2, G=32, R=64,
    32-token prompt + 199 fed tokens -> layer 0: 378 KB vs 1386 KB, 3.67x."""
    cache = KiviCacheOracle(1, 64, 12, 32, 64)
    _feed_seeded(cache, 1, 1, 12, 64, 199, seed=5, prefill=32)
    s = cache.get_stats(0)
    assert s["quantized_tokens"] == 192 and s["residual_tokens"] == 39
    assert s["kivi_bytes"] == 387072 and s["fp32_bytes"] == 1419264
    assert round(s["kivi_bytes"] / 1024, 1) == 378.0 and round(s["fp32_bytes"] / 1024, 1) == 1386.0
    assert round(s["compression"], 2) == 3.67
    assert s == closed_form_stats(1, 12, 64, 32, 64, 231)


def test_config1_accounting_and_history():
    """Benchmark config 1: 12 layers, B=1, H=12, D=64, R=G=32, 200 steps."""
    layers, B, H, D, G = 12, 1, 12, 64, 32
    cache = KiviCacheOracle(layers, D, None, G, G)
    k_all, v_all = _feed_seeded(cache, layers, B, H, D, 200, seed=1235)
    for layer in (0, 11):
        s = cache.get_stats(layer)
        assert s["quantized_tokens"] == 192 and s["residual_tokens"] == 8
        assert s["kivi_bytes"] == 196608 and s["fp32_bytes"] == 1228800
        assert s["compression"] == pytest.approx(6.25)
    assert cache.total_flushes == 6 * layers
    k, v = cache.served(0)
    kt = k_all[:, :, :192].reshape(B, H, 6, G, D).transpose(3, 4).contiguous()
    exp_k = codec.roundtrip_groups(kt.numpy(), G).reshape(B, H, 6, D, G)
    assert np.array_equal(k[:, :, :192].numpy(),
                          exp_k.transpose(0, 1, 2, 4, 3).reshape(B, H, 192, D))
    exp_v = codec.roundtrip_groups(v_all[:, :, :192].contiguous().numpy(), G)
    assert np.array_equal(v[:, :, :192].numpy().reshape(-1), exp_v)
    assert torch.equal(k[:, :, 192:], k_all[:, :, 192:])
