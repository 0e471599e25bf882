"""A stand-in for a HuggingFace causal LM's KV-cache contract, for cache
state-machine tests (the reference's tests use the same two behaviours,
tests/unit/test_manager_bookkeeping.py:83-144):

* ``in_place``: appends the new K/V to the ``DynamicCache`` it is given and
  returns that same object (what current transformers models do);
* ``legacy_tuple``: returns a new tuple of full-length (k, v) per layer and
  leaves the passed cache untouched (pre-Cache-API models).

Token t of every layer carries the value t plus a small seeded jitter, so a
dropped, duplicated or reordered token changes the served tensors.  The model
also checks that it was served exactly the tokens it has produced.
"""

import torch
from transformers.cache_utils import DynamicCache


def iter_layers(past):
    if hasattr(past, "layers"):
        return [(layer.keys, layer.values) for layer in past.layers]
    return [(k, v) for k, v in past]


class FakeModel:
    def __init__(self, num_layers, num_heads, head_dim, mode, batch=1, seed=0,
                 device="cpu", jitter=0.01):
        assert mode in ("in_place", "legacy_tuple")
        self.num_layers, self.num_heads, self.head_dim = num_layers, num_heads, head_dim
        self.mode, self.batch, self.device, self.jitter = mode, batch, device, jitter
        self.gen = torch.Generator().manual_seed(seed)
        self.total_tokens = 0
        self.truth_k = [None] * num_layers
        self.truth_v = [None] * num_layers

    def _new_kv(self, n):
        base = torch.arange(self.total_tokens, self.total_tokens + n, dtype=torch.float32)
        base = base.view(1, 1, n, 1).expand(self.batch, self.num_heads, n, self.head_dim)
        noise = torch.randn(self.batch, self.num_heads, n, self.head_dim,
                            generator=self.gen) * self.jitter
        return (base + noise).contiguous(), (base - noise).contiguous()

    def forward(self, n_new, past=None):
        new = [self._new_kv(n_new) for _ in range(self.num_layers)]
        for i, (k, v) in enumerate(new):
            self.truth_k[i] = k if self.truth_k[i] is None else torch.cat([self.truth_k[i], k], 2)
            self.truth_v[i] = v if self.truth_v[i] is None else torch.cat([self.truth_v[i], v], 2)
        past_layers = None
        if past is not None:
            past_layers = iter_layers(past)
            for i, (pk, _) in enumerate(past_layers):
                assert pk.shape[2] == self.total_tokens, (
                    f"model was served {pk.shape[2]} past tokens at layer {i}, "
                    f"expected {self.total_tokens}")
        self.total_tokens += n_new
        new = [(k.to(self.device), v.to(self.device)) for k, v in new]
        if self.mode == "in_place":
            cache = past if isinstance(past, DynamicCache) else DynamicCache()
            for i, (k, v) in enumerate(new):
                cache.update(k, v, i)
            return cache
        out = []
        for i, (k, v) in enumerate(new):
            if past_layers is not None:
                pk, pv = past_layers[i]
                k = torch.cat([pk.to(self.device), k], dim=2)
                v = torch.cat([pv.to(self.device), v], dim=2)
            out.append((k, v))
        return tuple(out)


def run_generation(cache, model, steps, prefill, check=None):
    """Prefill, then ``steps`` single-token decode steps through ``cache``,
    exactly as KiviCache's users drive it.  ``check(step, cache, past)`` runs
    before each decode step on the served cache."""
    cache.add_tokens(model.forward(prefill))
    for step in range(steps):
        past = cache.get_full_cache()
        served = iter_layers(past)[0][0].shape[2]
        assert served == model.total_tokens, (
            f"stale cache served: {served} tokens, model has produced {model.total_tokens}")
        if check is not None:
            check(step, cache, past)
        cache.add_tokens(model.forward(1, past))
    return cache
