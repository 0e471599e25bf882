"""Test infrastructure only: CPU restatement of the reference ``KiviCache``.

Follows src/kivi_sycl/cache/manager.py line by line (cited per method), with
the device round-trip (``quant_dequant_roundtrip_keys/values``,
manager.py:337-345) replaced by the C oracle codec.  It is the checker for the
HBM-resident ``intel_kivi_hybrid_amd.KiviCache``: served K/V, flush counts
and ``get_stats`` must match it exactly.
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import numpy as np
import torch
from transformers.cache_utils import DynamicCache

from . import codec


def iter_kv_layers(past_key_values):
    """manager.py:14-33."""
    if hasattr(past_key_values, "layers"):
        for layer in past_key_values.layers:
            yield layer.keys, layer.values
        return
    if hasattr(past_key_values, "key_cache") and hasattr(past_key_values, "value_cache"):
        for k, v in zip(past_key_values.key_cache, past_key_values.value_cache):
            yield k, v
        return
    for item in past_key_values:
        yield item[0], item[1]


def build_cache(layers):
    """manager.py:36-49."""
    cache = DynamicCache()
    for i, (k, v) in enumerate(layers):
        cache.update(k, v, i)
    return cache


def roundtrip(t: torch.Tensor, group_size: int) -> torch.Tensor:
    """The fused round-trip over flat groups, on CPU (roundtrip_kernels.cpp)."""
    x = t.detach().to("cpu", torch.float32).contiguous()
    out = codec.roundtrip_groups(x.numpy(), group_size)
    return torch.from_numpy(out.reshape(tuple(x.shape)))


class KiviCacheOracle:
    """manager.py:52-423, state kept on the CPU as the reference keeps it."""

    def __init__(self, num_layers, head_dim, num_kv_heads=None, group_size=32,
                 residual_length=128, roundtrip_fn=None):
        """``roundtrip_fn(t, group_size)`` replaces the device round-trip
        (default: the C oracle codec); the reference's unit tests also run
        with an identity round-trip (tests/unit/test_manager_bookkeeping.py:56-69)."""
        self._roundtrip = roundtrip if roundtrip_fn is None else roundtrip_fn
        # manager.py:82-90
        assert head_dim % group_size == 0
        assert group_size >= 4 and group_size % 4 == 0
        assert group_size <= residual_length
        self.G = group_size
        self.R = residual_length
        self.head_dim = head_dim
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.batch_size: Optional[int] = None
        self._quant_token_count: List[int] = [0] * num_layers
        self._quant_bytes: List[int] = [0] * num_layers
        self.res_keys: List[Optional[torch.Tensor]] = [None] * num_layers
        self.res_values: List[Optional[torch.Tensor]] = [None] * num_layers
        self._deq_history: List[Optional[Tuple[torch.Tensor, torch.Tensor]]] = [None] * num_layers
        self._flush_count: List[int] = [0] * num_layers
        self._cache_view = None
        self._cache_view_valid = False

    def add_tokens(self, past_key_values):
        """manager.py:162-249."""
        if past_key_values is not self._cache_view:
            self._cache_view_valid = False
        for i, (k, v) in enumerate(iter_kv_layers(past_key_values)):
            k = k.detach().to("cpu")
            v = v.detach().to("cpu")
            if self.batch_size is None:
                self.batch_size = k.shape[0]
                self.num_kv_heads = k.shape[1]
            else:
                assert k.shape[0] == self.batch_size, "batch size changed"
            if self.res_keys[i] is not None:
                new_start = self._quant_token_count[i] + self.res_keys[i].shape[2]
                assert k.shape[2] >= new_start, "desync"
                new_k = k[:, :, new_start:, :].float()
                new_v = v[:, :, new_start:, :].float()
            else:
                new_k = k.float()
                new_v = v.float()
            assert new_k.shape[2] > 0, "desync"
            if self.res_keys[i] is None:
                self.res_keys[i] = new_k
                self.res_values[i] = new_v
            else:
                self.res_keys[i] = torch.cat([self.res_keys[i], new_k], dim=2)
                self.res_values[i] = torch.cat([self.res_values[i], new_v], dim=2)
            while self.res_keys[i].shape[2] >= self.R:       # manager.py:242
                self._flush_group(i)
                self._cache_view_valid = False

    def get_full_cache(self):
        """manager.py:251-290."""
        if self._cache_view is not None and self._cache_view_valid:
            return self._cache_view
        full = []
        for i in range(self.num_layers):
            pk, pv = [], []
            if self._deq_history[i] is not None:
                pk.append(self._deq_history[i][0])
                pv.append(self._deq_history[i][1])
            if self.res_keys[i] is not None and self.res_keys[i].shape[2] > 0:
                pk.append(self.res_keys[i])
                pv.append(self.res_values[i])
            fk = pk[0] if len(pk) == 1 else (torch.cat(pk, dim=2) if pk else torch.empty(0))
            fv = pv[0] if len(pv) == 1 else (torch.cat(pv, dim=2) if pv else torch.empty(0))
            full.append((fk, fv))
        self._cache_view = build_cache(full)
        self._cache_view_valid = True
        return self._cache_view

    def served(self, layer: int):
        """[history || residual] for one layer, as get_full_cache builds it."""
        pk, pv = [], []
        if self._deq_history[layer] is not None:
            pk.append(self._deq_history[layer][0])
            pv.append(self._deq_history[layer][1])
        if self.res_keys[layer] is not None and self.res_keys[layer].shape[2] > 0:
            pk.append(self.res_keys[layer])
            pv.append(self.res_values[layer])
        return torch.cat(pk, dim=2), torch.cat(pv, dim=2)

    def reset(self):
        """manager.py:292-303."""
        heads = self.num_kv_heads      # reset() keeps it (manager.py:292-303)
        self.__init__(self.num_layers, self.head_dim, heads, self.G, self.R, self._roundtrip)

    def _flush_group(self, i: int):
        """manager.py:309-374."""
        G = self.G
        assert self.res_keys[i].shape[2] >= G
        k_trans = self.res_keys[i][:, :, :G, :].transpose(2, 3).contiguous()  # [B,H,D,G]
        batch, heads, dim, seq = k_trans.shape
        deq_k = self._roundtrip(k_trans, G)
        v_chunk = self.res_values[i][:, :, :G, :].contiguous()                 # [B,H,G,D]
        deq_v = self._roundtrip(v_chunk, G)
        groups_per_token = self.head_dim // G
        self._quant_token_count[i] += G
        self._quant_bytes[i] += (
            batch * heads * dim * (seq // 4)
            + batch * heads * dim * 4 * 2
            + batch * heads * G * (self.head_dim // 4)
            + batch * heads * G * groups_per_token * 4 * 2
        )
        self.res_keys[i] = self.res_keys[i][:, :, G:, :].contiguous()
        self.res_values[i] = self.res_values[i][:, :, G:, :].contiguous()
        new_k = deq_k.transpose(2, 3)
        new_v = deq_v
        cur = self._deq_history[i]
        if cur is not None:
            hist = (torch.cat([cur[0], new_k], dim=2), torch.cat([cur[1], new_v], dim=2))
        else:
            hist = (new_k.contiguous(), new_v)
        self._flush_count[i] += 1
        self._deq_history[i] = hist

    @property
    def total_flushes(self) -> int:
        return sum(self._flush_count)

    def get_stats(self, layer: int = 0) -> dict:
        """manager.py:384-419."""
        B = self.batch_size or 1
        H = self.num_kv_heads or 1
        quant_tokens = self._quant_token_count[layer]
        res_tokens = self.res_keys[layer].shape[2] if self.res_keys[layer] is not None else 0
        total = quant_tokens + res_tokens
        quant_bytes = self._quant_bytes[layer]
        res_bytes = 0
        if self.res_keys[layer] is not None:
            res_bytes = (self.res_keys[layer].numel() + self.res_values[layer].numel()) * 4
        fp32_bytes = 2 * B * H * total * self.head_dim * 4
        return {
            "total_tokens": total,
            "quantized_tokens": quant_tokens,
            "residual_tokens": res_tokens,
            "kivi_bytes": quant_bytes + res_bytes,
            "fp32_bytes": fp32_bytes,
            "compression": fp32_bytes / (quant_bytes + res_bytes)
            if (quant_bytes + res_bytes) > 0 else 0,
        }


def closed_form_stats(B, H, D, G, R, total_tokens):
    """get_stats in closed form for a run that fed `total_tokens` one or more at
    a time: flushes happen while residual >= R (manager.py:242), each flush
    quantises G tokens (manager.py:350-356)."""
    n_flush = 0 if total_tokens < R else (total_tokens - R) // G + 1
    quant = n_flush * G
    res = total_tokens - quant
    per_flush = B * H * D * (G // 4) + B * H * D * 8 + B * H * G * (D // 4) + B * H * G * (D // G) * 8
    kivi = n_flush * per_flush + 2 * B * H * res * D * 4
    fp32 = 2 * B * H * total_tokens * D * 4
    return {"total_tokens": total_tokens, "quantized_tokens": quant,
            "residual_tokens": res, "kivi_bytes": kivi, "fp32_bytes": fp32,
            "compression": fp32 / kivi if kivi else 0}


__all__ = ["KiviCacheOracle", "iter_kv_layers", "build_cache", "roundtrip",
           "closed_form_stats", "np"]
