"""KiviCache: the KIVI 2-bit asymmetric KV-cache state manager, HBM-resident.

Drop-in for the reference's ``KiviCache`` (src/kivi_sycl/cache/manager.py:52-423):
same constructor, ``from_model``, ``add_tokens``, ``get_full_cache``,
``reset``, ``get_stats``, ``total_flushes`` and assertion messages, and the
same served K/V bit for bit.  What changes is where the state lives.  The
reference keeps an fp32 residual and an fp32 dequantised history on the CPU
and ships one G-token chunk to the device per flush (transpose, copy in,
round-trip kernel, copy out, concatenate; manager.py:309-374).  Here each
layer owns a :class:`~intel_kivi_hybrid_amd.store.PackedKVStore` in HBM:

* an fp32 residual ring of exactly R tokens per (batch, kv-head);
* the packed 2-bit store (codes, scales, zeros per G-token chunk);
* the dequantised history that ``get_full_cache()`` serves, written by the
  flush kernel itself (bit-identical to the reference's round-trip ops).

All the flushes one add_tokens() owes for a layer are one kernel launch over
every (batch, kv-head) pair, reading the residual ring and the new K/V in
place (fp32, bf16 or fp16, any strides); no host copy is involved and only
the tokens left over are copied into the ring.  New tokens are moved to the
device once (a no-op when the model already runs on it); served tensors are
placed on the device the model's K/V came from.
"""

from typing import List, Optional

import torch
from transformers.cache_utils import DynamicCache

from ..config.model_config import detect_model_config
from ..extension.loader import kivi_native  # noqa: F401  (fails loudly without the HIP library)
from ..store import PackedKVStore, append_layers

__all__ = ["KiviCache"]


def _iter_kv_layers(past_key_values):
    """Per-layer (key, value) from any HF cache surface: ``.layers`` (current
    transformers), ``key_cache``/``value_cache`` lists (older releases), or
    the legacy tuple of tuples (manager.py:14-33)."""
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


def _build_cache(layers):
    """Wrap per-layer (key, value) tensors in a ``DynamicCache`` through its
    ``update()`` API (manager.py:36-49)."""
    cache = DynamicCache()
    for i, (k, v) in enumerate(layers):
        cache.update(k, v, i)
    return cache


def _resolve_device(device) -> torch.device:
    """The store lives on a HIP device ("cuda" on ROCm torch).  The
    reference's "xpu" spelling is accepted as an alias for it.

    The reference also runs its cache with ``device="cpu"`` behind a stubbed
    ``_C`` (tests/unit/test_manager_bookkeeping.py:72-80,166-170), because its
    flush only crosses to the device for the round-trip op.  Here the whole
    state (residual ring, packed chunks, served history) is device memory
    written by the HIP kernels, so a CPU cache is refused; the CPU restatement
    of that bookkeeping is the test oracle (oracle/kivi_cache.py)."""
    name = str(device)
    if name.startswith("xpu"):
        name = "cuda" + name[3:]
    dev = torch.device(name)
    if dev.type != "cuda":
        raise ValueError(
            f"KiviCache keeps its packed store and residual window in GPU memory; "
            f"device must be a HIP device ('cuda' or 'cuda:N'), got {device!r}. "
            f"(The reference's CPU cache with a stubbed _C, as in its "
            f"test_manager_bookkeeping.py, has no counterpart here: every flush "
            f"and append runs a HIP kernel.)")
    return dev


def flush_bytes(batch: int, heads: int, head_dim: int, group_size: int) -> int:
    """Bytes one flush adds to the 2-bit store (manager.py:350-356): packed
    keys, per-channel key scales/zeros, packed values, per-group value
    scales/zeros."""
    B, H, D, G = batch, heads, head_dim, group_size
    return (B * H * D * (G // 4) + B * H * D * 4 * 2
            + B * H * G * (D // 4) + B * H * G * (D // G) * 4 * 2)


class KiviCache:
    """KIVI 2-bit asymmetric KV cache manager.

    Args:
        num_layers:       Number of transformer layers.
        head_dim:         Dimension per attention head.
        num_kv_heads:     Number of KV heads (optional, detected on first call).
        device:           HIP device holding the store ("cuda", "cuda:N").
        group_size:       Quantisation group size G; must divide head_dim, be
                          >= 4 and divisible by 4.
        residual_length:  Number of recent fp32 tokens kept (R).
    """

    def __init__(self, num_layers: int, head_dim: int, num_kv_heads: Optional[int] = None,
                 device: str = "cuda", group_size: int = 32, residual_length: int = 128):
        assert head_dim % group_size == 0, \
            f"head_dim ({head_dim}) must be divisible by group_size ({group_size})"
        assert group_size >= 4 and group_size % 4 == 0, \
            f"group_size ({group_size}) must be >= 4 and divisible by 4"
        assert group_size <= residual_length, (
            f"group_size ({group_size}) must not exceed residual_length "
            f"({residual_length}) — flushing requires a full group of tokens "
            f"to be available in the residual buffer, or tokens are silently dropped.")
        self.device = _resolve_device(device)
        self.G = group_size
        self.R = residual_length
        self.head_dim = head_dim
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.batch_size: Optional[int] = None

        self._quant_token_count: List[int] = [0] * num_layers
        self._quant_bytes: List[int] = [0] * num_layers
        self._flush_count: List[int] = [0] * num_layers
        self._fed: List[bool] = [False] * num_layers
        self._stores: List[Optional[PackedKVStore]] = [None] * num_layers
        self._serve_device: List[Optional[torch.device]] = [None] * num_layers
        # Served tensors take the dtype of the model's own K/V: fp32 for the
        # fp32 models the reference runs (identical to its .float() cache), and
        # bf16/fp16 for half-precision models, whose attention cannot take an
        # fp32 cache (the store itself is fp32 either way).
        self._serve_dtype: List[Optional[torch.dtype]] = [None] * num_layers

        # The DynamicCache handed out by get_full_cache(); valid while the
        # model grows that same object in place and no flush has happened.
        self._cache_view: Optional[DynamicCache] = None
        self._cache_view_valid: bool = False

    # ------------------------------------------------------------------ factory
    @classmethod
    def from_model(cls, model, device: str = "cuda", group_size: int = 32,
                   residual_length: int = 128) -> "KiviCache":
        """A KiviCache configured from a HuggingFace model (manager.py:135-156)."""
        cfg = detect_model_config(model)
        return cls(num_layers=cfg["num_layers"], head_dim=cfg["head_dim"],
                   num_kv_heads=cfg["num_kv_heads"], device=device, group_size=group_size,
                   residual_length=residual_length)

    # ----------------------------------------------------------------- core API
    def add_tokens(self, past_key_values):
        """Ingest the K/V of one forward pass (manager.py:162-249).

        ``past_key_values`` is whatever the model returned (a ``Cache`` or the
        legacy tuple); each tensor is ``[B, H, Seq, D]`` holding every token
        the model has seen.  The tokens beyond those already tracked are
        appended to the layer's residual window; while the window holds R or
        more tokens, its oldest G are flushed into the 2-bit store."""
        # The served view stays valid only if the model grew that exact object
        # in place; a different object (legacy tuples, rebuilt caches) means
        # the view no longer reflects what was generated.
        if past_key_values is not self._cache_view:
            self._cache_view_valid = False

        # Layers whose window takes this step's tokens without a flush are
        # appended together after the loop (one launch for all of them); the
        # others flush and append on their own, as before.
        appends = []
        try:
            for i, (k, v) in enumerate(_iter_kv_layers(past_key_values)):
                if self.batch_size is None:
                    self.batch_size = k.shape[0]
                    self.num_kv_heads = k.shape[1]
                else:
                    assert k.shape[0] == self.batch_size, (
                        f"KiviCache batch size changed mid-session "
                        f"({self.batch_size} -> {k.shape[0]}) at layer {i}. "
                        f"Call reset() before starting a new request/batch.")
                assert k.shape[-1] == self.head_dim, (
                    f"KiviCache was built for head_dim {self.head_dim} but layer {i} "
                    f"has key head_dim {k.shape[-1]}")

                new_start = 0
                if self._fed[i]:
                    new_start = self._quant_token_count[i] + self._stores[i].res_len
                    assert k.shape[2] >= new_start, (
                        f"KiviCache desync at layer {i}: expected past length "
                        f"{new_start} but got {k.shape[2]}. add_tokens() must be "
                        f"called exactly once per forward pass, seeded by "
                        f"get_full_cache().")
                    new_k = k[:, :, new_start:, :]
                    new_v = v[:, :, new_start:, :]
                else:
                    new_k, new_v = k, v

                assert new_k.shape[2] > 0, (
                    f"KiviCache desync at layer {i}: the forward pass produced "
                    f"no tokens beyond the {new_start} already tracked. "
                    f"add_tokens() was called twice on the same forward output, "
                    f"or the model was fed a past_key_values not obtained from "
                    f"get_full_cache(). Silently skipping here would drop this "
                    f"step's KV and corrupt all subsequent attention.")

                fed = self._fed[i]
                store = self._store_for(i, k.shape[0], k.shape[1], new_k.shape[2])
                self._serve_device[i] = k.device
                self._serve_dtype[i] = k.dtype if k.dtype in (torch.bfloat16, torch.float16) \
                    else torch.float32
                # fp32, bf16 and fp16 K/V are read as they are (widening to fp32
                # is exact, as the reference's .float() is, manager.py:210-214).
                if fed and store.res_len + new_k.shape[2] < self.R:
                    appends.append((store, new_k, new_v))
                    continue
                flushes = store.extend(new_k, new_v, flush_at=self.R)
                if flushes:
                    self._record_flushes(i, flushes)
                    self._cache_view_valid = False
        finally:
            # (layers before a failed check keep this step's tokens, as when
            # each layer appended on its own)
            if appends:
                append_layers(*zip(*appends))

    def get_full_cache(self) -> DynamicCache:
        """The cache to pass as ``past_key_values`` to the next forward pass
        (manager.py:251-290): per layer, the dequantised history followed by
        the fp32 residual window, on the model's device -- fp32 as in the
        reference, or the model's own bf16/fp16 dtype for half-precision
        models."""
        if self._cache_view is not None and self._cache_view_valid:
            return self._cache_view
        full = []
        for i in range(self.num_layers):
            if not self._fed[i]:
                full.append((torch.empty(0), torch.empty(0)))
                continue
            full.append(self._served(i))
        self._cache_view = _build_cache(full)
        self._cache_view_valid = True
        return self._cache_view

    def reset(self):
        """Clear all cached data so the cache can serve a new sequence
        (manager.py:292-303).  Device buffers are kept for reuse when the
        next sequence has the same batch and head counts."""
        for i in range(self.num_layers):
            self._quant_token_count[i] = 0
            self._quant_bytes[i] = 0
            self._flush_count[i] = 0
            self._fed[i] = False
            self._serve_device[i] = None
            self._serve_dtype[i] = None
            if self._stores[i] is not None:
                self._stores[i].reset()
        self.batch_size = None
        self._cache_view = None
        self._cache_view_valid = False

    # ---------------------------------------------------------------- internals
    def _store_for(self, i: int, batch: int, heads: int, incoming: int) -> PackedKVStore:
        st = self._stores[i]
        if self._fed[i]:
            return st
        if st is None or st.B != batch or st.H != heads:
            st = PackedKVStore(batch, heads, self.head_dim, self.G, self.R, self.device,
                               chunk_capacity=incoming // self.G + 4, keep_history=True)
            self._stores[i] = st
        self._fed[i] = True
        return st

    def _record_flushes(self, i: int, n: int) -> None:
        st = self._stores[i]
        self._quant_token_count[i] += n * self.G
        self._quant_bytes[i] += n * flush_bytes(st.B, st.H, self.head_dim, self.G)
        self._flush_count[i] += n

    def _flush_group(self, layer_idx: int):
        """Quantise the G oldest residual tokens of one layer into its 2-bit
        store (manager.py:309-374), on the device."""
        i = layer_idx
        st = self._stores[i]
        res = st.res_len if (st is not None and self._fed[i]) else 0
        assert res >= self.G, (
            f"Cannot flush {self.G} tokens: residual only has {res} at layer {i}.")
        st.flush()
        self._record_flushes(i, 1)
        self._cache_view_valid = False

    def _served(self, i: int):
        """[history || residual] of layer i on the model's device."""
        st = self._stores[i]
        n_hist = st.quantized_tokens
        parts_k, parts_v = [], []
        if n_hist:
            # Rows [0, n_hist) of the history are never written again.
            parts_k.append(st.k_hist[:, :, :n_hist])
            parts_v.append(st.v_hist[:, :, :n_hist])
        if st.res_len:
            rk, rv = st.residual()
            parts_k.append(rk)
            parts_v.append(rv)
        dev = self._serve_device[i] or self.device
        if len(parts_k) == 1:
            k, v = parts_k[0], parts_v[0]
            if st.res_len:
                # The ring slots are reused by later tokens: serve a copy.
                k, v = k.clone(), v.clone()
        else:
            k, v = torch.cat(parts_k, dim=2), torch.cat(parts_v, dim=2)
        dt = self._serve_dtype[i] or torch.float32
        return k.to(dev, dt), v.to(dev, dt)

    # ------------------------------------------------------------ stats / debug
    @property
    def total_flushes(self) -> int:
        return sum(self._flush_count)

    def get_stats(self, layer: int = 0) -> dict:
        """Token and byte accounting for one layer (manager.py:384-419):
        ``kivi_bytes`` is the 2-bit store (packed codes plus fp32 scales and
        zeros) plus the fp32 residual window; ``fp32_bytes`` is what an
        unquantised fp32 cache of the same length would take."""
        B = self.batch_size or 1
        H = self.num_kv_heads or 1
        i = layer
        st = self._stores[i] if self._fed[i] else None
        quant_tokens = self._quant_token_count[i]
        res_tokens = st.res_len if st is not None else 0
        total = quant_tokens + res_tokens
        quant_bytes = self._quant_bytes[i]
        res_bytes = 2 * st.B * st.H * res_tokens * self.head_dim * 4 if st is not None else 0
        fp32_bytes = 2 * B * H * total * self.head_dim * 4
        kivi = quant_bytes + res_bytes
        return {
            "total_tokens": total,
            "quantized_tokens": quant_tokens,
            "residual_tokens": res_tokens,
            "kivi_bytes": kivi,
            "fp32_bytes": fp32_bytes,
            "compression": fp32_bytes / kivi if kivi > 0 else 0,
        }

    # -------------------------------------------------- packed-store access
    def store(self, layer: int) -> Optional[PackedKVStore]:
        """The layer's HBM store (None before the layer was fed)."""
        return self._stores[layer] if self._fed[layer] else None

    def attention(self, layer: int, q: torch.Tensor, softmax_scale: Optional[float] = None,
                  out: Optional[torch.Tensor] = None, kv_start=None,
                  key_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Fused decode attention of one query token per sequence,
        ``q [B, Hq, D]``, over this layer's packed history and residual
        window, straight from the 2-bit store (no dequantised copy).
        ``kv_start`` / ``key_mask`` (``[B, T]`` over the layer's context,
        nonzero = attended): a padded batch's hidden positions, as
        ``PackedKVStore.attention`` takes them."""
        st = self.store(layer)
        if st is None:
            raise RuntimeError(f"layer {layer} holds no tokens yet")
        return st.attention(q.to(self.device, torch.float32), softmax_scale=softmax_scale,
                            out=out, kv_start=kv_start, key_mask=key_mask)

    def __repr__(self):
        return (f"KiviCache(layers={self.num_layers}, head_dim={self.head_dim}, "
                f"G={self.G}, R={self.R}, device='{self.device}')")
