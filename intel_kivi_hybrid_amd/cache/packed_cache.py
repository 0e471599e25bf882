"""KiviPackedCache: the KIVI 2-bit cache as a ``transformers.Cache`` whose
decode attention reads the packed store directly.

The reference hands the model a fresh fp32 ``DynamicCache`` built from the
dequantised history plus the fp32 residual window on every decode step
(src/kivi_sycl/cache/manager.py:251-290, generation/generate.py:75-77), and the
model's attention then reads 1,024 B per token and kv head (D=128) instead of
the 128 B the 2-bit store holds.  Here the cache plugs into the model's own
``past_key_values.update()`` call and its attention dispatch:

* ``update()`` appends the step's new K/V to the layer's HBM residual ring
  (:class:`~intel_kivi_hybrid_amd.store.PackedKVStore`) and returns them
  tagged with the layer;
* the attention function registered as ``"kivi_packed"`` runs the fused HIP
  decode kernel over [packed history ; residual ring] of that layer, with no
  dequantised copy of anything, and then performs the flushes the step owes
  (residual >= R), i.e. in the reference's order: attention of step t sees
  the new token in fp32, and add_tokens() flushes afterwards
  (manager.py:242-249);
* a prompt (more than one token on an empty layer) attends over its own
  unquantised K/V with PyTorch SDPA, exactly like the reference's prefill
  forward with a plain cache (generate.py:56-60), and is then quantised into
  the store with the same flush rule;
* a forward of several tokens on a non-empty layer (chunked prefill, the
  verification pass of assisted decoding) appends them all to the window and
  runs the multi-token kernel, causal over [packed history ; window]: what
  the reference's flow computes when the model is handed
  get_full_cache() and a multi-token input.  Its flushes wait for the next
  update, so crop() can still drop any of those tokens (assisted decoding
  discards the rejected drafts that way);
* a padded batch's mask (HF's ``[B, 1, q_len, kv_len]``: hidden key
  positions, causal among the new tokens) reaches the kernels as each
  sequence's first visible position (left padding) or as hidden-position
  bits (right padding, holes); the reference hands any mask to HF attention
  over get_full_cache() (generate.py:76).

The served-cache path (:class:`KiviCache` with ``get_full_cache()``) stays the
drop-in for the reference's control flow; this class is the fast path for
models that use HF's attention interface (GPT-2, Llama, Mistral, ...).
"""

from __future__ import annotations

import contextlib
from typing import List, Optional

import torch
from transformers.cache_utils import Cache, CacheLayerMixin
from transformers.integrations.sdpa_attention import sdpa_attention_forward
from transformers.masking_utils import AttentionMaskInterface, causal_mask_function, sdpa_mask
from transformers.modeling_utils import AttentionInterface

from .. import _C
from ..config.model_config import detect_model_config
from ..extension.loader import kivi_native  # noqa: F401  (fails loudly without the HIP library)
from ..store import PackedKVStore, decode_geometry_error
from .manager import _resolve_device

__all__ = ["KIVI_ATTENTION", "FORMAT_NAME", "FORMAT_VERSION", "KiviPackedCache",
           "kivi_packed_attention_forward", "packed_attention", "register_packed_attention"]

#: Name of the attention implementation that consumes a KiviPackedCache.
KIVI_ATTENTION = "kivi_packed"

#: safetensors metadata tags of a saved KiviPackedCache.
FORMAT_NAME = "kivi-packed-kv"
FORMAT_VERSION = 1

# The store class the layers allocate (a seam for host-only tests of the
# cache's control flow).
_STORE_CLASS = PackedKVStore


def store_bytes(B: int, H: int, D: int, G: int, Gv: int, n_chunks: int, res_len: int,
                res_elem_bytes: int = 4) -> dict:
    """Byte accounting of one layer's store contents (manager.py:350-356
    generalised to separate key and value group sizes): 2-bit codes, fp32
    scales and zeros (keys per channel and chunk, values per token and Gv
    channels), and the residual window (fp32 like the reference's, or 2
    bytes per element for a bf16/fp16 ring)."""
    tokens = n_chunks * G
    codes = 2 * B * H * tokens * D // 4
    k_meta = B * H * n_chunks * D * 4 * 2
    v_meta = B * H * tokens * (D // Gv) * 4 * 2
    residual = 2 * B * H * res_len * D * res_elem_bytes
    return {"codes": codes, "k_scales_zeros": k_meta, "v_scales_zeros": v_meta,
            "residual": residual, "quantized": codes + k_meta + v_meta}


class KiviPackedLayer(CacheLayerMixin):
    """One layer of a :class:`KiviPackedCache`: an HBM store plus the count of
    flushes it has done."""

    is_compileable = False
    is_sliding = False
    supports_early_init = False

    def __init__(self, owner: "KiviPackedCache", index: int):
        super().__init__()
        self.owner = owner
        self.index = index
        self.store: Optional[PackedKVStore] = None
        self.flushes = 0
        # True while the layer's latest update was a prompt (attended with SDPA).
        self._prompt = False
        # Set by a single-token update, cleared by the packed attention: an
        # update that finds it still set means the model attended with some
        # other implementation and saw only the new token.
        self._awaiting_attention = False

    # ------------------------------------------------------------ state
    @property
    def batch_size(self) -> int:
        if not self.is_initialized:
            raise AttributeError("batch_size")
        return self.store.B

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        o = self.owner
        B, H, _, D = key_states.shape
        if D != o.head_dim:
            raise ValueError(f"KiviPackedCache was built for head_dim {o.head_dim} but layer "
                             f"{self.index} has key head_dim {D}")
        if o.num_kv_heads is not None and H != o.num_kv_heads:
            raise ValueError(f"KiviPackedCache was built for {o.num_kv_heads} kv heads but "
                             f"layer {self.index} has {H}")
        # The ring keeps a half-precision model's K/V in their own type
        # (lossless, half the bytes); anything else in fp32.
        rdt = key_states.dtype if key_states.dtype in (torch.bfloat16, torch.float16) \
            else torch.float32
        st = self.store
        if st is None or st.B != B or st.H != H or st.residual_dtype != rdt:
            self.store = _STORE_CLASS(B, H, D, o.G, o.R, o.device, group_size_v=o.Gv,
                                      chunk_capacity=o.chunk_capacity, residual_dtype=rdt)
        else:
            st.reset()
        self.dtype, self.device = key_states.dtype, key_states.device
        self.flushes = 0
        self._awaiting_attention = False
        self.is_initialized = True

    def get_seq_length(self) -> int:
        if not self.is_initialized:
            return 0
        return self.store.quantized_tokens + self.store.res_len

    def get_mask_sizes(self, query_length: int) -> tuple:
        return self.get_seq_length() + query_length, 0

    def get_max_length(self) -> int:
        return -1

    def reset(self) -> None:
        if self.store is not None:
            self.store.reset()
        self.flushes = 0
        self._awaiting_attention = False
        self.is_initialized = False

    def settle(self) -> None:
        """Flush the G oldest residual tokens while the window holds R or more
        (manager.py:242-249)."""
        st = self.store
        while st.res_len >= self.owner.R:
            st.flush()
            self.flushes += 1

    # ------------------------------------------------------------ update
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        """Append ``[B, Hkv, n, D]`` new K/V and return them tagged with this
        layer for the ``"kivi_packed"`` attention."""
        if self._awaiting_attention:
            raise RuntimeError(
                f"KiviPackedCache layer {self.index}: the previous decode step did not run the "
                f"'{KIVI_ATTENTION}' attention, so it attended over the new token only.  Run the "
                f"model with attn_implementation='{KIVI_ATTENTION}' (see packed_attention()).")
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        st = self.store
        B, H = key_states.shape[0], key_states.shape[1]
        if B != st.B or H != st.H:
            raise ValueError(f"KiviPackedCache layer {self.index} holds batch {st.B} x {st.H} kv "
                             f"heads but got {B} x {H}; call reset() before a new batch")
        self.settle()
        n = key_states.shape[-2]
        k, v = key_states, value_states
        dev = st.device.index
        if k.get_device() != dev or v.get_device() != dev:
            k, v = k.to(st.device), v.to(st.device)
        if self.get_seq_length() == 0:
            # Prompt: attention reads these tensors, the store takes them
            # (every owed chunk in one flush launch).
            self.flushes += st.extend(k, v, flush_at=self.owner.R)
            self._prompt = True
        elif n == 1:
            st.stage_token(k, v)     # room: settle() left res_len < R; written by attend()
            self._prompt = False
            self._awaiting_attention = True
        else:
            # Every new token stays unquantised until the step has attended
            # (room for R - 1 + n, so steps of this size never grow it again).
            st.grow_residual(max(st.res_len + n, self.owner.R - 1 + n))
            st.append(k, v)
            self._prompt = False
            self._awaiting_attention = True
        kt, vt = key_states.view_as(key_states), value_states.view_as(value_states)
        kt._kivi_layer = self
        vt._kivi_layer = self
        return kt, vt

    # --------------------------------------------------------- attention
    def attend(self, query: torch.Tensor, scaling: Optional[float],
               kv_start: Optional[torch.Tensor] = None,
               hidden: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Attention of ``query [B, Hq, L, D]`` (the step's L new tokens, the
        window's newest) over this layer's store, causal among them; returns
        ``[B, L, Hq, D]`` in the query's dtype and device.  ``kv_start``
        (int32 ``[B]`` on the store's device): each sequence's first visible
        position, for a left-padded batch; ``hidden`` (int32 words,
        ``_C.hidden_positions``): any other padding pattern.  A one-token
        step does its flushes now; a longer one leaves them to the next
        update."""
        st = self.store
        B, Hq, L, D = query.shape
        # (each decode step calls this once per layer: no-op conversions are
        # skipped, since each costs about a microsecond of host time)
        native = query.dtype is torch.float32 and query.get_device() == st.device.index
        q = query if native else query.to(st.device, torch.float32)
        if L == 1:
            # [B, Hq, 1, D] is the decode kernel's query as it stands
            o = st.attention(q.contiguous(), softmax_scale=scaling, kv_start=kv_start,
                             hidden=hidden).view(B, 1, Hq, D)
        else:
            o = st.attention(q, softmax_scale=scaling, causal=True, kv_start=kv_start,
                             hidden=hidden)
        self._awaiting_attention = False
        if L == 1:
            self.settle()
        return o if native else o.to(query.device, query.dtype)

    # ------------------------------------------------------------ edits
    def crop(self, tokens_to_remove: int) -> None:
        """Drop the newest tokens (transformers' ``crop``: a negative count
        removes that many; a positive one is the length to keep).  Only
        tokens still in the residual window can go: a quantised chunk is
        final (the window holds every token of the latest multi-token step,
        and at least R - G of a prompt's last tokens)."""
        if not self.is_initialized:
            return
        tokens_to_remove = int(tokens_to_remove)
        n = self.get_seq_length()
        if tokens_to_remove > 0:
            if tokens_to_remove >= n:
                return
            drop = n - tokens_to_remove
        else:
            drop = -tokens_to_remove
        if drop:
            self.store.rollback(drop)

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        if self.get_seq_length() > 0:
            self.store.select_batch(beam_idx.to(self.store.device))

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        self.reorder_cache(indices)

    def batch_repeat_interleave(self, repeats: int) -> None:
        if self.get_seq_length() > 0:
            idx = torch.arange(self.store.B, device=self.store.device).repeat_interleave(repeats)
            self.store.select_batch(idx)

    def offload(self):
        raise NotImplementedError("KiviPackedCache keeps its store in GPU memory")

    def prefetch(self):
        raise NotImplementedError("KiviPackedCache keeps its store in GPU memory")


class KiviPackedCache(Cache):
    """KIVI 2-bit KV cache for HF models, attended in place.

    Args mirror :class:`KiviCache` (manager.py:52-133): ``num_layers``,
    ``head_dim``, ``num_kv_heads``, ``device`` (HIP device of the store),
    ``group_size`` (G, key group along tokens and chunk length),
    ``residual_length`` (R, the residual window: in the model's K/V type for
    bf16/fp16 models, else fp32), plus ``value_group_size`` (value
    group along channels, default G) and ``chunk_capacity`` (chunks to
    preallocate per layer; the store grows by doubling beyond it).

    Use it with the model's attention set to ``"kivi_packed"``::

        cache = KiviPackedCache.from_model(model)
        with packed_attention(model):
            out = model.generate(input_ids, past_key_values=cache, do_sample=False)
    """

    def __init__(self, num_layers: int, head_dim: int, num_kv_heads: Optional[int] = None,
                 device: str = "cuda", group_size: int = 32, residual_length: int = 128,
                 value_group_size: Optional[int] = None, chunk_capacity: int = 0):
        assert group_size >= 4 and group_size % 4 == 0, \
            f"group_size ({group_size}) must be >= 4 and divisible by 4"
        gv = group_size if value_group_size is None else value_group_size
        assert gv >= 4 and gv % 4 == 0 and head_dim % gv == 0, \
            f"head_dim ({head_dim}) must be divisible by value group size ({gv})"
        assert group_size <= residual_length, (
            f"group_size ({group_size}) must not exceed residual_length ({residual_length})")
        # Refuse a geometry the decode kernel cannot run now, not at the first
        # decode step after the prompt (the query-head ratio is checked at the
        # first attention call, where the query's head count is known).
        err = decode_geometry_error(num_kv_heads or 1, num_kv_heads or 1, head_dim, group_size,
                                    gv)
        if err:
            raise ValueError(f"KiviPackedCache: the packed decode attention does not support "
                             f"head_dim={head_dim}, group_size={group_size}, "
                             f"value_group_size={gv}: {err}")
        self._heads_checked = False
        # (mask, kv_start) of the latest padded forward: every layer of a
        # forward receives the same mask object, which is read once.
        self._mask_memo = None
        register_packed_attention()
        self.device = _resolve_device(device)
        self.head_dim = head_dim
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.G, self.Gv, self.R = group_size, gv, residual_length
        self.chunk_capacity = max(int(chunk_capacity), 1)
        super().__init__(layers=[KiviPackedLayer(self, i) for i in range(num_layers)])

    @classmethod
    def from_model(cls, model, device: str = "cuda", group_size: int = 32,
                   residual_length: int = 128, value_group_size: Optional[int] = None,
                   chunk_capacity: int = 0) -> "KiviPackedCache":
        """A cache sized from a HuggingFace model's config (manager.py:135-156)."""
        cfg = detect_model_config(model)
        return cls(cfg["num_layers"], cfg["head_dim"], cfg["num_kv_heads"], device=device,
                   group_size=group_size, residual_length=residual_length,
                   value_group_size=value_group_size, chunk_capacity=chunk_capacity)

    # ----------------------------------------------------------- access
    def store(self, layer: int) -> Optional[PackedKVStore]:
        lay = self.layers[layer]
        return lay.store if lay.is_initialized else None

    @property
    def total_flushes(self) -> int:
        return sum(lay.flushes for lay in self.layers)

    def get_stats(self, layer: int = 0) -> dict:
        """Token and byte accounting of one layer's store, with the keys of
        KiviCache.get_stats (manager.py:384-419); the byte counts are those
        of the tensors actually held, itemised under ``bytes``."""
        st = self.store(layer)
        if st is None:
            return {"total_tokens": 0, "quantized_tokens": 0, "residual_tokens": 0,
                    "kivi_bytes": 0, "fp32_bytes": 0, "compression": 0}
        b = store_bytes(st.B, st.H, st.D, st.G, st.Gv, st.n_chunks, st.res_len,
                        st.residual_dtype.itemsize)
        total = st.quantized_tokens + st.res_len
        kivi = b["quantized"] + b["residual"]
        fp32 = 2 * st.B * st.H * total * st.D * 4
        return {"total_tokens": total, "quantized_tokens": st.quantized_tokens,
                "residual_tokens": st.res_len, "kivi_bytes": kivi, "fp32_bytes": fp32,
                "compression": fp32 / kivi if kivi > 0 else 0, "bytes": b,
                "allocated_bytes": st.allocated_bytes()}

    # ----------------------------------------------------------- format
    def save(self, path: str) -> None:
        """Write the cache to a safetensors file.

        Per fed layer i, tensors ``layers.{i}.k_codes`` ``[B, Hkv, D, T/4]``
        u8, ``k_scale``/``k_zero`` ``[B, Hkv, D, T/G]``, ``v_codes``
        ``[B, Hkv, T, D/4]`` u8, ``v_scale``/``v_zero`` ``[B, Hkv, T, D/Gv]``
        (the layouts of the reference's quantize_keys / quantize_values over
        the T quantised tokens, kv_cache_ops.cpp:179-199) and the residual
        windows ``k_residual``/``v_residual`` ``[B, Hkv, r, D]`` in the
        ring's type (fp32, or bf16/fp16 for a half-precision model);
        the file metadata holds the format tag, version, cache geometry and
        per-layer flush counts.  The file holds the cache as the next update
        will find it: flushes a multi-token step still owes are done on a
        copy of that layer's store (the file's windows hold fewer than R
        tokens), and the live cache is left as it was, so a crop() of that
        step's tokens still works after a save."""
        from safetensors.torch import save_file
        meta = {"format": FORMAT_NAME, "version": str(FORMAT_VERSION),
                "num_layers": str(self.num_layers), "head_dim": str(self.head_dim),
                "num_kv_heads": str(self.num_kv_heads or 0), "group_size": str(self.G),
                "value_group_size": str(self.Gv), "residual_length": str(self.R)}
        tensors = {}
        for i, lay in enumerate(self.layers):
            st = self.store(i)
            if st is None:
                continue
            state, flushes = st.export_state(), lay.flushes
            if st.res_len >= self.R:
                tmp = _STORE_CLASS.from_state(state, self.G, st.res_len, st.device,
                                              group_size_v=self.Gv)
                while tmp.res_len >= self.R:       # settle(), on the copy
                    tmp.flush()
                    flushes += 1
                state = tmp.export_state()
                del tmp
            for name, t in state.items():
                tensors[f"layers.{i}.{name}"] = t.contiguous().cpu()
            meta[f"layers.{i}.flushes"] = str(flushes)
        save_file(tensors, path, metadata=meta)

    @classmethod
    def load(cls, path: str, device: str = "cuda") -> "KiviPackedCache":
        """Read a file written by :meth:`save` into a new cache on ``device``;
        the codes are re-ordered into this build's store layout."""
        from safetensors import safe_open
        with safe_open(path, framework="pt") as f:
            meta = f.metadata() or {}
            if meta.get("format") != FORMAT_NAME:
                raise ValueError(f"{path} is not a KiviPackedCache file "
                                 f"(format tag {meta.get('format')!r})")
            if meta.get("version") != str(FORMAT_VERSION):
                raise ValueError(f"{path} has format version {meta.get('version')!r}; this "
                                 f"build reads version {FORMAT_VERSION}")
            try:
                geo = {k: int(meta[k]) for k in ("num_layers", "head_dim", "num_kv_heads",
                                                 "group_size", "value_group_size",
                                                 "residual_length")}
            except (KeyError, ValueError) as exc:
                raise ValueError(f"{path} has incomplete cache metadata: {exc}") from exc
            cache = cls(geo["num_layers"], geo["head_dim"], geo["num_kv_heads"] or None,
                        device=device, group_size=geo["group_size"],
                        residual_length=geo["residual_length"],
                        value_group_size=geo["value_group_size"])
            keys = list(f.keys())
            for i, lay in enumerate(cache.layers):
                prefix = f"layers.{i}."
                names = [k for k in keys if k.startswith(prefix)]
                if not names:
                    continue
                state = {k[len(prefix):]: f.get_tensor(k) for k in names}
                lay.store = _STORE_CLASS.from_state(state, cache.G, cache.R, cache.device,
                                                    group_size_v=cache.Gv)
                lay.flushes = int(meta.get(prefix + "flushes", "0"))
                lay.dtype, lay.device = lay.store.residual_dtype, cache.device
                lay.is_initialized = True
            stray = [k for k in keys if not k.startswith("layers.")
                     or int(k.split(".")[1]) >= cache.num_layers]
            if stray:
                raise ValueError(f"{path} holds tensors outside the cache's layers: {stray[:4]}")
        return cache

    def __repr__(self):
        return (f"KiviPackedCache(layers={self.num_layers}, head_dim={self.head_dim}, "
                f"G={self.G}, Gv={self.Gv}, R={self.R}, device='{self.device}')")


def kivi_packed_attention_forward(module, query, key, value, attention_mask, scaling=None,
                                  dropout=0.0, **kwargs):
    """HF attention function for a :class:`KiviPackedCache`.

    One-token (decode) steps run the fused packed-KV kernel over the layer's
    store; prompt passes go to PyTorch SDPA over the prompt's own K/V.
    Returns ``(attn_output [B, q_len, Hq, D], None)`` as HF's attention
    functions do (models/gpt2/modeling_gpt2.py:54-73 in transformers)."""
    layer = getattr(key, "_kivi_layer", None)
    if layer is None:
        raise RuntimeError(f"the '{KIVI_ATTENTION}' attention needs past_key_values to be a "
                           f"KiviPackedCache and use_cache=True")
    owner = layer.owner
    if not owner._heads_checked:
        err = decode_geometry_error(query.shape[1], key.shape[1], owner.head_dim, owner.G,
                                    owner.Gv)
        if err:
            raise ValueError(f"KiviPackedCache: {query.shape[1]} query heads over "
                             f"{key.shape[1]} kv heads cannot be decoded from the packed "
                             f"store: {err}")
        owner._heads_checked = True
    if layer._prompt:
        return sdpa_attention_forward(module, query, key, value, attention_mask,
                                      dropout=dropout, scaling=scaling, **kwargs)
    if dropout:
        raise ValueError(f"'{KIVI_ATTENTION}' attention is inference-only (dropout={dropout})")
    for name in ("sliding_window", "softcap", "s_aux"):
        if kwargs.get(name) is not None:
            raise NotImplementedError(f"'{KIVI_ATTENTION}' attention does not support {name}")
    kv_start = hidden = None
    if attention_mask is not None:
        kv_start, hidden = _mask_plan(owner, attention_mask, query.shape[2],
                                      layer.get_seq_length(), layer.store.device)
    return layer.attend(query, scaling, kv_start, hidden), None


def _mask_plan(owner: "KiviPackedCache", mask: torch.Tensor, q_len: int, kv_len: int, device):
    """How the packed kernels apply HF's attention mask ``[B, 1, q_len,
    kv_len]`` (bool: True = attend; float: 0 = attend, at most half the
    dtype's lowest value = hidden): ``(kv_start, None)`` with each
    sequence's first visible position for a left-padded batch, else
    ``(None, hidden)`` with the hidden-position words of any other
    key-padding pattern (right padding, holes).  The mask must be exactly
    "the newest token's visible positions, causal among the new tokens",
    which is checked (one device sync per forward: every layer gets the same
    mask object, read once); anything else -- an additive bias, a
    per-query pattern other than causal -- is refused."""
    memo = owner._mask_memo
    if memo is not None and memo[0] is mask:
        return memo[1]
    plan = None
    if mask.dim() == 4 and mask.shape[1] == 1 and tuple(mask.shape[2:]) == (q_len, kv_len):
        m = mask[:, 0]
        attend = None
        if m.dtype == torch.bool:
            attend = m
        elif m.is_floating_point():
            low = torch.finfo(m.dtype).min / 2
            if bool(((m == 0) | (m <= low)).all()):
                attend = m == 0
        if attend is not None:
            vis = attend[:, -1, :]                      # the newest token's visible positions
            t = torch.arange(kv_len, device=mask.device)
            newest = kv_len - q_len + torch.arange(q_len, device=mask.device)
            if torch.equal(attend, vis[:, None, :] & (t[None, None, :] <= newest[None, :, None])):
                s = vis.int().argmax(-1)                # first visible position
                if torch.equal(vis, t[None, :] >= s[:, None]):
                    plan = (s.to(device=device, dtype=torch.int32), None)
                else:
                    plan = (None, _C.hidden_positions(vis, device))
    if plan is None:
        raise NotImplementedError(
            f"'{KIVI_ATTENTION}' attention over the cache takes HF's mask of a padded batch "
            f"(hidden key positions, causal among the new tokens); this mask is something "
            f"else (shape {tuple(mask.shape)}, dtype {mask.dtype})")
    owner._mask_memo = (mask, plan)
    return plan


def kivi_causal_mask(batch_size: int, q_length: int, kv_length: int, q_offset: int = 0,
                     kv_offset: int = 0, mask_function=causal_mask_function,
                     attention_mask: Optional[torch.Tensor] = None,
                     local_size: Optional[int] = None, allow_is_causal_skip: bool = True,
                     **kwargs):
    """Mask function of the ``"kivi_packed"`` attention: ``None`` when the
    mask is the plain causal one over [cache ; new tokens] with no padding
    (the new tokens are the newest kv positions), which the packed kernels
    apply themselves at any cache length; anything else is SDPA's mask
    (transformers.masking_utils.sdpa_mask), which prompt passes use and the
    packed path refuses."""
    if (allow_is_causal_skip and mask_function is causal_mask_function and local_size is None
            and kv_offset == 0 and q_offset + q_length == kv_length
            and (attention_mask is None or bool(attention_mask[:, -kv_length:].all()))):
        return None
    return sdpa_mask(batch_size=batch_size, q_length=q_length, kv_length=kv_length,
                     q_offset=q_offset, kv_offset=kv_offset, mask_function=mask_function,
                     attention_mask=attention_mask, local_size=local_size,
                     allow_is_causal_skip=allow_is_causal_skip, **kwargs)


_registered = False


def register_packed_attention() -> None:
    """Register ``"kivi_packed"`` with transformers' attention and mask
    interfaces."""
    global _registered
    if not _registered:
        AttentionInterface.register(KIVI_ATTENTION, kivi_packed_attention_forward)
        AttentionMaskInterface.register(KIVI_ATTENTION, kivi_causal_mask)
        _registered = True


@contextlib.contextmanager
def packed_attention(model):
    """Run ``model`` with the ``"kivi_packed"`` attention inside the block and
    restore its previous implementation afterwards."""
    register_packed_attention()
    prev = model.config._attn_implementation
    model.set_attn_implementation(KIVI_ATTENTION)
    if model.config._attn_implementation != KIVI_ATTENTION:
        raise RuntimeError(f"{type(model).__name__} does not accept the '{KIVI_ATTENTION}' "
                           f"attention implementation")
    try:
        yield model
    finally:
        model.set_attn_implementation(prev)
