"""HBM-resident packed KV store for one attention layer.

The reference keeps the fp32 residual and a dequantised fp32 history on the
CPU and sends one G-token chunk to the device per flush
(src/kivi_sycl/cache/manager.py:100-118,309-374).  Here everything stays in
device memory:

* a residual ring ``[B, Hkv, R, D]`` (``res_start``/``res_len`` track the
  window; a flush advances ``res_start`` by G instead of moving data), fp32
  like the reference's, or bf16/fp16 for a model whose K/V are of that type
  (lossless for them: the kernels widen exactly, so results equal those of
  an fp32 ring holding the same values);
* the packed store (codes, scales, zeros per chunk of G tokens, layout in
  include/kivi_hip.h), grown geometrically;
* optionally the dequantised history ``[B, Hkv, T, D]`` that
  ``KiviCache.get_full_cache()`` serves (written by the flush kernel itself).

Flushes and attention launch the HIP kernels of ``libkivi_hip.so`` on the
current stream; the only torch work is allocation and plain copies.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _C, _native
from ._device import on_device, stream_handle

_lib = _native.load()

# Element types the flush kernel reads directly (code passed to the C ABI).
_SRC_DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
_MAX_CHUNKS_PER_LAUNCH = 65535


def _vp(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _stream(device) -> int:
    return stream_handle(device)


def _pack_last(codes: torch.Tensor) -> torch.Tensor:
    """[..., N] codes (one per byte) -> [..., N/4] bytes, element 4j+k at bits 2k."""
    c = codes.to(torch.int32).reshape(*codes.shape[:-1], codes.shape[-1] // 4, 4)
    return (c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)).to(torch.uint8)


_MAPS = {}


def _mfma_maps(G: int, D: int, key: bool):
    """For the matrix-core code layout: the flat [G][D] index of every
    (lane, word, tile-in-word, element) and the bit shift of each of the 16
    codes of a word (include/kivi_hip.h documents the layout)."""
    cache_key = (G, D, key)
    if cache_key not in _MAPS:
        np_ = G * D // 1024
        flat = torch.empty(64, np_, 16, dtype=torch.long)
        shifts = torch.empty(16, dtype=torch.int32)
        for m in range(2):
            for j in range(8):
                shifts[8 * m + j] = 8 * m + 2 * (j // 2) + 16 * (j % 2)
        for lane in range(64):
            for w in range(np_):
                for m in range(2):
                    tile = 2 * w + m
                    for j in range(8):
                        if key:
                            ks, nb = divmod(tile, G // 16)
                            t, d = 16 * nb + lane % 16, 32 * ks + 8 * (lane // 16) + j
                        else:
                            kt, nb = divmod(tile, D // 16)
                            t, d = 32 * kt + 8 * (lane // 16) + j, 16 * nb + lane % 16
                        flat[lane, w, 8 * m + j] = t * D + d
        _MAPS[cache_key] = (flat.reshape(-1), shifts)
    return _MAPS[cache_key]


def _unpack_last(packed: torch.Tensor) -> torch.Tensor:
    """[..., N/4] bytes -> [..., N] codes (uint8), element 4j+k from bits 2k of byte j."""
    b = packed.to(torch.int32)
    c = torch.stack([(b >> (2 * k)) & 3 for k in range(4)], dim=-1)
    return c.reshape(*packed.shape[:-1], packed.shape[-1] * 4).to(torch.uint8)


def decode_codes(raw: torch.Tensor, G: int, D: int, layout: int, key: bool) -> torch.Tensor:
    """Chunk code bytes in the store's order (``raw [..., G*D/4]``) -> one
    code per byte as ``[..., G, D]`` (token, channel)."""
    lead = raw.shape[:-1]
    if layout == 0:
        c = _unpack_last(raw)
        if key:                                        # [G][D/4], channels packed
            return c.reshape(*lead, G, D)
        return c.reshape(*lead, D, G).transpose(-1, -2).contiguous()   # [D][G/4]
    words = raw.contiguous().view(torch.int32).reshape(*lead, -1)        # [..., 64*NP]
    flat, shifts = _mfma_maps(G, D, key)
    vals = (words[..., :, None] >> shifts.to(raw.device)) & 3          # [..., 64*NP, 16]
    out = torch.empty(*lead, G * D, dtype=torch.int32, device=raw.device)
    out[..., flat.to(raw.device)] = vals.reshape(*lead, -1)
    return out.reshape(*lead, G, D).to(torch.uint8)


def encode_codes(codes: torch.Tensor, G: int, D: int, layout: int, key: bool) -> torch.Tensor:
    """Inverse of :func:`decode_codes`: ``codes [..., G, D]`` (values 0..3) ->
    chunk code bytes ``[..., G*D/4]`` in the store's order."""
    lead = codes.shape[:-2]
    if layout == 0:
        if key:
            return _pack_last(codes).reshape(*lead, G * D // 4)
        return _pack_last(codes.transpose(-1, -2)).reshape(*lead, G * D // 4)
    flat, shifts = _mfma_maps(G, D, key)
    c = codes.reshape(*lead, G * D).to(torch.int64)[..., flat.to(codes.device)]
    c = c.reshape(*lead, -1, 16) << shifts.to(codes.device, torch.int64)
    words = c.sum(dim=-1)                                                # [..., 64*NP]
    b = torch.stack([(words >> (8 * k)) & 0xFF for k in range(4)], dim=-1)
    return b.to(torch.uint8).reshape(*lead, G * D // 4)


def decode_geometry_error(q_heads: int, kv_heads: int, head_dim: int, group_size: int,
                          group_size_v: int) -> Optional[str]:
    """None if the fused decode attention runs stores of this geometry (any
    context length), else the reason it would refuse them."""
    rc = _lib.kivi_packed_decode_attention_supported(q_heads, kv_heads, head_dim, group_size,
                                                     group_size_v)
    return None if rc == 0 else _native.last_error()


def append_layers(stores, ks, vs) -> None:
    """``stores[i].append(ks[i], vs[i])`` for one step of several stores (a
    model's layers), with one launch per 16 layers (kivi_store_append_layers)
    for the layers that share the first one's shapes, ring type, input type
    and strides and take their inputs as they are (on the store's device,
    channels contiguous, K and V alike); any other layer is appended on its
    own.  Every window must have room (callers flush first)."""
    n = len(stores)
    if n == 0:
        return
    st0, k0 = stores[0], ks[0]
    shape, dtype, strides = k0.shape, k0.dtype, k0.stride()
    ok = (k0.dim() == 4 and dtype in _SRC_DTYPES and strides[3] == 1 and
          (st0.k_res.dtype == torch.float32 or st0.k_res.dtype == dtype) and
          tuple(shape) == (st0.B, st0.H, shape[2], st0.D))
    batch, rest = [], []
    for st, k, v in zip(stores, ks, vs):
        if (ok and k.shape == shape and v.shape == shape and k.dtype is dtype and
                v.dtype is dtype and k.stride() == strides and v.stride() == strides and
                k.get_device() == st.device.index and v.get_device() == st.device.index and
                st.B == st0.B and st.H == st0.H and st.D == st0.D and st.R == st0.R and
                st.k_res.dtype is st0.k_res.dtype and st.device == st0.device):
            batch.append((st, k, v))
        else:
            rest.append((st, k, v))
    for st, k, v in rest:
        st.append(k, v)
    if not batch:
        return
    m, ntok = len(batch), shape[2]
    for st, _, _ in batch:
        st._commit()
        if st.res_len + ntok > st.R:
            raise RuntimeError(f"residual window overflow ({st.res_len} + {ntok} > {st.R})")
    kp, vp = (ctypes.c_void_p * m)(), (ctypes.c_void_p * m)()
    kr, vr = (ctypes.c_void_p * m)(), (ctypes.c_void_p * m)()
    sl = (ctypes.c_int32 * m)()
    for i, (st, k, v) in enumerate(batch):
        kp[i], vp[i] = k.data_ptr(), v.data_ptr()
        kr[i], vr[i] = st.k_res.data_ptr(), st.v_res.data_ptr()
        sl[i] = (st.res_start + st.res_len) % st.R
    sd = (ctypes.c_int64 * (3 * m))(*(strides[:3] * m))
    with on_device(st0.device):
        _native.check(_lib.kivi_store_append_layers(
            m, ctypes.addressof(kp), ctypes.addressof(vp), ctypes.addressof(sd),
            _SRC_DTYPES[dtype], ntok, ctypes.addressof(kr), ctypes.addressof(vr),
            st0.res_dtype_code, st0.B, st0.H, st0.D, st0.R, ctypes.addressof(sl),
            _stream(st0.device)), "kivi_store_append_layers")
    for st, _, _ in batch:
        st.res_len += ntok


class PackedKVStore:
    """Residual ring + packed chunks for one layer (all on ``device``)."""

    def __init__(self, batch: int, kv_heads: int, head_dim: int, group_size: int,
                 residual_capacity: int, device, group_size_v: Optional[int] = None,
                 chunk_capacity: int = 0, keep_history: bool = False,
                 residual_dtype: torch.dtype = torch.float32):
        if group_size <= 0 or group_size % 4:
            raise ValueError(f"group_size ({group_size}) must be >= 4 and divisible by 4")
        gv = group_size if group_size_v is None else group_size_v
        if gv <= 0 or gv % 4 or head_dim % gv:
            raise ValueError(f"head_dim ({head_dim}) must be divisible by group_size_v ({gv})")
        if residual_capacity < group_size:
            raise ValueError("residual capacity must hold at least one group")
        if residual_dtype not in _SRC_DTYPES:
            raise ValueError(f"residual_dtype must be float32, bfloat16 or float16, got "
                             f"{residual_dtype}")
        self.B, self.H, self.D = batch, kv_heads, head_dim
        self.G, self.Gv, self.R = group_size, gv, residual_capacity
        # 1: codes stored in matrix-core operand order, 0: plain byte order
        self.code_layout = int(_lib.kivi_store_code_layout(head_dim, group_size, gv))
        self.keep_history = keep_history
        self.k_res = torch.zeros(batch, kv_heads, residual_capacity, head_dim,
                                 dtype=residual_dtype, device=torch.device(device))
        self.device = self.k_res.device      # with its index ("cuda" names the current one)
        self.v_res = torch.zeros_like(self.k_res)
        self.res_start = 0
        self.res_len = 0
        self.n_chunks = 0
        self.capacity = 0
        # A token counted in res_len whose K/V are not in the ring yet: the
        # next attention launch writes it (fused), any other use of the ring
        # commits it first.
        self._pending = None
        self._alloc(max(int(chunk_capacity), 1))

    # ------------------------------------------------------------------ alloc
    def _alloc(self, cap: int) -> None:
        B, H, D, G, ng = self.B, self.H, self.D, self.G, self.D // self.Gv
        u8 = dict(dtype=torch.uint8, device=self.device)
        f32 = dict(dtype=torch.float32, device=self.device)
        new = {
            "k_codes": torch.empty(B, H, cap, G * D // 4, **u8),
            "k_scale": torch.empty(B, H, cap, D, **f32),
            "k_zero": torch.empty(B, H, cap, D, **f32),
            "v_codes": torch.empty(B, H, cap, G * D // 4, **u8),
            "v_scale": torch.empty(B, H, cap, ng, G, **f32),
            "v_zero": torch.empty(B, H, cap, ng, G, **f32),
        }
        if self.keep_history:
            new["k_hist"] = torch.empty(B, H, cap * G, D, **f32)
            new["v_hist"] = torch.empty(B, H, cap * G, D, **f32)
        n = self.n_chunks
        for name, t in new.items():
            if n and hasattr(self, name):
                old = getattr(self, name)
                if name.endswith("hist"):
                    t[:, :, :n * G].copy_(old[:, :, :n * G])
                else:
                    t[:, :, :n].copy_(old[:, :, :n])
            setattr(self, name, t)
        if not self.keep_history:
            self.k_hist = self.v_hist = None
        self.capacity = cap

    def reserve(self, n_chunks: int) -> None:
        if n_chunks > self.capacity:
            self._alloc(max(n_chunks, 2 * self.capacity))

    # --------------------------------------------------------------- tokens
    @property
    def quantized_tokens(self) -> int:
        return self.n_chunks * self.G

    @property
    def residual_dtype(self) -> torch.dtype:
        return self.k_res.dtype

    @property
    def res_dtype_code(self) -> int:
        """The ring's element type as the C ABI codes it (0 f32, 1 bf16, 2 f16)."""
        return _SRC_DTYPES[self.k_res.dtype]

    def _launch_append(self, k: torch.Tensor, v: torch.Tensor, slot: int) -> None:
        sb, sh, st, _ = k.stride()
        with on_device(self.device):
            _native.check(_lib.kivi_store_append(
                _vp(k), _vp(v), _SRC_DTYPES[k.dtype], sb, sh, st, k.shape[2], _vp(self.k_res),
                _vp(self.v_res), self.res_dtype_code, self.B, self.H, self.D, self.R, slot,
                _stream(self.device)),
                "kivi_store_append")

    def _commit(self) -> None:
        """Write a staged token into the ring (see stage_token)."""
        if self._pending is not None:
            k, v = self._pending
            self._pending = None
            self._launch_append(k, v, (self.res_start + self.res_len - 1) % self.R)

    def stage_token(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Add one new token ``[B, Hkv, 1, D]`` to the window.  It counts at
        once; its K/V are written by the next :meth:`attention` launch
        itself, which reads them from ``k``/``v`` (rows of the ring's type
        aligned to four elements), or by a separate append when anything
        else reads the ring first or the inputs do not allow the fused
        path."""
        k, v = self._token_source(k, v)
        if k.shape[2] != 1:
            raise ValueError(f"stage_token takes one token, got {k.shape[2]}")
        self._commit()
        if self.res_len + 1 > self.R:
            raise RuntimeError(f"residual window overflow ({self.res_len} + 1 > {self.R})")
        sb, sh = k.stride(0), k.stride(1)
        vb = 4 * k.element_size()
        if k.dtype == self.k_res.dtype and sb % 4 == 0 and sh % 4 == 0 and \
                k.data_ptr() % vb == 0 and v.data_ptr() % vb == 0:
            self._pending = (k, v)
            self.res_len += 1
        else:
            self.append(k, v)

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Copy new tokens ``[B, Hkv, n, D]`` into the residual window (one
        launch for K and V; into an fp32 ring fp32/bf16/fp16 are widened
        exactly; any strides with contiguous channels).  The window must have
        room (callers flush first)."""
        self._commit()
        self._append_source(*self._token_source(k, v))

    def _append_source(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """append() of tokens that _token_source has already prepared."""
        n = k.shape[2]
        if self.res_len + n > self.R:
            raise RuntimeError(f"residual window overflow ({self.res_len} + {n} > {self.R})")
        if n == 0:
            return
        self._launch_append(k, v, (self.res_start + self.res_len) % self.R)
        self.res_len += n

    def _token_source(self, k: torch.Tensor, v: torch.Tensor):
        """New tokens as the flush kernel reads them: on the store's device,
        fp32/bf16/fp16 (for a 16-bit ring: the ring's type, so that every
        token is quantised from the value the ring would hold), channels
        contiguous, K and V with the same strides (copies are made only when
        the inputs are not already so)."""
        if k.shape != v.shape or k.dim() != 4 or tuple(k.shape[:2]) != (self.B, self.H) \
                or k.shape[3] != self.D:
            raise ValueError(f"new tokens must be [B={self.B}, Hkv={self.H}, n, D={self.D}] for "
                             f"both K and V, got {tuple(k.shape)} and {tuple(v.shape)}")
        dev = self.device.index
        if k.get_device() != dev or v.get_device() != dev:
            k, v = k.to(self.device), v.to(self.device)
        if self.k_res.dtype != torch.float32:
            k, v = k.to(self.k_res.dtype), v.to(self.k_res.dtype)
        elif k.dtype not in _SRC_DTYPES or v.dtype != k.dtype:
            k, v = k.to(torch.float32), v.to(torch.float32)
        if k.stride(-1) != 1 or v.stride() != k.stride():
            k, v = k.contiguous(), v.contiguous()
        return k, v

    def extend(self, k: torch.Tensor, v: torch.Tensor, flush_at: Optional[int] = None) -> int:
        """Append ``[B, Hkv, n, D]`` tokens and flush the G oldest while the
        residual holds ``flush_at`` (default: the ring capacity) or more, with
        the result of KiviCache.add_tokens (manager.py:226-249): the flushes
        are ``0`` if res_len + n < flush_at, else ``(res_len + n - flush_at)
        // G + 1``, and they take the oldest tokens of [residual ; new].

        All owed chunks are quantised by one launch that reads the ring and
        ``k``/``v`` in place (any strides with contiguous channels; fp32,
        bf16 or fp16, widened exactly); only the tokens left over are copied
        into the ring.  Returns the number of flushes."""
        R = self.R if flush_at is None else int(flush_at)
        if not self.G <= R <= self.R:
            raise ValueError(f"flush threshold {R} must lie in [{self.G}, {self.R}]")
        self._commit()
        k, v = self._token_source(k, v)
        n = k.shape[2]
        total = self.res_len + n
        n_flush = 0 if total < R else (total - R) // self.G + 1
        skip = 0                        # new tokens already quantised
        done = 0
        if n_flush:
            self.reserve(self.n_chunks + n_flush)
        while done < n_flush:
            m = min(n_flush - done, _MAX_CHUNKS_PER_LAUNCH)
            self._flush_run(k[:, :, skip:], v[:, :, skip:], m)
            used = m * self.G
            from_ring = min(used, self.res_len)
            self.res_start = (self.res_start + from_ring) % self.R
            self.res_len -= from_ring
            skip += used - from_ring
            done += m
        if skip < n:
            if skip:
                k, v = k[:, :, skip:], v[:, :, skip:]
            self._append_source(k, v)
        return n_flush

    def _flush_run(self, k: torch.Tensor, v: torch.Tensor, n_chunks: int) -> None:
        """Quantise ``n_chunks`` chunks from [ring window ; k/v] (one launch)."""
        hist_cap = self.capacity * self.G if self.keep_history else 0
        sb, sh, st, _ = k.stride()
        with on_device(self.device):
            _native.check(_lib.kivi_store_flush_chunks(
                _vp(self.k_res), _vp(self.v_res), self.res_dtype_code, _vp(k), _vp(v),
                _SRC_DTYPES[k.dtype],
                sb, sh, st, k.shape[2], _vp(self.k_codes), _vp(self.k_scale), _vp(self.k_zero),
                _vp(self.v_codes), _vp(self.v_scale), _vp(self.v_zero), _vp(self.k_hist),
                _vp(self.v_hist), hist_cap, self.B, self.H, self.D, self.G, self.Gv, self.R,
                self.res_start, self.res_len, self.capacity, self.n_chunks, n_chunks,
                _stream(self.device)), "kivi_store_flush_chunks")
        self.n_chunks += n_chunks

    def residual(self):
        """The residual window in token order (a copy when it wraps)."""
        self._commit()
        s, n = self.res_start, self.res_len
        if s + n <= self.R:
            return self.k_res[:, :, s:s + n], self.v_res[:, :, s:s + n]
        return (torch.cat([self.k_res[:, :, s:], self.k_res[:, :, :s + n - self.R]], dim=2),
                torch.cat([self.v_res[:, :, s:], self.v_res[:, :, :s + n - self.R]], dim=2))

    def flush(self) -> None:
        """Quantise the G oldest residual tokens into the next chunk."""
        if self.res_len < self.G:
            raise RuntimeError(f"Cannot flush {self.G} tokens: residual only has {self.res_len}")
        self._commit()
        self.reserve(self.n_chunks + 1)
        hist_cap = self.capacity * self.G if self.keep_history else 0
        with on_device(self.device):
            _native.check(_lib.kivi_store_flush(
                _vp(self.k_res), _vp(self.v_res), self.res_dtype_code, _vp(self.k_codes),
                _vp(self.k_scale),
                _vp(self.k_zero), _vp(self.v_codes), _vp(self.v_scale), _vp(self.v_zero),
                _vp(self.k_hist), _vp(self.v_hist), hist_cap, self.B, self.H, self.D,
                self.G, self.Gv, self.R, self.res_start, self.capacity, self.n_chunks,
                _stream(self.device)), "kivi_store_flush")
        self.n_chunks += 1
        self.res_start = (self.res_start + self.G) % self.R
        self.res_len -= self.G

    def reset(self) -> None:
        self.res_start = self.res_len = self.n_chunks = 0
        self._pending = None

    def rollback(self, n: int) -> None:
        """Drop the newest ``n`` tokens of the residual window, e.g. draft
        tokens that a speculative decode rejects (HF ``Cache.crop``).  Only
        tokens not yet quantised can be dropped: a flushed chunk is final."""
        n = int(n)
        if n < 0 or n > self.res_len:
            raise ValueError(f"cannot roll back {n} tokens: the residual window holds "
                             f"{self.res_len} (quantised tokens cannot be rolled back)")
        if n and self._pending is not None:
            self._pending = None          # the staged token is the newest
        self.res_len -= n

    def grow_residual(self, capacity: int) -> None:
        """Give the residual ring room for ``capacity`` tokens (nothing
        happens if it has that already): a forward of several tokens holds
        them all in the window until it has attended.  The window is copied
        in token order into the new ring, which starts at slot 0."""
        capacity = int(capacity)
        if capacity <= self.R:
            return
        k, v = self.residual()
        n = self.res_len
        k_res = torch.zeros(self.B, self.H, capacity, self.D, dtype=self.k_res.dtype,
                            device=self.device)
        v_res = torch.zeros_like(k_res)
        k_res[:, :, :n].copy_(k)
        v_res[:, :, :n].copy_(v)
        self.k_res, self.v_res = k_res, v_res
        self.res_start = 0
        self.R = capacity

    _TENSORS = ("k_res", "v_res", "k_codes", "k_scale", "k_zero", "v_codes", "v_scale",
                "v_zero", "k_hist", "v_hist")

    def allocated_bytes(self) -> int:
        """Device bytes the store's tensors hold (capacity, not contents)."""
        return sum(t.numel() * t.element_size()
                   for t in (getattr(self, n) for n in self._TENSORS) if t is not None)

    def select_batch(self, index: torch.Tensor) -> None:
        """Keep (and reorder or repeat) batch rows ``index`` of every tensor,
        e.g. to follow a beam-search reorder."""
        self._commit()
        for name in self._TENSORS:
            t = getattr(self, name)
            if t is not None:
                setattr(self, name, t.index_select(0, index))
        self.B = int(index.numel())

    # ---------------------------------------------------------- inspection
    def _codes(self, which: str, chunk: int) -> torch.Tensor:
        """One chunk's 2-bit codes, one byte per element, as [B, Hkv, G, D]."""
        return decode_codes(getattr(self, which)[:, :, chunk], self.G, self.D, self.code_layout,
                            which == "k_codes")

    def unpermuted_k_codes(self, chunk: int) -> torch.Tensor:
        """Key codes of one chunk as ``[B, Hkv, G, D/4]`` bytes: byte (t, i)
        holds channels 4i..4i+3 of token t, channel 4i+k at bits 2k."""
        return _pack_last(self._codes("k_codes", chunk))

    def unpermuted_v_codes(self, chunk: int) -> torch.Tensor:
        """Value codes of one chunk as ``[B, Hkv, D, G/4]`` bytes: byte (d, j)
        holds tokens 4j..4j+3 of channel d, token 4j+k at bits 2k."""
        return _pack_last(self._codes("v_codes", chunk).transpose(2, 3))

    def chunk_v_scale(self, chunk: int) -> torch.Tensor:
        """Value scales of one chunk as ``[B, Hkv, G, D/Gv]`` (token-major)."""
        return self.v_scale[:, :, chunk].transpose(2, 3)

    def chunk_v_zero(self, chunk: int) -> torch.Tensor:
        return self.v_zero[:, :, chunk].transpose(2, 3)

    # ------------------------------------------------------------ format
    def export_state(self) -> dict:
        """The store's contents as tensors in the reference's own layouts
        (those of ``quantize_keys`` / ``quantize_values`` over the whole
        quantised history, kv_cache_ops.cpp:179-199), on the store's device:

        * ``k_codes [B, Hkv, D, T/4]`` u8, ``k_scale``/``k_zero [B, Hkv, D, T/G]``
          -- keys per channel, groups of G along the T quantised tokens;
        * ``v_codes [B, Hkv, T, D/4]`` u8, ``v_scale``/``v_zero [B, Hkv, T, D/Gv]``
          -- values per token, groups of Gv channels;
        * ``k_residual``/``v_residual [B, Hkv, r, D]``, the residual window in
          token order, in the ring's element type (fp32 unless the store was
          built with a 16-bit ring).

        ``_C.dequantize_keys``/``dequantize_values`` (or the reference's
        own ops) turn the codes back into the served history."""
        B, H, D, G, n = self.B, self.H, self.D, self.G, self.n_chunks
        ng = D // self.Gv
        kc = decode_codes(self.k_codes[:, :, :n], G, D, self.code_layout, True)    # [B,H,n,G,D]
        vc = decode_codes(self.v_codes[:, :, :n], G, D, self.code_layout, False)
        kr, vr = self.residual()
        return {
            "k_codes": _pack_last(kc.permute(0, 1, 4, 2, 3).reshape(B, H, D, n * G)),
            "k_scale": self.k_scale[:, :, :n].permute(0, 1, 3, 2).contiguous(),
            "k_zero": self.k_zero[:, :, :n].permute(0, 1, 3, 2).contiguous(),
            "v_codes": _pack_last(vc.reshape(B, H, n * G, D)),
            "v_scale": self.v_scale[:, :, :n].permute(0, 1, 2, 4, 3).reshape(B, H, n * G, ng)
                           .contiguous(),
            "v_zero": self.v_zero[:, :, :n].permute(0, 1, 2, 4, 3).reshape(B, H, n * G, ng)
                          .contiguous(),
            "k_residual": kr.contiguous(),
            "v_residual": vr.contiguous(),
        }

    @classmethod
    def from_state(cls, state: dict, group_size: int, residual_capacity: int, device,
                   group_size_v: Optional[int] = None, chunk_capacity: int = 0) -> "PackedKVStore":
        """A store holding what :meth:`export_state` returned (tensors on any
        device); codes are re-ordered into this build's code layout and the
        ring takes the residuals' element type."""
        need = ("k_codes", "k_scale", "k_zero", "v_codes", "v_scale", "v_zero",
                "k_residual", "v_residual")
        missing = [k for k in need if k not in state]
        if missing:
            raise ValueError(f"packed-store state lacks {missing}")
        G = int(group_size)
        ks = state["k_scale"]
        if ks.dim() != 4:
            raise ValueError(f"k_scale must be [B, Hkv, D, T/G], got {tuple(ks.shape)}")
        B, H, D, n = ks.shape
        gv = G if group_size_v is None else int(group_size_v)
        T = n * G
        ng = D // gv if gv > 0 and D % gv == 0 else -1
        expect = {
            "k_codes": ((B, H, D, T // 4), torch.uint8), "k_zero": ((B, H, D, n), torch.float32),
            "k_scale": ((B, H, D, n), torch.float32), "v_codes": ((B, H, T, D // 4), torch.uint8),
            "v_scale": ((B, H, T, ng), torch.float32), "v_zero": ((B, H, T, ng), torch.float32),
        }
        for name, (shape, dtype) in expect.items():
            t = state[name]
            if tuple(t.shape) != shape or t.dtype != dtype:
                raise ValueError(f"{name} must be {dtype} {shape} for G={G}, Gv={gv}, got "
                                 f"{t.dtype} {tuple(t.shape)}")
        kr, vr = state["k_residual"], state["v_residual"]
        if kr.dim() != 4 or tuple(kr.shape[:2]) != (B, H) or kr.shape[3] != D or \
                kr.shape != vr.shape or kr.dtype not in _SRC_DTYPES or vr.dtype != kr.dtype:
            raise ValueError(f"residuals must be fp32, bf16 or fp16 [B={B}, Hkv={H}, r, D={D}] "
                             f"of one type, got {kr.dtype} {tuple(kr.shape)} and {vr.dtype} "
                             f"{tuple(vr.shape)}")
        if kr.shape[2] > residual_capacity:
            raise ValueError(f"residual of {kr.shape[2]} tokens exceeds capacity "
                             f"{residual_capacity}")
        st = cls(B, H, D, G, residual_capacity, device, group_size_v=gv,
                 chunk_capacity=max(n, int(chunk_capacity)), residual_dtype=kr.dtype)
        dev = st.device
        if n:
            kc = _unpack_last(state["k_codes"].to(dev)).reshape(B, H, D, n, G).permute(0, 1, 3, 4, 2)
            st.k_codes[:, :, :n] = encode_codes(kc, G, D, st.code_layout, True)
            st.k_scale[:, :, :n] = state["k_scale"].to(dev).permute(0, 1, 3, 2)
            st.k_zero[:, :, :n] = state["k_zero"].to(dev).permute(0, 1, 3, 2)
            vc = _unpack_last(state["v_codes"].to(dev)).reshape(B, H, n, G, D)
            st.v_codes[:, :, :n] = encode_codes(vc, G, D, st.code_layout, False)
            st.v_scale[:, :, :n] = state["v_scale"].to(dev).reshape(B, H, n, G, ng).permute(0, 1, 2, 4, 3)
            st.v_zero[:, :, :n] = state["v_zero"].to(dev).reshape(B, H, n, G, ng).permute(0, 1, 2, 4, 3)
        st.n_chunks = n
        if kr.shape[2]:
            st.append(kr.to(dev), vr.to(dev))
        return st

    # ------------------------------------------------------------ attention
    def workspace_bytes(self, q_heads: int, num_splits: int = 0) -> int:
        return int(_lib.kivi_packed_decode_attention_workspace_size(
            self.B, q_heads, self.H, self.D, self.G, self.Gv, self.n_chunks, self.res_len,
            num_splits))

    def attention(self, q: torch.Tensor, softmax_scale: Optional[float] = None,
                  out: Optional[torch.Tensor] = None, num_splits: int = 0,
                  workspace: Optional[torch.Tensor] = None, causal: bool = True,
                  kv_start=None, key_mask: Optional[torch.Tensor] = None,
                  hidden: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Fused attention over [packed history ; residual].

        ``q [B, Hq, D]`` (or ``[B, Hq, 1, D]``): one decode token per
        sequence; returns ``[B, Hq, D]`` fp32.  ``q [B, Hq, L, D]`` with
        L > 1: L query tokens per sequence (see ``_C.packed_attention``;
        ``causal`` by default: they are the window's last L tokens); returns
        ``[B, L, Hq, D]`` fp32.  ``kv_start``: per-sequence first visible
        position of a left-padded batch; ``key_mask`` ``[B, T]`` (nonzero =
        attended) or its packed ``hidden`` words: any other padding pattern
        (``_C.packed_attention``)."""
        masked = kv_start is not None or key_mask is not None or hidden is not None
        if masked and (q.dim() == 3 or q.shape[2] == 1):
            q4 = q if q.dim() == 4 else q.unsqueeze(2)
            o = _C.packed_attention(q4, self, causal=True, softmax_scale=softmax_scale,
                                    num_splits=num_splits, workspace=workspace,
                                    kv_start=kv_start, key_mask=key_mask, hidden=hidden)[:, 0]
            if out is not None:
                out.copy_(o.view_as(out))
                return out
            return o
        if q.dim() == 4 and q.shape[2] > 1:
            return _C.packed_attention(q, self, causal=causal, softmax_scale=softmax_scale,
                                       out=out, num_splits=num_splits, workspace=workspace,
                                       kv_start=kv_start, key_mask=key_mask, hidden=hidden)
        return _C.packed_decode_attention(q, self, softmax_scale=softmax_scale, out=out,
                                          num_splits=num_splits, workspace=workspace)
