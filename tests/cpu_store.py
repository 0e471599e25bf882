"""A CPU stand-in for ``PackedKVStore`` built on the oracle, so that the
control flow of ``KiviPackedCache`` (when tokens are appended, flushed and
attended) can be checked without a GPU.  Test infrastructure only: it holds
the residual window and the round-tripped history as CPU tensors, quantises
with the C oracle codec and attends with the float64 oracle attention."""

import numpy as np
import torch

from oracle import attention as oracle_attention
from oracle.kivi_cache import roundtrip


class CpuPackedStore:
    def __init__(self, batch, kv_heads, head_dim, group_size, residual_capacity, device,
                 group_size_v=None, chunk_capacity=0, keep_history=False,
                 residual_dtype=torch.float32):
        self.B, self.H, self.D = batch, kv_heads, head_dim
        # values are held widened to fp32 after rounding to the ring's type
        self.residual_dtype = residual_dtype
        self.G = group_size
        self.Gv = group_size if group_size_v is None else group_size_v
        self.R = residual_capacity
        self.device = torch.device("cpu")
        self.reset()

    def reset(self):
        self.res_k = torch.zeros(self.B, self.H, 0, self.D)
        self.res_v = torch.zeros_like(self.res_k)
        self.hist_k = torch.zeros(self.B, self.H, 0, self.D)
        self.hist_v = torch.zeros_like(self.hist_k)
        self.n_chunks = 0

    @property
    def res_len(self):
        return self.res_k.shape[2]

    @property
    def quantized_tokens(self):
        return self.n_chunks * self.G

    def append(self, k, v):
        n = k.shape[2]
        if self.res_len + n > self.R:
            raise RuntimeError(f"residual window overflow ({self.res_len} + {n} > {self.R})")
        rd = self.residual_dtype
        self.res_k = torch.cat([self.res_k, k.cpu().to(rd).float()], dim=2)
        self.res_v = torch.cat([self.res_v, v.cpu().to(rd).float()], dim=2)

    def stage_token(self, k, v):
        self.append(k, v)

    def flush(self):
        G = self.G
        if self.res_len < G:
            raise RuntimeError(f"Cannot flush {G} tokens: residual only has {self.res_len}")
        ck = self.res_k[:, :, :G]
        cv = self.res_v[:, :, :G]
        k_hat = roundtrip(ck.transpose(2, 3).contiguous(), G).transpose(2, 3)
        v_hat = roundtrip(cv.contiguous(), self.Gv)
        self.hist_k = torch.cat([self.hist_k, k_hat], dim=2)
        self.hist_v = torch.cat([self.hist_v, v_hat], dim=2)
        self.res_k, self.res_v = self.res_k[:, :, G:], self.res_v[:, :, G:]
        self.n_chunks += 1

    def extend(self, k, v, flush_at=None):
        R = self.R if flush_at is None else flush_at
        n, t, flushes = k.shape[2], 0, 0
        while t < n:
            take = min(n - t, R - self.res_len)
            self.append(k[:, :, t:t + take], v[:, :, t:t + take])
            t += take
            while self.res_len >= R:
                self.flush()
                flushes += 1
        return flushes

    def attention(self, q, softmax_scale=None, causal=True, kv_start=None, hidden=None):
        starts = None if kv_start is None else [int(x) for x in kv_start]
        vis = None
        if hidden is not None:
            # hidden-position words -> visibility: bit p % 32 of word p // 32
            T = self.n_chunks * self.G + self.res_len
            w = hidden.cpu().numpy().astype(np.uint32)
            p = np.arange(T)
            vis = ((w[:, p // 32] >> (p % 32).astype(np.uint32)) & 1) == 0
        if q.dim() == 4 and q.shape[2] > 1:
            # [B, Hq, L, D] -> [B, L, Hq, D]: the window's newest L tokens
            assert causal and q.shape[2] <= self.res_len
            o = oracle_attention.prefix_attention(q.transpose(1, 2).numpy(), self.hist_k.numpy(),
                                                  self.hist_v.numpy(), self.res_k.numpy(),
                                                  self.res_v.numpy(), softmax_scale, starts, vis)
            return torch.from_numpy(o).float()
        if q.dim() == 4:                      # [B, Hq, 1, D]: one token, as [B, Hq, D]
            q = q[:, :, 0]
        o = oracle_attention.decode_attention(q.numpy(), self.hist_k.numpy(),
                                              self.hist_v.numpy(), self.res_k.numpy(),
                                              self.res_v.numpy(), softmax_scale, starts, vis)
        return torch.from_numpy(o).float()

    def grow_residual(self, capacity):
        self.R = max(self.R, int(capacity))

    def rollback(self, n):
        if n < 0 or n > self.res_len:
            raise ValueError(f"cannot roll back {n} tokens: the residual window holds "
                             f"{self.res_len} (quantised tokens cannot be rolled back)")
        m = self.res_len - n
        self.res_k, self.res_v = self.res_k[:, :, :m], self.res_v[:, :, :m]

    def select_batch(self, index):
        for name in ("res_k", "res_v", "hist_k", "hist_v"):
            setattr(self, name, getattr(self, name).index_select(0, index.cpu()))
        self.B = int(index.numel())

    def allocated_bytes(self):
        return sum(t.numel() * 4 for t in (self.res_k, self.res_v, self.hist_k, self.hist_v))
