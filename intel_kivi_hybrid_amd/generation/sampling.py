"""Next-token selection for the ``generate()`` loop
(src/kivi_sycl/generation/sampling.py:10-25 in the reference)."""

from typing import Optional

import torch

__all__ = ["sample_token"]


def sample_token(logits: torch.Tensor, temperature: float, top_k: Optional[int],
                 do_sample: bool) -> torch.Tensor:
    """``logits [B, V]`` -> next ids ``[B, 1]``.

    Greedy (``do_sample=False``) is the argmax.  Sampling divides by
    ``max(temperature, 1e-8)``, masks everything below the k-th largest logit
    to -inf when ``top_k`` is set, and draws from the softmax."""
    if not do_sample:
        return logits.argmax(dim=-1).unsqueeze(1)
    scaled = logits / max(temperature, 1e-8)
    if top_k is not None:
        kth = scaled.topk(top_k, dim=-1).values[:, -1:]
        scaled = scaled.masked_fill(scaled < kth, float("-inf"))
    return torch.multinomial(torch.softmax(scaled, dim=-1), num_samples=1)
