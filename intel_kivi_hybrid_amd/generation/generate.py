"""One-call text generation through a :class:`KiviCache`.

Same signature, control flow and stopping rule as the reference's
``generate`` (src/kivi_sycl/generation/generate.py:13-89): prefill, then
``max_new_tokens - 1`` decode steps that feed the model the cache served by
``KiviCache.get_full_cache()``, with the EOS check at the top of each step.
The only change is where things live: the cache keeps its state in HBM on the
HIP device, and the model may sit on the CPU (as in the reference) or on the
GPU -- the prompt ids are placed on the model's device.
"""

from typing import Optional

import torch

from ..cache.manager import KiviCache
from ..cache.packed_cache import KiviPackedCache, packed_attention
from .sampling import sample_token

__all__ = ["generate", "generate_packed"]


def _model_device(model) -> torch.device:
    dev = getattr(model, "device", None)
    if isinstance(dev, torch.device):
        return dev
    for p in model.parameters():
        return p.device
    return torch.device("cpu")


@torch.no_grad()
def generate(model, tokenizer, prompt: str, max_new_tokens: int = 200, group_size: int = 32,
             residual_length: int = 128, device: str = "cuda", temperature: float = 1.0,
             top_k: Optional[int] = None, do_sample: bool = False,
             verbose: bool = False) -> str:
    """Generate ``max_new_tokens`` tokens after ``prompt`` with the KIVI 2-bit
    KV cache and return prompt + completion as text.

    ``device`` is where the cache's packed store and residual window live (the
    HIP device; the reference's ``"xpu"`` is accepted as an alias)."""
    cache = KiviCache.from_model(model, device=device, group_size=group_size,
                                 residual_length=residual_length)
    input_ids = tokenizer(prompt, return_tensors="pt").input_ids.to(_model_device(model))

    out = model(input_ids, use_cache=True)
    cache.add_tokens(out.past_key_values)
    next_id = sample_token(out.logits[:, -1, :], temperature, top_k, do_sample)
    generated = [next_id]
    eos_id = tokenizer.eos_token_id

    for step in range(1, max_new_tokens):
        if eos_id is not None and next_id.item() == eos_id:
            break
        out = model(next_id, past_key_values=cache.get_full_cache(), use_cache=True)
        cache.add_tokens(out.past_key_values)
        next_id = sample_token(out.logits[:, -1, :], temperature, top_k, do_sample)
        generated.append(next_id)
        if verbose and (step + 1) % 10 == 0:
            print(".", end="", flush=True)
    if verbose:
        print()

    full_ids = torch.cat([input_ids, torch.cat(generated, dim=1)], dim=1)
    return tokenizer.decode(full_ids[0], skip_special_tokens=True)


@torch.no_grad()
def generate_packed(model, tokenizer, prompt: str, max_new_tokens: int = 200,
                    group_size: int = 32, residual_length: int = 128, device: str = "cuda",
                    temperature: float = 1.0, top_k: Optional[int] = None,
                    do_sample: bool = False, verbose: bool = False) -> str:
    """:func:`generate` with the model attending straight from the 2-bit store.

    Same arguments, token selection and stopping rule as the reference's
    ``generate`` (generate.py:13-89), and the same cache semantics: the
    prompt pass attends over its own fp32 K/V, every decode step attends over
    [dequantised history ; fp32 residual ; new token], and the G oldest
    residual tokens are quantised after a step leaves R or more.  The cache is
    a :class:`KiviPackedCache` that the model updates itself, and the decode
    attention is the fused packed-KV kernel (attention implementation
    ``"kivi_packed"``, set for the duration of the call), so no fp32 copy of
    the history is ever built."""
    cache = KiviPackedCache.from_model(model, device=device, group_size=group_size,
                                       residual_length=residual_length)
    input_ids = tokenizer(prompt, return_tensors="pt").input_ids.to(_model_device(model))
    eos_id = tokenizer.eos_token_id

    with packed_attention(model):
        out = model(input_ids, past_key_values=cache, use_cache=True)
        next_id = sample_token(out.logits[:, -1, :], temperature, top_k, do_sample)
        generated = [next_id]
        for step in range(1, max_new_tokens):
            if eos_id is not None and next_id.item() == eos_id:
                break
            out = model(next_id, past_key_values=cache, use_cache=True)
            next_id = sample_token(out.logits[:, -1, :], temperature, top_k, do_sample)
            generated.append(next_id)
            if verbose and (step + 1) % 10 == 0:
                print(".", end="", flush=True)
    if verbose:
        print()

    full_ids = torch.cat([input_ids, torch.cat(generated, dim=1)], dim=1)
    return tokenizer.decode(full_ids[0], skip_special_tokens=True)
