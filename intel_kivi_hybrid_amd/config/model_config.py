"""KV-cache shape detection from a HuggingFace model config.

Same attribute search order and error messages as the reference
(src/kivi_sycl/config/model_config.py:6-59), so ``KiviCache.from_model``
configures itself identically for every model family the reference supports.
"""

__all__ = ["detect_model_config"]

_LAYER_ATTRS = ("n_layer", "num_hidden_layers", "num_layers", "n_layers")
_KV_HEAD_ATTRS = ("num_key_value_heads", "num_kv_heads")
_HEAD_ATTRS = ("n_head", "num_attention_heads", "num_heads")


def _first_attr(config, names):
    for name in names:
        if hasattr(config, name):
            return True, getattr(config, name)
    return False, None


def detect_model_config(model) -> dict:
    """Return ``{"num_layers", "num_kv_heads", "head_dim"}`` for ``model``.

    * layers: first of n_layer / num_hidden_layers / num_layers / n_layers;
    * kv heads: num_key_value_heads / num_kv_heads (GQA), else the query-head
      count n_head / num_attention_heads / num_heads;
    * head_dim: ``config.head_dim`` if present, else hidden_size (or n_embd)
      divided by the query-head count.
    """
    config = model.config
    name = type(config).__name__

    found, num_layers = _first_attr(config, _LAYER_ATTRS)
    if not found:
        raise ValueError(f"Cannot detect num_layers from {name}. Pass num_layers= explicitly.")

    num_kv_heads = None
    for group in (_KV_HEAD_ATTRS, _HEAD_ATTRS):
        found, value = _first_attr(config, group)
        if found and value is not None:
            num_kv_heads = value
            break
    if num_kv_heads is None:
        raise ValueError(f"Cannot detect num_heads from {name}. Pass num_kv_heads= explicitly.")

    if hasattr(config, "head_dim"):
        head_dim = config.head_dim
    else:
        hidden = getattr(config, "hidden_size", getattr(config, "n_embd", None))
        q_heads = getattr(config, "num_attention_heads", getattr(config, "n_head", None))
        if not (hidden and q_heads):
            raise ValueError(f"Cannot detect head_dim from {name}. Pass head_dim= explicitly.")
        head_dim = hidden // q_heads

    return {"num_layers": num_layers, "num_kv_heads": num_kv_heads, "head_dim": head_dim}
