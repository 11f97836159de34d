"""Cache helpers the answer path shares (the part of scripts/common.py it uses).

``build_cache`` keeps the reference's one-line construction (scripts/common.py:70-76): the exact
tail that HF's attention layers update is an ordinary ``DynamicCache``.  Model loading and the
WikiText reader of that file need downloads and are not part of this build.
"""

from __future__ import annotations

import torch


def choose_device() -> torch.device:
    """The compressed cache lives on an AMD GPU; with none visible there is nothing to run on."""
    if not torch.cuda.is_available():
        raise RuntimeError("dimmer-kv's compressed-cache path runs on an AMD GPU (no GPU visible)")
    return torch.device("cuda")


def cache_tensors(cache) -> tuple[list[torch.Tensor], list[torch.Tensor]]:
    """(keys, values): the per-layer [batch, kv_heads, tokens, head_dim] tensors a DynamicCache holds."""
    per_layer = list(getattr(cache, "layers", None) or [])
    if not per_layer:
        raise RuntimeError("expected a DynamicCache with per-layer entries (cache.layers)")
    return [entry.keys for entry in per_layer], [entry.values for entry in per_layer]


def build_cache(keys: list[torch.Tensor], values: list[torch.Tensor], model):
    """A fresh DynamicCache from per-layer tensors (scripts/common.py:70-76)."""
    from transformers import DynamicCache

    return DynamicCache(list(zip(keys, values)), config=model.config)
