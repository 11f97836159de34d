"""Shared helpers (mirror of scripts/common.py, the parts the answer path uses).

``choose_device`` and ``build_cache`` follow scripts/common.py:26-31, 70-76.
Model loading (``load_model``, :34-47) and WikiText chunks (:79-107) need a
network download and are not part of this build; ``load_model`` raises.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

DEFAULT_MODEL = "meta-llama/Llama-3.2-1B-Instruct"


@dataclass(frozen=True)
class KVConfig:
    """Cache geometry derived from the model configuration (scripts/common.py:13-23)."""

    layers: int
    kv_heads: int
    head_dim: int

    def fp16_bytes_per_token(self) -> int:
        return self.layers * self.kv_heads * self.head_dim * 2 * 2


def choose_device() -> torch.device:
    """The HIP kernels need a GPU; there is no CPU path for the compressed cache."""
    if torch.cuda.is_available():
        return torch.device("cuda")
    raise RuntimeError("dimmer-kv's compressed-cache path runs on an AMD GPU (no GPU visible)")


def load_model(model_id: str = DEFAULT_MODEL):
    raise RuntimeError(f"loading {model_id} needs a model download, which this build does not perform")


def kv_config(model) -> KVConfig:
    config = model.config
    head_dim = getattr(config, "head_dim", None) or (config.hidden_size // config.num_attention_heads)
    return KVConfig(layers=config.num_hidden_layers,
                    kv_heads=getattr(config, "num_key_value_heads", config.num_attention_heads), head_dim=head_dim)


def cache_tensors(cache):
    """Per-layer keys and values [batch, kv_heads, tokens, head_dim] of a DynamicCache (:62-67)."""
    layers = getattr(cache, "layers", None)
    if not layers:
        raise RuntimeError("The model did not return a DynamicCache with .layers.")
    return [layer.keys for layer in layers], [layer.values for layer in layers]


def build_cache(keys: list[torch.Tensor], values: list[torch.Tensor], model):
    """A fresh DynamicCache from per-layer tensors (scripts/common.py:70-76)."""
    from transformers import DynamicCache

    return DynamicCache(list(zip(keys, values)), config=model.config)
