"""RoPE restated in numpy (oracle; test infrastructure only).

Follows:
- transformers/modeling_rope_utils.py:621-662 (``_compute_llama3_parameters``),
  which Llama-3.2 uses through ``LlamaRotaryEmbedding`` (modeling_llama.py:64-126);
- scripts/kvtc.py:27-29 (``rotate_half``), :32-37 (``rope_tables``), :46-47 (``rerotate``).

Pinned by tests/test_oracle_rope_attention.py against transformers' own
``LlamaRotaryEmbedding`` (a library routine present in this container) and
by the closed-form identities cos^2 + sin^2 = 1 and rerotate o derotate = id.
numpy's float32 ``power`` can differ from torch's by one ulp in an inverse
frequency, so the tables agree with transformers' to within that ulp times the
position (checked), not bit for bit.  The product path and the parity tests
take their cos/sin tables from transformers itself, as the reference does.
"""

from __future__ import annotations

import math

import numpy as np

LLAMA32_ROPE = {"rope_theta": 500000.0, "factor": 32.0, "low_freq_factor": 1.0,
                "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}


def llama3_inv_freq(head_dim: int, theta: float = 500000.0, factor: float = 32.0, low_freq_factor: float = 1.0,
                    high_freq_factor: float = 4.0, original_max: int = 8192) -> np.ndarray:
    """float32 inverse frequencies [head_dim // 2] (modeling_rope_utils.py:641-662)."""
    exponent = (np.arange(0, head_dim, 2, dtype=np.int64).astype(np.float32) / np.float32(head_dim)).astype(np.float32)
    inv_freq = (np.float32(1.0) / np.power(np.float32(theta), exponent, dtype=np.float32)).astype(np.float32)
    low_freq_wavelen = original_max / low_freq_factor
    high_freq_wavelen = original_max / high_freq_factor
    wavelen = (np.float32(2 * math.pi) / inv_freq).astype(np.float32)
    inv_llama = np.where(wavelen > low_freq_wavelen, inv_freq / np.float32(factor), inv_freq).astype(np.float32)
    smooth = ((np.float32(original_max) / wavelen - np.float32(low_freq_factor))
              / np.float32(high_freq_factor - low_freq_factor)).astype(np.float32)
    smoothed = ((np.float32(1) - smooth) * inv_llama / np.float32(factor) + smooth * inv_llama).astype(np.float32)
    medium = ~(wavelen < high_freq_wavelen) & ~(wavelen > low_freq_wavelen)
    return np.where(medium, smoothed, inv_llama).astype(np.float32)


def default_inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """Plain RoPE inverse frequencies (modeling_llama.py:80-94)."""
    exponent = (np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)).astype(np.float32)
    return (np.float32(1.0) / np.power(np.float32(theta), exponent, dtype=np.float32)).astype(np.float32)


def rope_tables(positions: np.ndarray, inv_freq: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """cos, sin float32 [n, head_dim] (modeling_llama.py:113-126: freqs = inv_freq x pos in fp32,
    emb = cat(freqs, freqs), attention_scaling = 1.0 for llama3)."""
    freqs = (positions.astype(np.float32)[:, None] * inv_freq[None, :]).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def rotate_half(x: np.ndarray) -> np.ndarray:
    """scripts/kvtc.py:27-29: half-split rotation cat(-x2, x1)."""
    half = x.shape[-1] // 2
    return np.concatenate([-x[..., half:], x[..., :half]], axis=-1)


def rerotate(keys: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """scripts/kvtc.py:46-47."""
    return keys * cos + rotate_half(keys) * sin


def derotate(keys: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """scripts/kvtc.py:40-43 (inverse rotation, divided by cos^2 + sin^2)."""
    return (keys * cos - rotate_half(keys) * sin) / (cos * cos + sin * sin)
