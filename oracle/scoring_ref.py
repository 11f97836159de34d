"""Question-time scoring of the hot tier and top-k selection, restated in numpy
(oracle; test infrastructure only).

Follows:
- scripts/progressive.py:239-254 ``question_importance``: the attention every
  context token receives from the question, summed over layers and heads;
- scripts/dimmer.py:52-66: per layer, scores = q.k * scaling + causal mask,
  fp32 softmax over *all* keys (context + the question's own tokens), summed
  over query positions and over the query heads of each KV head;
- scripts/methods.py:244-248: count = max(1, round(fraction * middle)) (Python
  round, half to even) and ``topk`` over the middle tokens.

The softmax here is exact fp32 per row in numpy order.  torch's fp32 sum
order can differ in the last bit, so index sets are compared with the score
margin between the count-th and (count+1)-th value recorded; at a near-tie
the set is parity unpinned.

Pins (tests/test_oracle_kvtc_scoring_packing.py): per-layer probabilities
against a float64 brute force over every key, the selection count against
Python's rounding, the index set against torch.topk on distinct scores.
"""

from __future__ import annotations

import numpy as np

from .attention_ref import layer_keys


def layer_probabilities(query, keys_c, key_exact, key_question, scaling):
    """query [Hq, q_len, d]; keys_c [Hkv, n, d]; key_exact [Hkv, T_e, d]; key_question [Hkv, q_len, d].
    Returns fp32 probabilities over the compressed keys only, summed per KV head: [Hkv, n]."""
    q_heads, q_len, dim = query.shape
    heads = keys_c.shape[0]
    groups = q_heads // heads
    q = query.astype(np.float32).reshape(heads, groups, q_len, dim)
    s_c = np.einsum("hgqd,hnd->hgqn", q, keys_c.astype(np.float32)) * np.float32(scaling)
    s_e = np.einsum("hgqd,hnd->hgqn", q, key_exact.astype(np.float32)) * np.float32(scaling)
    s_q = np.einsum("hgqd,hnd->hgqn", q, key_question.astype(np.float32)) * np.float32(scaling)
    causal = np.triu(np.full((q_len, q_len), -np.inf, dtype=np.float32), k=1)
    s_q = s_q + causal
    s = np.concatenate([s_c, s_e, s_q], axis=-1)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    p = e / e.sum(axis=-1, keepdims=True)
    n = keys_c.shape[1]
    return p[..., :n].sum(axis=2).sum(axis=1)  # over query positions, then GQA group


def importance(queries, coef_k_hot, basis_k, mean_k, cos, sin, key_exact, key_question, heads, scaling=None):
    """Sum over layers of ``layer_probabilities`` -> f32 [n] over the compressed (middle) tokens.

    queries [L, Hq, q_len, d]; basis_k [r, L, Hkv*d]; mean_k [L, Hkv*d];
    key_exact [L, Hkv, T_e, d]; key_question [L, Hkv, q_len, d]."""
    layers, q_heads, q_len, dim = queries.shape
    scaling = dim ** -0.5 if scaling is None else scaling
    total = np.zeros(coef_k_hot.shape[0], dtype=np.float32)
    for layer in range(layers):
        keys = layer_keys(coef_k_hot, basis_k[:, layer], mean_k[layer], cos, sin, heads)
        total += layer_probabilities(queries[layer], keys, key_exact[layer], key_question[layer],
                                     scaling).sum(axis=0).astype(np.float32)
    return total


def select_count(fraction: float, middle: int) -> int:
    """methods.py:246."""
    return max(1, int(round(fraction * middle)))


def topk_indices(scores: np.ndarray, count: int) -> np.ndarray:
    """Indices of the ``count`` largest values; ties by lower index (torch.topk leaves tie order unspecified)."""
    order = np.argsort(-scores.astype(np.float64), kind="stable")
    return np.sort(order[:count])


def topk_margin(scores: np.ndarray, count: int) -> float:
    """Gap between the count-th and (count+1)-th largest values (0 when count == len)."""
    if count >= scores.size:
        return float("inf")
    s = np.sort(scores.astype(np.float64))[::-1]
    return float(s[count - 1] - s[count])
