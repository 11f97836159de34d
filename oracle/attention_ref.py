"""Attention directly over compressed coefficients, restated in numpy
(oracle; test infrastructure only).

``attend`` follows scripts/compressed_attention.py:105-137 operation by
operation, in float32 (the reference's ``dtype=torch.float32`` context):

- keys of layer l: ``coef_k @ basis_k[:, l]`` + mean_k[l], viewed [n, Hkv, d],
  transposed to [Hkv, n, d], re-RoPE'd at the tokens' positions (:105-111);
- GQA view q[B, Hkv, g, q_len, d] (q head = h*g + j, :119);
- one fp32 softmax over [compressed | exact] scores, the exact part with the
  additive mask (:120-128);
- values in coefficient space: sum(p_c) * mean_v + (p_c @ coef_v) @ basis_v
  (:130-134), plus p_e @ V_exact (:135);
- output [B, q_len, Hq, d] (:136-137).

``decode_then_attend_f64`` is the independent pin: it decodes every key and
value in full (``inverse_transform``, scripts/kvtc.py:88-97) and runs textbook
softmax attention in float64 with repeat_kv GQA
(transformers/models/llama/modeling_llama.py:179-188).  The equality of the two
(scripts/compressed_attention.py:15-19) is checked in tests/test_oracle_rope_attention.py.
"""

from __future__ import annotations

import numpy as np

from .rope_ref import rerotate


def layer_keys(coef_k: np.ndarray, basis_k_layer: np.ndarray, mean_k_layer: np.ndarray,
               cos: np.ndarray, sin: np.ndarray, heads: int, dtype=np.float32) -> np.ndarray:
    """compressed_attention.py:105-111 -> [Hkv, n, d]."""
    n = coef_k.shape[0]
    flat = coef_k.astype(dtype) @ basis_k_layer.astype(dtype) + mean_k_layer.astype(dtype)
    heads_first = flat.reshape(n, heads, flat.shape[1] // heads).transpose(1, 0, 2)
    return rerotate(heads_first, cos.astype(dtype), sin.astype(dtype)).astype(dtype)


def _softmax(x: np.ndarray) -> np.ndarray:
    m = x.max(axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=-1, keepdims=True)


def attend(query, coef_k, coef_v, basis_k_layer, basis_v_layer, mean_k_layer, mean_v_layer, cos, sin,
           key_exact=None, value_exact=None, mask=None, scaling=None, dtype=np.float32):
    """One layer of compressed attention (compressed_attention.py:113-137).

    query [B, Hq, q_len, d]; coef_* [n, r]; basis_*_layer [r, Hkv*d]; mean_*_layer [Hkv*d];
    cos/sin [n, d]; key/value_exact [B, Hkv, T_e, d] or None; mask [B, 1, q_len, T_e] or None.
    Returns [B, q_len, Hq, d]."""
    batch, q_heads, q_len, dim = query.shape
    heads = mean_k_layer.shape[0] // dim
    groups = q_heads // heads
    scaling = dim ** -0.5 if scaling is None else scaling
    q = query.astype(dtype).reshape(batch, heads, groups, q_len, dim)
    keys = layer_keys(coef_k, basis_k_layer, mean_k_layer, cos, sin, heads, dtype)
    scores_c = np.einsum("bhgqd,hnd->bhgqn", q, keys).astype(dtype) * dtype(scaling)
    parts = [scores_c]
    if key_exact is not None and key_exact.shape[2] > 0:
        scores_e = np.einsum("bhgqd,bhnd->bhgqn", q, key_exact.astype(dtype)).astype(dtype) * dtype(scaling)
        if mask is not None:
            scores_e = scores_e + mask.astype(dtype)[:, :, None]
        parts.append(scores_e)
    middle = scores_c.shape[-1]
    probabilities = _softmax(np.concatenate(parts, axis=-1).astype(np.float32)).astype(dtype)
    p_c, p_e = probabilities[..., :middle], probabilities[..., middle:]
    out = p_c.sum(axis=-1, keepdims=True) * mean_v_layer.astype(dtype).reshape(1, heads, 1, 1, dim)
    if middle > 0:  # no einsum over an empty token axis: its result is not reliably zero-filled
        weighted = np.einsum("bhgqn,nr->bhgqr", p_c, coef_v.astype(dtype))
        layer_basis = basis_v_layer.astype(dtype).reshape(-1, heads, dim)
        out = out + np.einsum("bhgqr,rhd->bhgqd", weighted, layer_basis)
    if p_e.shape[-1] > 0:
        out = out + np.einsum("bhgqn,bhnd->bhgqd", p_e, value_exact.astype(dtype))
    return out.reshape(batch, q_heads, q_len, dim).transpose(0, 2, 1, 3).astype(dtype)


def decode_then_attend_f64(query, coef_k, coef_v, basis_k_layer, basis_v_layer, mean_k_layer, mean_v_layer,
                           cos, sin, key_exact=None, value_exact=None, mask=None, scaling=None):
    """Textbook attention (float64) over the fully decoded keys and values."""
    batch, q_heads, q_len, dim = query.shape
    heads = mean_k_layer.shape[0] // dim
    groups = q_heads // heads
    scaling = dim ** -0.5 if scaling is None else scaling
    n = coef_k.shape[0]
    k = (coef_k.astype(np.float64) @ basis_k_layer.astype(np.float64) + mean_k_layer).reshape(n, heads, dim)
    k = rerotate(k.transpose(1, 0, 2), cos.astype(np.float64), sin.astype(np.float64))  # [Hkv, n, d]
    v = (coef_v.astype(np.float64) @ basis_v_layer.astype(np.float64) + mean_v_layer).reshape(n, heads, dim)
    v = v.transpose(1, 0, 2)
    k = np.broadcast_to(k[None], (batch, heads, n, dim))
    v = np.broadcast_to(v[None], (batch, heads, n, dim))
    m = None
    if key_exact is not None and key_exact.shape[2] > 0:
        k = np.concatenate([k, key_exact.astype(np.float64)], axis=2)
        v = np.concatenate([v, value_exact.astype(np.float64)], axis=2)
        if mask is not None:
            m = np.concatenate([np.zeros(mask.shape[:-1] + (n,)), mask.astype(np.float64)], axis=-1)
    k = np.repeat(k, groups, axis=1)  # repeat_kv: q head h*g + j uses kv head h
    v = np.repeat(v, groups, axis=1)
    s = np.einsum("bhqd,bhnd->bhqn", query.astype(np.float64), k) * scaling
    if m is not None:
        s = s + m
    p = _softmax(s)
    out = np.einsum("bhqn,bhnd->bhqd", p, v)
    return out.transpose(0, 2, 1, 3)
