"""Pins of oracle/rope_ref.py and oracle/attention_ref.py (CPU).

RoPE: the oracle's llama3 inverse frequencies and cos/sin tables against
transformers' own LlamaRotaryEmbedding (the routine the reference calls through
``model.model.rotary_emb``), plus the rotation identities.

Attention: ``attend`` (the reference's fp32 operation order over coefficients)
against ``decode_then_attend_f64`` (full decode + textbook softmax attention),
that one against torch's scaled_dot_product_attention in float64, and the
closed-form special cases: all tokens at zero planes give the value mean, a
zero query gives the plain average, one token gives its own value, token
permutation leaves the output unchanged, and a log-sum-exp merge of two token
sets equals one pass.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import synth
from oracle import attention_ref as ar
from oracle import rope_ref


@pytest.mark.parametrize("head_dim", [64, 128])
def test_llama3_inv_freq_matches_transformers(head_dim):
    shape = synth.ModelShape(2, 2, head_dim, 4, 256)
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    emb = LlamaRotaryEmbedding(synth.llama_config(shape))
    ours = rope_ref.llama3_inv_freq(head_dim)
    theirs = emb.inv_freq.float().numpy()
    np.testing.assert_allclose(ours, theirs, rtol=2e-7, atol=0)


@pytest.mark.parametrize("head_dim", [64, 128])
def test_rope_tables_match_transformers(head_dim):
    shape = synth.ModelShape(2, 2, head_dim, 4, 256)
    positions = np.array([0, 1, 2, 17, 255, 4096, 8191, 8192, 16383, 20000])
    cos_t, sin_t = synth.rope_tables(shape, 20001, "cpu")
    inv = rope_ref.llama3_inv_freq(head_dim)
    cos_o, sin_o = rope_ref.rope_tables(positions, inv)
    # float32 pow may differ from torch's by one ulp of an inverse frequency; at position p that
    # moves the angle by up to p * inv_freq * 2^-23 (plus the rounding of the angle itself)
    inv2 = np.concatenate([inv, inv]).astype(np.float64)
    tol = positions[:, None] * inv2[None, :] * 2.0 ** -22 + 2e-6
    assert (np.abs(cos_o - cos_t[positions].numpy()) <= tol).all()
    assert (np.abs(sin_o - sin_t[positions].numpy()) <= tol).all()
    # the two halves of HF's emb are equal, which the kernels' half tables rely on
    half = head_dim // 2
    assert np.array_equal(cos_t[:, :half].numpy(), cos_t[:, half:].numpy())


def test_rotation_identities():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 7, 64)).astype(np.float64)
    cos, sin = rope_ref.rope_tables(np.arange(7), rope_ref.llama3_inv_freq(64))
    cos, sin = cos.astype(np.float64), sin.astype(np.float64)
    np.testing.assert_allclose(rope_ref.rotate_half(rope_ref.rotate_half(x)), -x)
    np.testing.assert_allclose(rope_ref.derotate(rope_ref.rerotate(x, cos, sin), cos, sin), x, atol=1e-12)
    # a rotation keeps the norm of every (d, d + D/2) pair
    y = rope_ref.rerotate(x, cos, sin)
    np.testing.assert_allclose(x[..., :32] ** 2 + x[..., 32:] ** 2, y[..., :32] ** 2 + y[..., 32:] ** 2, atol=1e-12)
    # rotate_half is the half-split (NeoX/Llama) form, not interleaved
    v = np.arange(8.0)
    assert rope_ref.rotate_half(v).tolist() == [-4.0, -5.0, -6.0, -7.0, 0.0, 1.0, 2.0, 3.0]


def _problem(seed, n=37, heads=2, dim=16, q_heads=6, rank=64, q_len=2, exact=5, scale=1.0):
    rng = np.random.default_rng(seed)
    F = heads * dim
    basis_k = np.linalg.qr(rng.standard_normal((F, rank)))[0].T.astype(np.float32) if rank <= F else \
        rng.standard_normal((rank, F)).astype(np.float32) / np.sqrt(rank)
    basis_v = rng.standard_normal((rank, F)).astype(np.float32) / np.sqrt(rank)
    coef_k = (rng.standard_normal((n, rank)) * scale).astype(np.float32)
    coef_v = rng.standard_normal((n, rank)).astype(np.float32)
    mean_k = (rng.standard_normal(F) * 0.1).astype(np.float32)
    mean_v = (rng.standard_normal(F) * 0.1).astype(np.float32)
    cos, sin = rope_ref.rope_tables(rng.permutation(1000)[:n], rope_ref.default_inv_freq(dim, 10000.0))
    q = rng.standard_normal((1, q_heads, q_len, dim)).astype(np.float32)
    ke = rng.standard_normal((1, heads, exact, dim)).astype(np.float32)
    ve = rng.standard_normal((1, heads, exact, dim)).astype(np.float32)
    mask = np.zeros((1, 1, q_len, exact), dtype=np.float32)
    mask[0, 0, 0, -1] = -np.inf  # causal: the first query does not see the last exact token
    return dict(query=q, coef_k=coef_k, coef_v=coef_v, basis_k_layer=basis_k, basis_v_layer=basis_v,
                mean_k_layer=mean_k, mean_v_layer=mean_v, cos=cos, sin=sin, key_exact=ke, value_exact=ve, mask=mask)


def test_attend_fp32_matches_f64_decode_then_attend():
    for seed in range(4):
        p = _problem(seed)
        got = ar.attend(**p)
        ref = ar.decode_then_attend_f64(**p)
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)


def test_decode_then_attend_matches_torch_sdpa_f64():
    p = _problem(7)
    n, dim = p["coef_k"].shape[0], p["query"].shape[-1]
    heads = p["mean_k_layer"].shape[0] // dim
    k = (p["coef_k"].astype(np.float64) @ p["basis_k_layer"] + p["mean_k_layer"]).reshape(n, heads, dim).transpose(1, 0, 2)
    k = rope_ref.rerotate(k, p["cos"].astype(np.float64), p["sin"].astype(np.float64))
    v = (p["coef_v"].astype(np.float64) @ p["basis_v_layer"] + p["mean_v_layer"]).reshape(n, heads, dim).transpose(1, 0, 2)
    K = torch.from_numpy(np.concatenate([k[None], p["key_exact"].astype(np.float64)], 2))
    V = torch.from_numpy(np.concatenate([v[None], p["value_exact"].astype(np.float64)], 2))
    groups = p["query"].shape[1] // heads
    K, V = K.repeat_interleave(groups, 1), V.repeat_interleave(groups, 1)
    m = np.concatenate([np.zeros((1, 1, p["query"].shape[2], n)), p["mask"].astype(np.float64)], -1)
    out = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(p["query"].astype(np.float64)), K, V,
                                                           attn_mask=torch.from_numpy(m))
    ref = out.transpose(1, 2).numpy()
    np.testing.assert_allclose(ar.decode_then_attend_f64(**p), ref, rtol=1e-10, atol=1e-12)


def test_zero_planes_give_value_mean():
    p = _problem(3)
    p["coef_k"][:] = 0
    p["coef_v"][:] = 0
    p["key_exact"] = p["value_exact"] = p["mask"] = None
    got = ar.attend(**p)
    heads, dim = 2, 16
    want = np.broadcast_to(p["mean_v_layer"].reshape(heads, 1, dim).repeat(3, 0).reshape(1, 1, 6, dim), got.shape)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)


def test_zero_query_gives_plain_average():
    p = _problem(4)
    p["query"][:] = 0
    p["mask"] = None
    got = ar.attend(**p)
    heads, dim = 2, 16
    v = (p["coef_v"] @ p["basis_v_layer"] + p["mean_v_layer"]).reshape(-1, heads, dim)
    allv = np.concatenate([v.transpose(1, 0, 2), p["value_exact"][0]], 1)  # [heads, n + E, d]
    want = allv.mean(1)  # [heads, d]
    for qh in range(6):
        np.testing.assert_allclose(got[0, :, qh], np.broadcast_to(want[qh // 3], (2, dim)), rtol=1e-5, atol=1e-6)


def test_no_compressed_tokens_is_plain_attention_over_the_exact_tokens():
    """A conversation shorter than sinks + recent has no compressed token: the output is textbook
    softmax attention over the exact tokens (torch's SDPA in float64, GQA by repeating KV heads)."""
    p = _problem(6, n=0)
    got = ar.attend(**p)
    assert np.isfinite(got).all()
    K = torch.from_numpy(np.repeat(p["key_exact"].astype(np.float64), 3, axis=1))
    V = torch.from_numpy(np.repeat(p["value_exact"].astype(np.float64), 3, axis=1))
    out = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(p["query"].astype(np.float64)), K, V,
                                                           attn_mask=torch.from_numpy(p["mask"].astype(np.float64)))
    np.testing.assert_allclose(got, out.transpose(1, 2).numpy(), rtol=1e-5, atol=1e-6)


def test_single_token_gives_its_value():
    p = _problem(5, n=1)
    p["key_exact"] = p["value_exact"] = p["mask"] = None
    got = ar.attend(**p)
    v = (p["coef_v"] @ p["basis_v_layer"] + p["mean_v_layer"]).reshape(2, 16)
    for qh in range(6):
        np.testing.assert_allclose(got[0, :, qh], np.broadcast_to(v[qh // 3], (2, 16)), rtol=1e-5, atol=1e-6)


def test_permutation_invariance_and_lse_merge():
    p = _problem(6, n=50)
    base = ar.decode_then_attend_f64(**p)
    perm = np.random.default_rng(1).permutation(50)
    q = dict(p, coef_k=p["coef_k"][perm], coef_v=p["coef_v"][perm], cos=p["cos"][perm], sin=p["sin"][perm])
    np.testing.assert_allclose(ar.decode_then_attend_f64(**q), base, rtol=1e-10, atol=1e-12)
    # split the compressed tokens into two sets; merge softmax partials with log-sum-exp
    n, dim, heads = 50, 16, 2
    k = (p["coef_k"].astype(np.float64) @ p["basis_k_layer"] + p["mean_k_layer"]).reshape(n, heads, dim).transpose(1, 0, 2)
    k = rope_ref.rerotate(k, p["cos"].astype(np.float64), p["sin"].astype(np.float64))
    v = (p["coef_v"].astype(np.float64) @ p["basis_v_layer"] + p["mean_v_layer"]).reshape(n, heads, dim).transpose(1, 0, 2)
    qv = p["query"][0].astype(np.float64).reshape(heads, 3, 2, dim)
    s = np.einsum("hgqd,hnd->hgqn", qv, k) / np.sqrt(dim)
    parts = []
    for sl in (slice(0, 20), slice(20, 50)):
        m = s[..., sl].max(-1, keepdims=True)
        e = np.exp(s[..., sl] - m)
        parts.append((m, e.sum(-1, keepdims=True), np.einsum("hgqn,hnd->hgqd", e, v[:, sl])))
    M = np.maximum(parts[0][0], parts[1][0])
    L = sum(l * np.exp(m - M) for m, l, _ in parts)
    O = sum(o * np.exp(m - M) for m, _, o in parts) / L
    full = np.einsum("hgqn,hnd->hgqd", np.exp(s - s.max(-1, keepdims=True)) /
                     np.exp(s - s.max(-1, keepdims=True)).sum(-1, keepdims=True), v)
    np.testing.assert_allclose(O, full, rtol=1e-12, atol=1e-13)
