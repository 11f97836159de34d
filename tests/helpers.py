"""Shared builders for the parity tests: one seeded synthetic conversation seen two ways,
through the oracle (numpy, CPU) and through the HIP library (GPU)."""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

import synth
from oracle import progressive_ref as pr


@dataclass
class Case:
    shape: synth.ModelShape
    ctx: synth.SyntheticContext
    order: pr.Order
    codes: dict
    low: dict
    span: dict
    pieces: dict
    coef_hot: dict          # oracle-dequantized hot coefficients, float32 [middle, r]
    cos: torch.Tensor       # [P, d]
    sin: torch.Tensor
    positions: np.ndarray   # middle positions
    key_exact: torch.Tensor  # [L, Hkv, E, d]
    value_exact: torch.Tensor
    queries: torch.Tensor    # [L, 1, Hq, q_len, d]
    mask: torch.Tensor | None
    q_len: int

    def layer_slice(self, kind: str, layer: int) -> np.ndarray:
        s = self.shape
        w = s.kv_heads * s.head_dim
        return self.ctx.basis[kind][layer * w:(layer + 1) * w].T.numpy()  # [r, Hkv*d]

    def mean_slice(self, kind: str, layer: int) -> np.ndarray:
        w = self.shape.kv_heads * self.shape.head_dim
        return self.ctx.mean[kind][layer * w:(layer + 1) * w].numpy()


def build_case(shape: synth.ModelShape, tokens: int, seed: int, budget=None, zero_frac=0.05, p=None,
               query_scale=1.0, q_len=1, query_dtype=torch.float32, sinks=4, recent=32, mean_scale=0.01,
               basis=None, mean=None, rope_rows=None) -> Case:
    ctx = synth.make_context(shape, tokens, seed, sinks=sinks, recent=recent, budget=budget, zero_frac=zero_frac,
                             p=p, mean_scale=mean_scale, basis=basis, mean=mean)
    order = pr.plane_major_order(shape.groups)
    codes, low, span, pieces, coef_hot = {}, {}, {}, {}, {}
    for kind in ("key", "value"):
        c, lo, sp = pr.quantize8(ctx.coef[kind].numpy(), 64)
        codes[kind], low[kind], span[kind] = c, lo, sp
        pieces[kind] = ctx.pieces(kind)
        coef_hot[kind] = pr.dequantize(c, lo, sp, pr.token_planes(order, pieces[kind]))
    cos, sin = synth.rope_tables(shape, rope_rows or tokens + q_len, "cpu")
    positions = np.arange(ctx.start, ctx.end)
    new_coef = {kind: synth.coefficients(q_len, shape.rank, seed + 50 + i) for i, kind in enumerate(("key", "value"))}
    exact_coef = {kind: torch.cat([ctx.exact_coef[kind], new_coef[kind]]) for kind in ("key", "value")}
    exact_pos = torch.cat([ctx.exact_positions(), torch.arange(tokens, tokens + q_len)])
    key_exact, value_exact = synth.decode_exact(ctx, exact_coef, exact_pos, cos, sin)
    queries = synth.make_queries(shape, q_len, seed + 60, dtype=query_dtype, scale=query_scale)
    n_ctx_exact = tokens - ctx.middle
    mask = synth.causal_mask(q_len, n_ctx_exact)[0, 0] if q_len > 1 else None
    return Case(shape, ctx, order, codes, low, span, pieces, coef_hot, cos, sin, positions, key_exact, value_exact,
                queries, mask, q_len)


def oracle_attend(case: Case, layer: int, dtype=np.float32):
    from oracle import attention_ref

    q = case.queries[layer].float().numpy()
    mask = None if case.mask is None else case.mask.numpy()[None, None]
    return attention_ref.attend(
        q, case.coef_hot["key"], case.coef_hot["value"], case.layer_slice("key", layer),
        case.layer_slice("value", layer), case.mean_slice("key", layer), case.mean_slice("value", layer),
        case.cos[case.positions].numpy(), case.sin[case.positions].numpy(),
        case.key_exact[layer][None].numpy(), case.value_exact[layer][None].numpy(), mask, dtype=dtype)


def gpu_context(case: Case, refine_capacity: int = 0, device="cuda"):
    """Pack both streams on the GPU and build the CompressedContext."""
    from compressed_attention import CompressedContext, ModelTables
    from hot_tier import OrderTables, PackedStream

    s = case.shape
    tables = ModelTables(case.ctx.basis["key"].to(device), case.ctx.basis["value"].to(device),
                         case.ctx.mean["key"].to(device), case.ctx.mean["value"].to(device), s.layers, s.kv_heads,
                         s.head_dim, case.cos.to(device), case.sin.to(device))
    otab = OrderTables(case.order.planes, case.order.prefix_bytes, device)
    streams = {}
    for kind in ("key", "value"):
        streams[kind] = PackedStream.pack(
            torch.from_numpy(case.codes[kind]).to(device), torch.from_numpy(case.low[kind]).to(device),
            torch.from_numpy(case.span[kind]).to(device), torch.from_numpy(case.pieces[kind]).to(device), otab,
            refine_capacity=refine_capacity)
    ctx = CompressedContext(tables, streams["key"], streams["value"], torch.from_numpy(case.positions), s.q_heads)
    return ctx, tables, streams


def gpu_attend(case: Case, ctx, layer: int, out_dtype=torch.float32, device="cuda"):
    import dkv_hip

    q = case.queries[layer].to(device).contiguous()
    out = torch.empty(1, case.q_len, case.shape.q_heads, case.shape.head_dim, dtype=out_dtype, device=device)
    ke = case.key_exact[layer].to(device).contiguous()
    ve = case.value_exact[layer].to(device).contiguous()
    mask = None if case.mask is None else case.mask.to(device).contiguous()
    args = ctx.layer_args(layer, q, out, ke, ve, mask)
    ctx.run_layer(args)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def assert_close(got: np.ndarray, ref: np.ndarray, atol=2e-3, rtol=1e-2, rel_fro=1e-2, what="", base=0.0):
    """The north-star bar (|err| <= atol + rtol*|ref|) plus a relative Frobenius bound on the
    part of the output that attention moves (ref - base, base = e.g. the value mean), which
    catches structural mistakes the loose absolute bound would hide."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert np.isfinite(ref).all(), f"{what}: the oracle's output is not finite"
    assert np.isfinite(got).all(), f"{what}: the GPU output is not finite"
    err = np.abs(got - ref)
    ok = err <= atol + rtol * np.abs(ref)
    fro = np.linalg.norm(got - ref) / max(np.linalg.norm(ref - base), 1e-30)
    assert ok.all(), f"{what}: max abs err {err.max():.3e} (ref max {np.abs(ref).max():.3e})"
    assert fro <= rel_fro, f"{what}: relative Frobenius error {fro:.3e} > {rel_fro}"
    return float(err.max()), float(fro)


def value_mean_base(case: Case, layer: int) -> np.ndarray:
    """mean_v of the layer broadcast to the attend output layout [1, q_len, Hq, d]."""
    s = case.shape
    m = case.mean_slice("value", layer).reshape(s.kv_heads, 1, s.head_dim)
    m = np.repeat(m, s.gqa, axis=1).reshape(s.q_heads, s.head_dim)
    return np.broadcast_to(m[None, None], (1, case.q_len, s.q_heads, s.head_dim))
