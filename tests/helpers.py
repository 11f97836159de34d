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


def assert_close(got: np.ndarray, ref: np.ndarray, atol=2e-3, rtol=1e-2, rel_fro=1e-2, what="", base=0.0,
                 rel_max=2e-2):
    """The north-star bar (|err| <= atol + rtol*|ref|) plus two bars on the part of the output
    that attention moves (ref - base, base = e.g. the value mean): a relative Frobenius bound and
    an elementwise one (|err| <= rel_max * max|ref - base|).  The synthetic caches' outputs are of
    order 1e-2, where the north-star absolute term alone would pass almost anything; the two
    relative bars catch the structural mistakes it hides."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert np.isfinite(ref).all(), f"{what}: the oracle's output is not finite"
    assert np.isfinite(got).all(), f"{what}: the GPU output is not finite"
    err = np.abs(got - ref)
    ok = err <= atol + rtol * np.abs(ref)
    moved = np.abs(ref - base)
    fro = np.linalg.norm(got - ref) / max(np.linalg.norm(ref - base), 1e-30)
    assert ok.all(), f"{what}: max abs err {err.max():.3e} (ref max {np.abs(ref).max():.3e})"
    assert fro <= rel_fro, f"{what}: relative Frobenius error {fro:.3e} > {rel_fro}"
    if rel_max is not None and moved.max() > 0:
        assert err.max() <= rel_max * moved.max(), \
            f"{what}: max abs err {err.max():.3e} > {rel_max} x max|ref - base| = {moved.max():.3e}"
    return float(err.max()), float(fro)


def value_mean_base(case: Case, layer: int) -> np.ndarray:
    """mean_v of the layer broadcast to the attend output layout [1, q_len, Hq, d]."""
    s = case.shape
    m = case.mean_slice("value", layer).reshape(s.kv_heads, 1, s.head_dim)
    m = np.repeat(m, s.gqa, axis=1).reshape(s.q_heads, s.head_dim)
    return np.broadcast_to(m[None, None], (1, case.q_len, s.q_heads, s.head_dim))


def workload_oracle(w, coef: dict, layer: int, b: int = 0, query_zero: bool = False) -> np.ndarray:
    """The oracle's output [1, q_len, Hq, d] for conversation ``b`` of a workloads.DecodeWorkload
    built with ``keep_host_basis`` (its float32 host bases), over ``coef`` (per stream float32
    [n_total, r]: every compressed token's coefficients).  ``query_zero`` replaces the query by 0,
    which makes the softmax uniform: the output a kernel whose scores carried no information would
    produce."""
    from oracle import attention_ref

    s = w.shape
    cu = w.context.cu_host.numpy()
    t0, t1 = int(cu[b]), int(cu[b + 1])
    e_off = np.concatenate([[0], np.cumsum(w.exact_lengths)])
    e0, e1 = int(e_off[b]), int(e_off[b + 1])
    positions = w.context.positions[t0:t1].long().cpu()
    cos = w.tables.rope_cos.cpu()[positions].numpy()
    sin = w.tables.rope_sin.cpu()[positions].numpy()
    cos, sin = np.concatenate([cos, cos], -1), np.concatenate([sin, sin], -1)
    wd = s.kv_heads * s.head_dim
    bk = w.synthetic_basis_host["key"][layer * wd:(layer + 1) * wd].T
    bv = w.synthetic_basis_host["value"][layer * wd:(layer + 1) * wd].T
    mk = w.tables.mean_k[layer].cpu().numpy()
    mv = w.tables.mean_v[layer].cpu().numpy()
    q = w.queries[layer][b:b + 1].float().cpu().numpy()
    if query_zero:
        q = np.zeros_like(q)
    return attention_ref.attend(q, coef["key"][t0:t1], coef["value"][t0:t1], bk, bv, mk, mv, cos, sin,
                                w.key_exact[layer][None, :, e0:e1].cpu().numpy(),
                                w.value_exact[layer][None, :, e0:e1].cpu().numpy())


def mean_base(shape, mean_v_layer: np.ndarray, out_shape) -> np.ndarray:
    """mean_v of a layer broadcast to an attend output of shape [B, q_len, Hq, d]."""
    m = np.repeat(np.asarray(mean_v_layer).reshape(shape.kv_heads, 1, -1), shape.gqa, axis=1)
    return np.broadcast_to(m.reshape(1, 1, shape.q_heads, -1), out_shape)


def assert_sensitive(ref: np.ndarray, uniform: np.ndarray, base, what="", rel_fro=1e-2, rel_max=2e-2,
                     factor=20.0) -> float:
    """The check is only as strong as the gap between the true output and the output of attention
    whose scores carry nothing (uniform weights): that gap must exceed ``assert_close``'s relative
    Frobenius bar ``factor`` times over, and its largest element must exceed the elementwise bar on
    the moved part (``rel_max`` x max|ref - base|) ``factor`` times over."""
    ref = np.asarray(ref, dtype=np.float64)
    diff = np.asarray(uniform, np.float64) - ref
    gap = np.linalg.norm(diff) / max(np.linalg.norm(ref - base), 1e-30)
    assert gap > factor * rel_fro, f"{what}: uniform attention is only {gap:.3e} away (bar {rel_fro})"
    moved = np.abs(ref - base).max()
    assert np.abs(diff).max() > factor * rel_max * moved, \
        f"{what}: uniform attention's largest difference {np.abs(diff).max():.3e} is within {factor} x the bar"
    return float(gap)


def importance_bar(ref: np.ndarray, atol_rel=2e-3, rtol=1e-2) -> np.ndarray:
    """The question-importance bar per token: atol_rel x max|ref| + rtol x |ref|."""
    ref = np.asarray(ref, dtype=np.float64)
    return atol_rel * np.abs(ref).max() + rtol * np.abs(ref)


def assert_importance_close(got: np.ndarray, ref: np.ndarray, alternatives: dict | None = None, what="",
                            rel_fro=1e-2, factor=20.0) -> tuple[float, float]:
    """Question importance against the oracle: every token within ``importance_bar`` and a relative
    Frobenius bound on the part of the importance the question moves (ref - mean(ref)).

    ``alternatives`` maps a name to the importance a wrong kernel would produce (uniform attention,
    keys rebuilt from 0 planes, ...), computed by the oracle on the same inputs.  Each must miss both
    bars ``factor`` times over: its largest ratio to the elementwise bar and its relative Frobenius
    distance.  A check that these alternatives would pass proves nothing, which happens when the
    question's queries leave the attention nearly uniform."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert np.isfinite(ref).all() and np.isfinite(got).all(), f"{what}: non-finite importance"
    bar = importance_bar(ref)
    moved = max(np.linalg.norm(ref - ref.mean()), 1e-30)
    for name, alt in (alternatives or {}).items():
        d = np.abs(np.asarray(alt, np.float64) - ref)
        ratio, fro_alt = float((d / bar).max()), float(np.linalg.norm(d) / moved)
        assert ratio >= factor, f"{what}: {name} misses the elementwise bar only {ratio:.1f}x (need {factor}x)"
        assert fro_alt >= factor * rel_fro, f"{what}: {name} is only {fro_alt:.3e} away (bar {rel_fro})"
        print(f"  {what}: {name} misses the bar {ratio:.0f}x (relative Frobenius {fro_alt:.2e})", flush=True)
    err = np.abs(got - ref)
    worst = float((err / bar).max())
    fro = float(np.linalg.norm(got - ref) / moved)
    assert worst <= 1.0, f"{what}: importance max err {err.max():.3e} ({worst:.2f} x the bar; max {np.abs(ref).max():.3e})"
    assert fro <= rel_fro, f"{what}: importance relative Frobenius error {fro:.3e} > {rel_fro}"
    return float(err.max()), fro
