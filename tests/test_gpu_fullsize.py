"""Parity at the benchmark's full size (Llama-3.2-3B shape, 16,384-token context at 3 %):
the question stage and a whole 28-layer decode step over the packed cache, checked against
the oracle on layers spread over the model, plus size-independent properties (byte
accounting within the budget, refined tokens decoding at full precision, the decode being
deterministic step to step)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_3b_16k_question_then_decode_matches_oracle():
    import workloads
    from helpers import assert_close
    from oracle import attention_ref, scoring_ref
    from oracle import progressive_ref as pr

    print("[case] full size 3b-16k-3pct: question stage + decode step", flush=True)
    w = workloads.build_decode("3b-16k-3pct", device=DEV, keep_host_basis=True, refine_fraction=0.01)
    s = w.shape
    # byte accounting of the packed hot tier (progressive.py:185-188) fits the 3 % budget
    hot = w.context.key.hot_bytes() + w.context.value.hot_bytes()
    exact_tokens = w.tokens - w.middle
    budget = int(0.03 * w.tokens * 2 * s.exact_bytes)
    assert hot + exact_tokens * 2 * s.exact_bytes <= budget
    # question: score, select, gather
    q = w.question
    imp = q.score().clone()
    idx = q.select().cpu().numpy()
    assert np.array_equal(idx, scoring_ref.topk_indices(imp.cpu().numpy(), q.count))
    before = {k: w.streams[k].pieces.clone() for k in ("key", "value")}
    fetched = q.gather()
    order = pr.plane_major_order(s.groups)
    pieces = {k: before[k].long().cpu().numpy() for k in ("key", "value")}
    assert fetched == pr.fetched_bytes({"key": order, "value": order}, pieces, idx)
    for k in ("key", "value"):
        after = w.streams[k].pieces.cpu().numpy()
        assert (after[idx] == order.pieces).all()
        mask = np.ones(len(after), bool)
        mask[idx] = False
        assert np.array_equal(after[mask], pieces[k][mask])
    # decode step over the refined cache, twice: deterministic
    w.step()
    torch.cuda.synchronize()
    first = w.outs.clone()
    w.step()
    torch.cuda.synchronize()
    assert torch.equal(first, w.outs)
    coef = {k: w.streams[k].dequantize(dtype=torch.float32).cpu().numpy() for k in ("key", "value")}
    positions = w.context.positions.long().cpu()
    cos = w.tables.rope_cos.cpu()[positions].numpy()
    sin = w.tables.rope_sin.cpu()[positions].numpy()
    cos, sin = np.concatenate([cos, cos], -1), np.concatenate([sin, sin], -1)
    wd = s.kv_heads * s.head_dim
    for layer in (0, 13, 27):
        bk = w.synthetic_basis_host["key"][layer * wd:(layer + 1) * wd].T
        bv = w.synthetic_basis_host["value"][layer * wd:(layer + 1) * wd].T
        mk = w.tables.mean_k[layer].cpu().numpy()
        mv = w.tables.mean_v[layer].cpu().numpy()
        ref = attention_ref.attend(w.queries[layer].float().cpu().numpy(), coef["key"], coef["value"], bk, bv, mk, mv,
                                   cos, sin, w.key_exact[layer][None].cpu().numpy(),
                                   w.value_exact[layer][None].cpu().numpy())
        base = np.broadcast_to(np.repeat(mv.reshape(s.kv_heads, 1, -1), s.gqa, axis=1).reshape(1, 1, s.q_heads, -1),
                               ref.shape)
        # the benchmark's decode writes bf16 (the model's dtype): elementwise bar on that output;
        # the same layer with an fp32 output must also meet the relative Frobenius bar
        assert_close(w.outs[layer].float().cpu().numpy(), ref, what=f"3b-16k layer {layer} (bf16 out)", rel_fro=1e9)
        out32 = torch.empty(1, 1, s.q_heads, s.head_dim, dtype=torch.float32, device=DEV)
        args = w.context.layer_args(layer, w.queries[layer], out32, w.key_exact[layer], w.value_exact[layer])
        w.context.run_layer(args)
        torch.cuda.synchronize()
        err, fro = assert_close(out32.cpu().numpy(), ref, what=f"3b-16k layer {layer}", base=base)
        print(f"  layer {layer}: max abs err {err:.2e}, rel fro {fro:.2e}", flush=True)


def test_3b_16k_dkvtc_decode_matches_oracle():
    """The dkvtc@0.03:snap:floor1 entry point at full size: prefill -> Methods.apply ->
    CompressedContext(codec, keys, values, model) -> 28-layer decode over the ladder codes,
    deterministic, and equal to the oracle's attention over codec.last_coefficients on layers
    spread over the model."""
    import workloads
    from helpers import assert_close
    from oracle import attention_ref

    print("[case] full size 3b-16k-3pct: dkvtc decode step", flush=True)
    w = workloads.build_dkvtc("3b-16k-3pct", device=DEV)
    s, codec, ctx = w.shape, w.codec, w.context
    start, _ = codec.last_span
    choice_k = codec.last_choice["key"].cpu().numpy()
    kept = choice_k >= 0
    n_extra = 0 if ctx.extra is None else ctx.extra["key"][0].shape[1]
    print(f"  coded tokens {ctx.key.n}, exact-rung tokens {n_extra}, ladder groups {ctx.tables.rank // 64}",
          flush=True)
    w.step()
    torch.cuda.synchronize()
    first = w.outs.clone()
    w.step()
    torch.cuda.synchronize()
    assert torch.equal(first, w.outs)
    coef = {k: codec.last_coefficients[k].float().cpu().numpy()[kept] for k in ("key", "value")}
    pos = np.nonzero(kept)[0] + start
    cos = w.tables.rope_cos.cpu().numpy()[pos]
    sin = w.tables.rope_sin.cpu().numpy()[pos]
    cos, sin = np.concatenate([cos, cos], -1), np.concatenate([sin, sin], -1)
    wd = s.kv_heads * s.head_dim
    for layer in (0, 13, 27):
        basis = {k: codec.streams[k].basis[layer * wd:(layer + 1) * wd].T.cpu().numpy() for k in ("key", "value")}
        mean = {k: codec.streams[k].mean[layer * wd:(layer + 1) * wd].cpu().numpy() for k in ("key", "value")}
        ref = attention_ref.attend(w.queries[layer].float().cpu().numpy(), coef["key"], coef["value"], basis["key"],
                                   basis["value"], mean["key"], mean["value"], cos, sin,
                                   w.key_exact[layer][None, :, n_extra:].cpu().numpy(),
                                   w.value_exact[layer][None, :, n_extra:].cpu().numpy())
        base = np.broadcast_to(np.repeat(mean["value"].reshape(s.kv_heads, 1, -1), s.gqa, axis=1)
                               .reshape(1, 1, s.q_heads, -1), ref.shape)
        assert_close(w.outs[layer].float().cpu().numpy(), ref, what=f"dkvtc layer {layer} (bf16 out)", rel_fro=1e9)
        out32 = torch.empty(1, 1, s.q_heads, s.head_dim, dtype=torch.float32, device=DEV)
        args = ctx.layer_args(layer, w.queries[layer], out32, w.key_exact[layer], w.value_exact[layer])
        ctx.run_layer(args)
        torch.cuda.synchronize()
        err, fro = assert_close(out32.cpu().numpy(), ref, what=f"dkvtc layer {layer}", base=base)
        print(f"  layer {layer}: max abs err {err:.2e}, rel fro {fro:.2e}", flush=True)
