"""GPU parity of question-time work and of ragged batches (through the C ABI) against the oracle.

- K4a: question scoring over the hot tier with the first 2 planes per group
  (scripts/progressive.py:239-254 with scripts/dimmer.py:52-66), against
  oracle/scoring_ref.importance on the same capped coefficients;
- K4b: top 1 % selection (scripts/methods.py:246-247) - exact on the GPU's own
  scores, and equal to the oracle's set wherever the score margin exceeds the
  scores' tolerance;
- K4c + re-attend: refined tokens decode at full precision and attention over
  the refined cache matches the oracle;
- varlen: one fused decode over several conversations (cu_seqlens) equals the
  per-conversation oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import synth
from helpers import (assert_close, assert_importance_close, build_case, gpu_attend, gpu_context, oracle_attend,
                     value_mean_base)
from oracle import progressive_ref as pr
from oracle import scoring_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _oracle_importance(case, plane_cap):
    s = case.shape
    planes = np.minimum(pr.token_planes(case.order, case.pieces["key"]), plane_cap)
    coef = pr.dequantize(case.codes["key"], case.low["key"], case.span["key"], planes)
    basis = case.ctx.basis["key"].numpy().T.reshape(s.rank, s.layers, s.kv_heads * s.head_dim)
    mean = case.ctx.mean["key"].numpy().reshape(s.layers, s.kv_heads * s.head_dim)
    e_ctx = case.key_exact.shape[2] - case.q_len
    return scoring_ref.importance(case.queries[:, 0].float().numpy(), coef, basis, mean,
                                  case.cos[case.positions].numpy(), case.sin[case.positions].numpy(),
                                  case.key_exact[:, :, :e_ctx].numpy(), case.key_exact[:, :, e_ctx:].numpy(),
                                  s.kv_heads)


def _gpu_importance(case, ctx, plane_cap):
    s = case.shape
    ctx.begin_scoring(plane_cap)
    for layer in range(s.layers):
        q = case.queries[layer].to(DEV).contiguous()
        key = case.key_exact[layer][None].to(DEV).contiguous()
        ctx._score(layer, q, key, None)
    imp = ctx.end_scoring()
    torch.cuda.synchronize()
    return imp


@pytest.mark.parametrize("shape_name,tokens,q_len,plane_cap,qdtype", [
    ("1b2", 1100, 16, 2, "float32"),
    ("3b2", 900, 8, 2, "float32"),
    ("1b2", 600, 4, 8, "float32"),
    ("3b2", 1300, 16, 2, "bfloat16"),  # the scoring epilogue is instantiated per query type
    ("1b2", 800, 8, 2, "float16"),
    # more than 192 query rows per KV head: the scoring epilogue stages its query rows in two chunks
    ("1b2", 700, 64, 2, "bfloat16"),
    ("3b2", 600, 72, 2, "float32"),
])
def test_question_scoring_and_topk(shape_name, tokens, q_len, plane_cap, qdtype):
    import dkv_hip

    shape = synth.ModelShape(2, 8, 64, 32, 1024) if shape_name == "1b2" else synth.ModelShape(2, 8, 128, 24, 2048)
    print(f"[case] scoring {shape_name} T={tokens} q_len={q_len} cap={plane_cap} {qdtype}", flush=True)
    case = build_case(shape, tokens, seed=321, query_scale=40.0, q_len=q_len, query_dtype=getattr(torch, qdtype))
    ctx, _, _ = gpu_context(case)
    got = _gpu_importance(case, ctx, plane_cap).cpu().numpy()
    ref = _oracle_importance(case, plane_cap)
    scale = float(np.abs(ref).max())
    # what a kernel whose scores carried nothing (zero query: uniform attention) or whose keys kept
    # no plane would give; both must miss the bar 20 times over
    queries = case.queries
    case.queries = torch.zeros_like(queries)
    uniform = _oracle_importance(case, plane_cap)
    case.queries = queries
    alternatives = {"uniform attention": uniform, "0-plane keys": _oracle_importance(case, 0)}
    err, fro = assert_importance_close(got, ref, alternatives, what="importance")
    # K4b on the GPU's scores is exact
    n = ctx.key.n
    count = scoring_ref.select_count(0.01, n)
    idx = torch.empty(count, dtype=torch.int32, device=DEV)
    dkv_hip.topk(torch.from_numpy(got).to(DEV), count, idx)
    gpu_set = idx.cpu().numpy()
    assert np.array_equal(gpu_set, scoring_ref.topk_indices(got, count))
    # equal to the oracle's selection except where the two scores' order is within tolerance
    ref_set = scoring_ref.topk_indices(ref, count)
    kth = np.sort(ref)[::-1][count - 1]
    tol = 2e-3 * scale + 1e-2 * abs(kth)
    ambiguous = set(np.nonzero(np.abs(ref - kth) <= 2 * tol)[0].tolist())
    diff = set(gpu_set.tolist()) ^ set(ref_set.tolist())
    assert diff <= ambiguous, f"selection differs outside the tie band: {sorted(diff - ambiguous)}"
    print(f"  max err {err:.2e} of {scale:.2e} (rel fro {fro:.2e}); margin {scoring_ref.topk_margin(ref, count):.2e}; "
          f"set differences inside the tie band: {len(diff)}", flush=True)


def test_refine_then_attend():
    """Top tokens get their cold planes (K4c); attention then sees them at full precision."""
    shape = synth.ModelShape(2, 8, 64, 32, 1024)
    print("[case] refine then attend", flush=True)
    case = build_case(shape, 1200, seed=77, query_scale=60.0)
    ctx, _, streams = gpu_context(case, refine_capacity=64)
    got0 = gpu_attend(case, ctx, 1)
    rows = np.array([0, 5, 100, 400, 777, case.ctx.middle - 1])
    fetched = sum(streams[k].refine(torch.from_numpy(rows).to(DEV)) for k in ("key", "value"))
    orders = {"key": case.order, "value": case.order}
    assert fetched == pr.fetched_bytes(orders, case.pieces, rows)
    for kind in ("key", "value"):
        case.pieces[kind] = case.pieces[kind].copy()
        case.pieces[kind][rows] = case.order.pieces
        planes = pr.token_planes(case.order, case.pieces[kind])
        case.coef_hot[kind] = pr.dequantize(case.codes[kind], case.low[kind], case.span[kind], planes)
        got_coef = streams[kind].dequantize(dtype=torch.float32).cpu().numpy()
        assert np.array_equal(got_coef.view(np.uint32), case.coef_hot[kind].view(np.uint32))
    got = gpu_attend(case, ctx, 1)
    assert_close(got, oracle_attend(case, 1), what="refined attend", base=value_mean_base(case, 1))
    assert not np.array_equal(got, got0)
    # refining again is a no-op with zero bytes fetched
    assert sum(streams[k].refine(torch.from_numpy(rows).to(DEV)) for k in ("key", "value")) == 0


@pytest.mark.parametrize("tier", ["device", "host"])
def test_refine_with_repeated_rows(tier):
    """Rows given more than once: ``fetched`` counts each occurrence (the reference's formula over
    the rows as given, scripts/progressive.py:232) and each distinct row is merged once.  The host
    tier gathers the sorted distinct rows, so its refined tier is byte for byte the tier refined
    with them; the device tier (dkv_refine_rows) puts each row at its first entry's slot, so its
    tokens decode to the same values with the same pieces.  Rows outside the stream raise and
    change nothing."""
    from hot_tier import OrderTables, PackedStream

    shape = synth.ModelShape(2, 8, 64, 32, 1024)
    print(f"[case] refine with repeated rows ({tier} cold tier)", flush=True)
    case = build_case(shape, 900, seed=79, query_scale=60.0)
    otab = OrderTables(case.order.planes, case.order.prefix_bytes, DEV)

    def packed():
        return PackedStream.pack(torch.from_numpy(case.codes["key"]).to(DEV), torch.from_numpy(case.low["key"]).to(DEV),
                                 torch.from_numpy(case.span["key"]).to(DEV),
                                 torch.from_numpy(case.pieces["key"]).to(DEV), otab, refine_capacity=16, cold_tier=tier)

    rows = np.array([7, 300, 7, 42, 300, 300, 5])
    a, b = packed(), packed()
    fetched = a.refine(torch.from_numpy(rows).to(DEV))
    assert fetched == pr.fetched_bytes({"key": case.order}, {"key": case.pieces["key"]}, rows)
    b.refine(torch.from_numpy(np.unique(rows)).to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(a.pieces, b.pieces)
    if tier == "host":
        assert a.refined == b.refined == len(np.unique(rows))
        assert torch.equal(a.tok_off, b.tok_off) and torch.equal(a.blob, b.blob)
    else:
        assert a.refined == len(rows) and b.refined == len(np.unique(rows))
        assert torch.equal(a.dequantize(), b.dequantize())
    state = (a.refined, a.pieces.clone(), a.tok_off.clone(), a.blob.clone(), a.version)
    with pytest.raises(ValueError, match="refine rows"):
        a.refine(torch.tensor([0, case.ctx.middle], device=DEV))
    torch.cuda.synchronize()
    assert a.refined == state[0] and torch.equal(a.pieces, state[1]) and torch.equal(a.tok_off, state[2])
    assert torch.equal(a.blob, state[3]) and a.version == state[4]


def test_refine_from_host_cold_tier_matches_device_tier():
    """A cold tier in pinned host memory (only the chosen tokens' planes copied over) refines to the
    same bytes as the device-resident one, including rows refined twice and rows already full."""
    from hot_tier import OrderTables, PackedStream

    shape = synth.ModelShape(2, 8, 64, 32, 1024)
    print("[case] host cold tier", flush=True)
    case = build_case(shape, 1200, seed=78, query_scale=60.0)
    otab = OrderTables(case.order.planes, case.order.prefix_bytes, DEV)
    full_pieces = case.pieces["key"].copy()
    full_pieces[[3, 9]] = case.order.pieces  # two tokens already at full precision
    packs = {}
    for tier in ("device", "host"):
        packs[tier] = PackedStream.pack(torch.from_numpy(case.codes["key"]).to(DEV),
                                        torch.from_numpy(case.low["key"]).to(DEV),
                                        torch.from_numpy(case.span["key"]).to(DEV),
                                        torch.from_numpy(full_pieces).to(DEV), otab, refine_capacity=64,
                                        cold_tier=tier)
    assert packs["host"].cold_on_host and not packs["device"].cold_on_host
    assert torch.equal(packs["host"].cold.cuda()[:packs["device"].cold.numel()], packs["device"].cold)
    for rows in ([0, 3, 5, 100, 777], [5, 9, 400, 1100, 0], [case.ctx.middle - 1]):
        r = torch.tensor(rows, device=DEV)
        fetched = [packs[t].refine(r) for t in ("device", "host")]
        torch.cuda.synchronize()
        assert fetched[0] == fetched[1]
        a, b = packs["device"], packs["host"]
        assert torch.equal(a.tok_off, b.tok_off) and torch.equal(a.pieces, b.pieces)
        assert torch.equal(a.blob, b.blob)
    got = packs["host"].dequantize().cpu().numpy()
    want = packs["device"].dequantize().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("lengths", [(700, 1333, 300), (700, 36, 300), (36, 36)],
                         ids=["ragged", "one-all-exact", "all-exact"])
def test_varlen_matches_per_sequence_oracle(lengths):
    """Conversations in one packed buffer, one fused decode step (cu_seqlens, cu_exact); a
    conversation of 36 tokens (4 sinks + 32 recent) has no compressed token at all."""
    from compressed_attention import CompressedContext, ModelTables
    from hot_tier import OrderTables, PackedStream

    shape = synth.ModelShape(2, 8, 128, 24, 2048)
    print(f"[case] varlen {lengths}", flush=True)
    basis = {"key": synth.orthonormal_basis(shape.features, shape.rank, 901),
             "value": synth.orthonormal_basis(shape.features, shape.rank, 902)}
    g = torch.Generator("cpu").manual_seed(903)
    mean = {k: torch.randn(shape.features, generator=g) * 0.01 for k in ("key", "value")}
    rope_rows = max(lengths) + 1
    cases = [build_case(shape, T, seed=500 + 17 * i, query_scale=80.0, basis=basis, mean=mean, rope_rows=rope_rows)
             for i, T in enumerate(lengths)]
    c0 = cases[0]
    tables = ModelTables(basis["key"].to(DEV), basis["value"].to(DEV), mean["key"].to(DEV), mean["value"].to(DEV),
                         shape.layers, shape.kv_heads, shape.head_dim, c0.cos.to(DEV), c0.sin.to(DEV))
    otab = OrderTables(c0.order.planes, c0.order.prefix_bytes, DEV)
    streams = {}
    for kind in ("key", "value"):
        cat = lambda f: torch.from_numpy(np.concatenate([getattr(c, f)[kind] for c in cases])).to(DEV)  # noqa: E731
        streams[kind] = PackedStream.pack(cat("codes"), cat("low"), cat("span"), cat("pieces"), otab)
    mids = [c.ctx.middle for c in cases]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(mids)]), dtype=torch.int32)
    positions = torch.from_numpy(np.concatenate([c.positions for c in cases]))
    ctx = CompressedContext(tables, streams["key"], streams["value"], positions, shape.q_heads, cu_seqlens=cu)
    for layer in range(shape.layers):
        q = torch.cat([c.queries[layer] for c in cases]).to(DEV).contiguous()  # [B, Hq, 1, d]
        ke = torch.cat([c.key_exact[layer] for c in cases], dim=1).to(DEV).contiguous()
        ve = torch.cat([c.value_exact[layer] for c in cases], dim=1).to(DEV).contiguous()
        out = torch.empty(len(cases), 1, shape.q_heads, shape.head_dim, device=DEV)
        args = ctx.layer_args(layer, q, out, ke, ve, None, tuple(c.key_exact.shape[2] for c in cases))
        ctx.run_layer(args)
        torch.cuda.synchronize()
        for b, c in enumerate(cases):
            err, fro = assert_close(out[b:b + 1].cpu().numpy(), oracle_attend(c, layer),
                                    what=f"seq {b} layer {layer}", base=value_mean_base(c, layer))
            print(f"  seq {b} (T={lengths[b]}) layer {layer}: max abs err {err:.2e}, rel fro {fro:.2e}", flush=True)
