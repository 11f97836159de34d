"""The two other decode workloads at their real sizes, against the oracle.

- 1b-8k-2pct: Llama-3.2-1B shape, 8,192 tokens at 2 %, bf16 query, all 16 layers.  Its 64
  256-row K2 workgroups would leave CUs idle, so the decode runs one KV head per workgroup
  (``keys_scores_head_kernel<64>``, 32 tiles x 8 heads): this is its real-size check.
- The head form at head_dim 128 (a 3B-shaped 9,000-token context) and over a ragged batch of
  1B-shaped conversations.
- 3b-ragged-32: 32 Llama-3.2-3B-shaped conversations of U[2K, 16K] tokens at 3 % in one packed
  buffer, one fused varlen decode step.  The reference decodes one conversation at a time
  (scripts/dimmer.py:195-197), so the pin is the oracle per conversation: the shortest, the
  longest and a middle one, at the first and last layer; plus properties of the whole batch
  (graph replay equals the eager step, the step is deterministic, every conversation's hot
  tier fits its own budget).

Queries are peaked (N(0, 100^2)) so that the outputs depend on the scores; each checked layer
first shows that uniform attention misses the bar by a wide margin.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
PEAKED = 100.0


def _fp32_outputs(w, layer):
    """One layer of the workload again, with a float32 output [B, 1, Hq, d]."""
    s = w.shape
    out32 = torch.empty(w.batch, 1, s.q_heads, s.head_dim, dtype=torch.float32, device=DEV)
    args = w.context.layer_args(layer, w.queries[layer], out32, w.key_exact[layer], w.value_exact[layer], None,
                                tuple(w.exact_lengths))
    w.context.run_layer(args)
    torch.cuda.synchronize()
    return out32.cpu().numpy()


def test_1b_8k_2pct_all_layers_match_oracle():
    import workloads
    from helpers import assert_close, assert_sensitive, mean_base, workload_oracle

    print("[case] 1b-8k-2pct: 16-layer decode step, one KV head per K2 workgroup (peaked queries)", flush=True)
    w = workloads.build_decode("1b-8k-2pct", device=DEV, keep_host_basis=True, query_scale=PEAKED)
    s = w.shape
    tiles = -(-w.middle // 256)
    assert tiles * (s.kv_heads // (256 // s.head_dim)) < 256 <= tiles * s.kv_heads, "expected the head form"
    w.step()
    torch.cuda.synchronize()
    first = w.outs.clone()
    w.step()
    torch.cuda.synchronize()
    assert torch.equal(first, w.outs)
    coef = {k: w.streams[k].dequantize(dtype=torch.float32).cpu().numpy() for k in ("key", "value")}
    for layer in range(s.layers):
        ref = workload_oracle(w, coef, layer)
        base = mean_base(s, w.tables.mean_v[layer].cpu().numpy(), ref.shape)
        what = f"1b-8k-2pct layer {layer}"
        gap = assert_sensitive(ref, workload_oracle(w, coef, layer, query_zero=True), base, what=what)
        assert_close(w.outs[layer].float().cpu().numpy(), ref, what=f"{what} (bf16 out)", rel_fro=1e9)
        err, fro = assert_close(_fp32_outputs(w, layer), ref, what=what, base=base)
        print(f"  {what}: max abs err {err:.2e}, rel fro {fro:.2e} (uniform attention {gap:.2e} away)", flush=True)


@pytest.mark.parametrize("case", ["3b-shape-9000", "1b-ragged-5", "1b-ragged-3-short"])
def test_head_form_k2_matches_oracle(case):
    """``keys_scores_head_kernel`` (one KV head per K2 workgroup) at head_dim 128, and over ragged
    batches whose tiles belong to several conversations, the short one with half a tile per
    workgroup (128-token softmax statistics for K3a and K3c): every layer and (ragged) conversation
    against the oracle, with the uniform-attention sensitivity check; eager steps deterministic and a
    graph replay equal to them."""
    import synth
    import workloads
    from helpers import assert_close, assert_sensitive, mean_base, workload_oracle

    if case == "3b-shape-9000":
        shape = synth.ModelShape(2, 8, 128, 24, 2048)
        w = workloads.build_decode("3b-shape-9000", shape=shape, tokens=9000, budget=0.03, budget_shape=synth.SHAPE_3B,
                                   device=DEV, query_dtype=torch.bfloat16, keep_host_basis=True, query_scale=PEAKED)
        convs = [0]
    else:
        shape = synth.ModelShape(2, 8, 64, 32, 1024)
        # a two-layer model's own budget: 25 % of its 4 KB per token leaves the compressed tokens
        # about 3.3 planes on average
        count, lo, hi, seed = (5, 1000, 3000, 77) if case == "1b-ragged-5" else (3, 300, 1500, 78)
        w = workloads.build_ragged(count=count, lo=lo, hi=hi, budget=0.25, seed=seed, device=DEV, shape=shape,
                                   query_scale=PEAKED, keep_host_basis=True)
        convs = list(range(count))
    cu = w.context.cu_host.numpy()
    tiles = int(sum(-(-int(cu[b + 1] - cu[b]) // 256) for b in range(len(cu) - 1)))
    print(f"[case] head-form K2: {case}, {tiles} tiles x {shape.kv_heads} heads (peaked queries)", flush=True)
    assert tiles * (shape.kv_heads // (256 // shape.head_dim)) < 256, "expected the head form"
    half = 2 * tiles * shape.kv_heads <= 256  # half a tile per workgroup
    assert half == (case == "1b-ragged-3-short"), "expected the half-tile workgroups only for the short batch"
    w.step()
    torch.cuda.synchronize()
    eager = w.outs.clone()
    w.step()
    torch.cuda.synchronize()
    assert torch.equal(eager, w.outs)
    graph = w.capture()
    w.outs.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(w.outs, eager), "graph replay differs from the eager step"
    coef = {k: w.streams[k].dequantize(dtype=torch.float32).cpu().numpy() for k in ("key", "value")}
    for layer in range(shape.layers):
        out32 = _fp32_outputs(w, layer)
        for b in convs:
            ref = workload_oracle(w, coef, layer, b)
            base = mean_base(shape, w.tables.mean_v[layer].cpu().numpy(), ref.shape)
            what = f"{case} b={b} layer {layer}"
            gap = assert_sensitive(ref, workload_oracle(w, coef, layer, b, query_zero=True), base, what=what)
            err, fro = assert_close(out32[b:b + 1], ref, what=what, base=base)
            print(f"  {what}: max abs err {err:.2e}, rel fro {fro:.2e} (uniform attention {gap:.2e} away)",
                  flush=True)


def test_3b_ragged_32_matches_per_conversation_oracle():
    import workloads
    from helpers import assert_close, assert_sensitive, mean_base, workload_oracle

    print("[case] 3b-ragged-32: 32 conversations, one varlen decode step (peaked queries)", flush=True)
    w = workloads.build_ragged(device=DEV, query_scale=PEAKED, keep_host_basis=True)
    s = w.shape
    lengths = np.asarray(w.lengths)
    cu = w.context.cu_host.numpy()
    assert len(lengths) == 32 and lengths.min() >= 2048 and lengths.max() <= 16384
    print(f"  {int(lengths.sum())} tokens, {int(cu[-1])} compressed; lengths {lengths.min()}..{lengths.max()}",
          flush=True)
    # every conversation's hot tier (progressive.py:185-188) fits its own 3 % budget
    for b, tokens in enumerate(lengths):
        hot = 0
        for k in ("key", "value"):
            st = w.streams[k]
            hot += int(st.tables.prefix64[st.pieces[cu[b]:cu[b + 1]].long()].sum()) + int(cu[b + 1] - cu[b])
        exact = int(tokens) - int(cu[b + 1] - cu[b])
        assert hot + exact * 2 * s.exact_bytes <= int(w.budget * tokens * 2 * s.exact_bytes), f"conversation {b}"
    # eager step twice (deterministic), then graph replays with eager work between them
    w.step()
    torch.cuda.synchronize()
    eager = w.outs.clone()
    w.step()
    torch.cuda.synchronize()
    assert torch.equal(eager, w.outs)
    graph = w.capture()
    for rep in range(2):
        w.outs.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(w.outs, eager), f"graph replay {rep} differs from the eager step"
    coef = {k: w.streams[k].dequantize(dtype=torch.float32).cpu().numpy() for k in ("key", "value")}
    order = np.argsort(lengths, kind="stable")
    picks = {"shortest": int(order[0]), "middle": int(order[len(order) // 2]), "longest": int(order[-1])}
    for layer in (0, s.layers - 1):
        out32 = _fp32_outputs(w, layer)
        for label, b in picks.items():
            ref = workload_oracle(w, coef, layer, b)
            base = mean_base(s, w.tables.mean_v[layer].cpu().numpy(), ref.shape)
            what = f"ragged {label} (b={b}, T={lengths[b]}) layer {layer}"
            gap = assert_sensitive(ref, workload_oracle(w, coef, layer, b, query_zero=True), base, what=what)
            assert_close(w.outs[layer][b:b + 1].float().cpu().numpy(), ref, what=f"{what} (bf16 out)", rel_fro=1e9)
            err, fro = assert_close(out32[b:b + 1], ref, what=what, base=base)
            print(f"  {what}: max abs err {err:.2e}, rel fro {fro:.2e} (uniform attention {gap:.2e} away)",
                  flush=True)
