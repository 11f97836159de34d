"""GPU parity of the progressive encoder (scripts/progressive.py:135-172) against the oracle.

Each stage is checked on the GPU's own inputs to that stage, so the comparison
is exact wherever the reference's arithmetic is exact: quantize8 bit for bit,
the error table to float32 summation order, the allocation bit for bit given
the same errors, the packed tiers byte for byte, and the byte accounting
against the reference's formulas.  The end-to-end encode is then attended
over and compared with the oracle's attention over the same codes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import synth
from helpers import assert_close
from oracle import attention_ref, kvtc_ref, packing_ref
from oracle import progressive_ref as pr

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_quantize8_kernel_bit_exact_with_degenerate_group():
    """The HIP encoder (dkv_quantize8) equals the oracle's quantize8 bit for bit over groups whose
    scales span four decades, including a group whose fp16 span rounds to 0 (code 0 by this build's
    definition), and its error table matches the oracle's to float32 summation order."""
    import progressive

    print("[case] quantize8 kernel, 64 x 512 coefficients incl. a degenerate group", flush=True)
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 512)) * rng.uniform(0.001, 10, (64, 1))).astype(np.float32)
    x[0, :64] = 0.0  # degenerate group: span rounds to 0
    x[0, 1] = 1e-9
    c0, l0, s0 = pr.quantize8(x, 64)
    coef = torch.from_numpy(x).to(DEV)
    c1, l1, s1 = progressive.quantize8(coef, 64)
    assert np.array_equal(c0, c1.cpu().numpy())
    assert np.array_equal(l0.view(np.uint16), l1.cpu().numpy().view(np.uint16))
    assert np.array_equal(s0.view(np.uint16), s1.cpu().numpy().view(np.uint16))
    table = progressive._quantize8_hip(coef, 64, True)[3].cpu().numpy()
    np.testing.assert_allclose(table, pr.error_table(x, c0, l0, s0), rtol=2e-5, atol=1e-12)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_centered_rows_bit_exact(dtype):
    """dkv_centered_rows (KVTCCodec.centered on GPU caches) equals the torch arithmetic it replaces,
    (to_matrix(caches)[start:end] - mean) with the keys de-rotated (scripts/kvtc.py:40-43, :137-140,
    :189), bit for bit, for keys and values, head_dim 64 and 128 (every rotate_half branch), with
    positions whose cos^2 + sin^2 differs from 1 in the last bits."""
    import kvtc

    for shape, tokens, start, end in [(synth.ModelShape(2, 8, 64, 32, 1024), 300, 4, 268),
                                      (synth.ModelShape(3, 8, 128, 24, 2048), 257, 0, 257)]:
        print(f"[case] centered rows {dtype} head_dim={shape.head_dim} rows {start}..{end}", flush=True)
        ctx = synth.make_context(shape, tokens, seed=11)
        model = synth.RopeModel(shape, DEV)
        codec = kvtc.KVTCCodec(synth.kvtc_checkpoint(ctx), DEV, model)
        keys, values = synth.prefill_cache(ctx, device=DEV, dtype=dtype)
        cos, sin = kvtc.rope_tables(model, tokens, DEV)
        for kind, caches in (("key", keys), ("value", values)):
            caches = [t.to(DEV) for t in caches]
            want = codec.to_matrix(caches, kind, cos, sin)[start:end] - codec.streams[kind].mean
            got = codec.centered(caches, kind, cos, sin, start, end)
            assert got.shape == want.shape and torch.equal(got, want), \
                f"{kind}: max diff {(got - want).abs().max().item():.3e}"


@pytest.mark.parametrize("budget,weighted", [(0.25, False), (0.2, True)])
def test_encode_stages_match_oracle(budget, weighted):
    import kvtc
    import progressive

    shape = synth.ModelShape(2, 8, 64, 32, 1024)
    tokens = 700
    print(f"[case] encode budget={budget} weighted={weighted}", flush=True)
    ctx = synth.make_context(shape, tokens, seed=42)
    model = synth.RopeModel(shape, DEV)
    codec = progressive.ProgressiveCodec(synth.kvtc_checkpoint(ctx), synth.order_checkpoint(shape), DEV, model)
    keys, values = synth.prefill_cache(ctx, device=DEV, dtype=torch.float16)
    weights = None
    if weighted:
        weights = torch.rand(tokens, generator=torch.Generator("cpu").manual_seed(5)).to(DEV) + 0.1
    stored = codec.encode(keys, values, budget, 32, weights=weights, refine_capacity=8)
    torch.cuda.synchronize()
    start, end = stored.start, stored.end
    middle = end - start
    cos, sin = kvtc.rope_tables(model, tokens, DEV)
    order = pr.plane_major_order(shape.groups)
    for i, kind in enumerate(("key", "value")):
        coef = codec.stream_coefficients(kind, keys if kind == "key" else values, cos, sin, start, end)
        c_np = coef.float().cpu().numpy()
        codes, low, span = pr.quantize8(c_np, 64)
        g_codes, g_low, g_span = codec.last_quantized[kind]
        assert np.array_equal(g_codes.cpu().numpy(), codes), f"{kind}: quantize8 codes"
        assert np.array_equal(g_low.cpu().numpy().view(np.uint16), low.view(np.uint16))
        assert np.array_equal(g_span.cpu().numpy().view(np.uint16), span.view(np.uint16))
        table = codec.error_table(coef).cpu().numpy()
        np.testing.assert_allclose(table, pr.error_table(c_np, codes, low, span), rtol=2e-5, atol=1e-9)
        # the reference's signature, with the codes given: they must be quantize8's
        assert torch.equal(codec.error_table(coef, g_codes, g_low, g_span), codec.error_table(coef))
        with pytest.raises(ValueError, match="codes are not"):
            codec.error_table(coef, g_codes ^ 1, g_low, g_span)
        # packed tiers byte for byte at the chosen prefixes
        pieces = stored.stores[kind].hot_pieces.cpu().numpy()
        hot, hot_off, cold, cold_off = packing_ref.pack(codes, low, span, pieces, order)
        packed = stored.stores[kind].packed
        assert np.array_equal(packed.blob[: packed.hot_used].cpu().numpy(), hot)
        assert np.array_equal(packed.cold[: int(cold_off[-1])].cpu().numpy(), cold)
    # allocation: same rule on the same float32 errors
    errors = codec.last_errors.float().cpu().numpy()
    remaining = stored.budget_bytes - (tokens - middle) * 2 * codec.exact_bytes
    want = kvtc_ref.allocate_rungs(errors, np.array(codec.last_level_bytes), middle, remaining)
    assert np.array_equal(codec.last_chosen.cpu().numpy(), want)
    rungs = np.array(order.rungs)
    for i, kind in enumerate(("key", "value")):
        assert np.array_equal(stored.stores[kind].hot_pieces.cpu().numpy(), rungs[want[i * middle:(i + 1) * middle]])
    # byte accounting (progressive.py:185-194) and the budget
    orders = {"key": order, "value": order}
    pieces = {k: stored.stores[k].hot_pieces.cpu().numpy() for k in ("key", "value")}
    assert stored.hot_bytes == pr.hot_bytes(orders, pieces, tokens - middle, shape.exact_bytes)
    assert stored.cold_bytes == pr.cold_bytes(orders, pieces)
    assert stored.hot_bytes <= stored.budget_bytes


def test_encode_then_attend_over_codes():
    """encode -> context() -> one layer of attention; the oracle attends over the same codes."""
    import kvtc
    import progressive

    shape = synth.ModelShape(2, 8, 64, 32, 1024)
    tokens = 800
    print("[case] encode then attend", flush=True)
    ctx = synth.make_context(shape, tokens, seed=43)
    model = synth.RopeModel(shape, DEV)
    codec = progressive.ProgressiveCodec(synth.kvtc_checkpoint(ctx), synth.order_checkpoint(shape), DEV, model)
    keys, values = synth.prefill_cache(ctx, device=DEV, dtype=torch.float32)
    stored = codec.encode(keys, values, 0.25, 32)
    cc = stored.context(shape.q_heads, rope_rows=tokens + 1)
    layer = 1
    q = synth.make_queries(shape, 1, 99, scale=30.0)[layer].to(DEV)
    ke = stored.exact["key"][layer][0].float().contiguous()
    ve = stored.exact["value"][layer][0].float().contiguous()
    out = torch.empty(1, 1, shape.q_heads, shape.head_dim, device=DEV)
    args = cc.layer_args(layer, q, out, ke, ve)
    cc.run_layer(args)
    torch.cuda.synchronize()
    w = shape.kv_heads * shape.head_dim
    cos, sin = kvtc.rope_tables(model, tokens + 1, DEV)
    pos = np.arange(stored.start, stored.end)
    coef = {k: stored.stores[k].packed.dequantize().cpu().numpy() for k in ("key", "value")}
    ref = attention_ref.attend(
        q.cpu().numpy(), coef["key"], coef["value"], ctx.basis["key"][layer * w:(layer + 1) * w].T.numpy(),
        ctx.basis["value"][layer * w:(layer + 1) * w].T.numpy(), ctx.mean["key"][layer * w:(layer + 1) * w].numpy(),
        ctx.mean["value"][layer * w:(layer + 1) * w].numpy(), cos.cpu().numpy()[pos], sin.cpu().numpy()[pos],
        ke[None].cpu().numpy(), ve[None].cpu().numpy())
    base = np.broadcast_to(np.repeat(ctx.mean["value"][layer * w:(layer + 1) * w].numpy().reshape(shape.kv_heads, 1, -1),
                                     shape.gqa, axis=1).reshape(1, 1, shape.q_heads, -1), ref.shape)
    assert_close(out.cpu().numpy(), ref, what="encode->attend", base=base)


def test_3b_16k_encode_bit_exact():
    """Config 4 at full size: Llama-3.2-3B shape, 16,384 tokens, 3 % budget, 2-plane floor.  quantize8
    bit for bit, the error table to float32 summation order, the allocation bit for bit on the GPU's
    errors (floor offset as scripts/kvtc.py:209-219), packed tiers byte for byte for every token,
    every tier size and the budget by the reference's byte formulas.  The allocator is also run on
    the oracle's own error table; slots whose rung differs (near-ties of last-bit fp32 sums) are
    counted and must stay rare."""
    import time

    import kvtc
    import progressive

    shape = synth.SHAPE_3B
    tokens = 16384
    print("[case] full-size encode (3B, 16384 tokens, 3 %, 2-plane floor)", flush=True)
    ctx = synth.make_context(shape, tokens, seed=4040, device=DEV)
    model = synth.RopeModel(shape, DEV)
    codec = progressive.ProgressiveCodec(synth.kvtc_checkpoint(ctx), synth.order_checkpoint(shape), DEV, model)
    keys, values = synth.prefill_cache(ctx, device=DEV, dtype=torch.float16, compute_device=DEV)
    order = pr.plane_major_order(shape.groups)
    floor = order.rungs.index(2 * shape.groups)  # the rung holding 2 planes of every group
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    stored = codec.encode(keys, values, 0.03, 32, floor_rung=floor)
    torch.cuda.synchronize()
    print(f"  encode {1e3 * (time.perf_counter() - t0):.1f} ms", flush=True)
    start, end = stored.start, stored.end
    middle = end - start
    cos, sin = kvtc.rope_tables(model, tokens, DEV)
    oracle_errors = []
    for kind in ("key", "value"):
        coef = codec.stream_coefficients(kind, keys if kind == "key" else values, cos, sin, start, end)
        c_np = coef.float().cpu().numpy()
        codes, low, span = pr.quantize8(c_np, 64)
        g_codes, g_low, g_span = codec.last_quantized[kind]
        assert np.array_equal(g_codes.cpu().numpy(), codes), f"{kind}: quantize8 codes"
        assert np.array_equal(g_low.cpu().numpy().view(np.uint16), low.view(np.uint16))
        assert np.array_equal(g_span.cpu().numpy().view(np.uint16), span.view(np.uint16))
        table_o = pr.error_table(c_np, codes, low, span)
        table = codec.error_table(coef).cpu().numpy()
        np.testing.assert_allclose(table, table_o, rtol=2e-5, atol=1e-9)
        oracle_errors.append(pr.rung_errors(c_np, table_o, order))
        del coef, table, table_o
        pieces = stored.stores[kind].hot_pieces.cpu().numpy()
        assert (pieces >= order.rungs[floor]).all(), f"{kind}: a token below the 2-plane floor"
        packed = stored.stores[kind].packed
        hot, hot_off, cold, cold_off = packing_ref.pack_fast(codes, low, span, pieces, order)
        del c_np, codes, low, span
        assert np.array_equal(packed.tok_off.cpu().numpy(), hot_off[:-1]) and packed.hot_used == hot_off[-1]
        assert np.array_equal(packed.blob[: packed.hot_used].cpu().numpy(), hot), f"{kind}: hot tier bytes"
        assert np.array_equal(packed.cold_off.cpu().numpy(), cold_off[:-1])
        assert np.array_equal(packed.cold[: int(cold_off[-1])].cpu().numpy(), cold), f"{kind}: cold tier bytes"
        print(f"  {kind}: {middle} tokens' hot ({hot.size} B) and cold ({cold.size} B) tiers byte for byte",
              flush=True)
    # allocation: the reference rule over levels[floor:] on the GPU's float32 errors
    errors = codec.last_errors.float().cpu().numpy()
    levels = len(order.rungs)
    kept = [b for i, b in enumerate(codec.last_level_bytes) if i % levels >= floor]
    remaining = stored.budget_bytes - (tokens - middle) * 2 * codec.exact_bytes
    want = kvtc_ref.allocate_rungs(errors[:, floor:], np.array(kept), middle, remaining) + floor
    chosen = codec.last_chosen.cpu().numpy()
    assert np.array_equal(chosen, want)
    # and on the oracle's own errors: the level bytes are the reference's formula
    assert codec.last_level_bytes == pr.level_bytes(order) * 2
    own = np.concatenate(oracle_errors)
    np.testing.assert_allclose(errors, own, rtol=1e-4, atol=1e-12)
    want_own = kvtc_ref.allocate_rungs(own[:, floor:], np.array(kept), middle, remaining) + floor
    differ = int((want_own != chosen).sum())
    print(f"  allocation on the oracle's own error table: {differ} of {chosen.size} slots differ", flush=True)
    assert differ <= chosen.size // 200, f"{differ} slots differ from the allocation over the oracle's errors"
    orders = {"key": order, "value": order}
    pieces = {k: stored.stores[k].hot_pieces.cpu().numpy() for k in ("key", "value")}
    assert stored.hot_bytes == pr.hot_bytes(orders, pieces, tokens - middle, shape.exact_bytes)
    assert stored.cold_bytes == pr.cold_bytes(orders, pieces)
    assert stored.hot_bytes <= stored.budget_bytes
    print(f"  hot {stored.hot_bytes} B of budget {stored.budget_bytes} B, cold {stored.cold_bytes} B; "
          f"mean planes K {np.mean(pieces['key']) / shape.groups:.2f}, V {np.mean(pieces['value']) / shape.groups:.2f}",
          flush=True)
