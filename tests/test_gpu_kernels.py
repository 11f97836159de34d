"""GPU parity of the HIP kernels (through the C ABI) against the oracle on seeded inputs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import synth
from helpers import assert_close, assert_sensitive, build_case, gpu_attend, gpu_context, oracle_attend, value_mean_base
from oracle import packing_ref, progressive_ref as pr

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _random_order(groups: int, seed: int) -> pr.Order:
    """A non-plane-major order: a random interleaving of every group's 8 planes."""
    rng = np.random.default_rng(seed)
    seq = np.repeat(np.arange(groups), 8)
    rng.shuffle(seq)
    return pr.order_from_sequence(list(seq), groups)


@pytest.mark.parametrize("order_kind", ["plane_major", "random"])
def test_pack_unpack_bit_exact(order_kind):
    from hot_tier import OrderTables, PackedStream

    print(f"[case] pack/unpack order={order_kind}", flush=True)
    groups, n = 4, 97
    order = pr.plane_major_order(groups) if order_kind == "plane_major" else _random_order(groups, 3)
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((n, groups * 64)) * rng.uniform(0.01, 2.0, size=(n, 1))).astype(np.float32)
    codes, low, span = pr.quantize8(x, 64)
    pieces = rng.integers(0, order.pieces + 1, size=n)
    pieces[:5] = [0, order.pieces, 1, groups, order.pieces - 1]
    hot_ref, hot_off_ref, cold_ref, cold_off_ref = packing_ref.pack(codes, low, span, pieces, order)
    tables = OrderTables(order.planes, order.prefix_bytes, DEV)
    st = PackedStream.pack(torch.from_numpy(codes).to(DEV), torch.from_numpy(low).to(DEV),
                           torch.from_numpy(span).to(DEV), torch.from_numpy(pieces).to(DEV), tables,
                           refine_capacity=n)
    torch.cuda.synchronize()
    assert np.array_equal(st.tok_off.cpu().numpy(), hot_off_ref[:-1])
    assert np.array_equal(st.blob[: st.hot_used].cpu().numpy(), hot_ref)
    assert np.array_equal(st.cold[: int(cold_off_ref[-1])].cpu().numpy(), cold_ref)
    # byte totals = reference accounting (progressive.py:185-194)
    assert st.hot_bytes() == int(order.prefix_bytes[pieces].sum()) + n
    assert st.cold_bytes() == int((order.prefix_bytes[-1] - order.prefix_bytes[pieces]).sum())
    # K1 (fp32) is bit-identical to the reference dequantize at the hot planes
    planes = pr.token_planes(order, pieces)
    ref = pr.dequantize(codes, low, span, planes)
    got = st.dequantize(dtype=torch.float32).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # the oracle unpacker agrees with the GPU-packed bytes
    c2, l2, s2, p2 = packing_ref.unpack(st.blob.cpu().numpy(), st.tok_off.cpu().numpy(), pieces, order, groups)
    assert np.array_equal(pr.dequantize(c2, l2, s2, p2).view(np.uint32), ref.view(np.uint32))
    # K4c: refine a set of rows -> full precision for them, fetched = reference formula
    rows = np.array([0, 2, 5, 17, 40, 96])
    fetched = st.refine(torch.from_numpy(rows).to(DEV))
    assert fetched == int((order.prefix_bytes[-1] - order.prefix_bytes[pieces[rows]]).sum())
    pieces2 = pieces.copy()
    pieces2[rows] = order.pieces
    ref2 = pr.dequantize(codes, low, span, pr.token_planes(order, pieces2))
    got2 = st.dequantize(dtype=torch.float32).cpu().numpy()
    assert np.array_equal(got2.view(np.uint32), ref2.view(np.uint32))


def test_dequantize_codes_exhaustive():
    """Reference dequantize on unpacked codes: every code x every plane count, bit-exact."""
    from progressive import dequantize

    print("[case] dequantize exhaustive", flush=True)
    rng = np.random.default_rng(11)
    n, groups = 9 * 8, 4
    codes = np.tile(np.arange(256, dtype=np.uint8), n * groups // 4).reshape(n, groups, 64)
    low = rng.standard_normal((n, groups)).astype(np.float16)
    span = np.abs(rng.standard_normal((n, groups))).astype(np.float16) + np.float16(1e-3)
    planes = np.repeat(np.arange(9, dtype=np.uint8), 8)[:, None].repeat(groups, axis=1)
    ref = pr.dequantize(codes, low, span, planes)
    got = dequantize(torch.from_numpy(codes).to(DEV), torch.from_numpy(low).to(DEV),
                     torch.from_numpy(span).to(DEV), torch.from_numpy(planes).to(DEV)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("shape_name,tokens,layers,query_scale,q_len,qdtype", [
    ("1b", 1500, (0, 7, 15), 1.0, 1, "float32"),    # 1500-token 1B shape, N(0,1) query
    ("1b", 1500, (3,), 150.0, 1, "float32"),        # peaked attention
    ("3b2", 900, (0, 1), 120.0, 1, "float32"),      # head_dim 128 path
    ("3b2", 700, (1,), 120.0, 5, "float32"),        # q_len > 1 with a causal exact part
    ("3b2", 700, (0,), 120.0, 5, "bfloat16"),       # many-row epilogue, per query type
    ("1b", 900, (2,), 150.0, 3, "float16"),
    # one KV head per K2 workgroup with 1, 2 and 4 query rows per KV head (GQA groups of 1 and 2)
    ("mha64", 700, (0, 1), 120.0, 1, "float32"),
    ("mha64", 700, (1,), 120.0, 4, "bfloat16"),
    ("gq2_128", 900, (0,), 120.0, 1, "float16"),
    ("gq2_128", 700, (1,), 120.0, 2, "float32"),
])
def test_attend_matches_oracle(shape_name, tokens, layers, query_scale, q_len, qdtype):
    shape = {"1b": synth.SHAPE_1B, "3b2": synth.ModelShape(2, 8, 128, 24, 2048),
             "mha64": synth.ModelShape(2, 8, 64, 8, 1024), "gq2_128": synth.ModelShape(2, 8, 128, 16, 2048)}[shape_name]
    print(f"[case] attend {shape_name} T={tokens} scale={query_scale} q_len={q_len} {qdtype}", flush=True)
    case = build_case(shape, tokens, seed=1234, query_scale=query_scale, q_len=q_len,
                      query_dtype=getattr(torch, qdtype))
    ctx, _, _ = gpu_context(case)
    for layer in layers:
        ref = oracle_attend(case, layer)
        got = gpu_attend(case, ctx, layer)
        err, fro = assert_close(got, ref, what=f"layer {layer}", base=value_mean_base(case, layer))
        print(f"  layer {layer}: max abs err {err:.2e}, rel fro {fro:.2e}", flush=True)


@pytest.mark.parametrize("shape_name,tokens,sinks,recent,q_len", [
    ("3b2", 600, 0, 2, 1),      # 3 exact tokens: one per share, the fourth share empty
    ("3b2", 900, 4, 300, 1),    # 305: every share past its first round of keys and of values
    ("1b", 1400, 4, 1000, 1),   # 1,005 of the 1,024 allowed: 252 per share
    ("1b", 800, 2, 200, 3),     # 205 with a causal mask across the shares
])
def test_attend_exact_tail_lengths(shape_name, tokens, sinks, recent, q_len):
    """The exact tail's token shares (four per output row, merged by the finish kernel) at lengths
    the 37-token default never reaches; with a long tail, zeroing its values must move the oracle's
    output far past the bar, so the tail is what the check sees."""
    shape = {"1b": synth.SHAPE_1B, "3b2": synth.ModelShape(2, 8, 128, 24, 2048)}[shape_name]
    print(f"[case] exact tail {shape_name} T={tokens} sinks={sinks} recent={recent} q_len={q_len}", flush=True)
    case = build_case(shape, tokens, seed=4321, query_scale=20.0, q_len=q_len, sinks=sinks, recent=recent)
    ctx, _, _ = gpu_context(case)
    layer = shape.layers - 1
    ref = oracle_attend(case, layer)
    got = gpu_attend(case, ctx, layer)
    base = value_mean_base(case, layer)
    err, fro = assert_close(got, ref, what=f"exact tail E={case.key_exact.shape[2]}", base=base)
    print(f"  E={case.key_exact.shape[2]}: max abs err {err:.2e}, rel fro {fro:.2e}", flush=True)
    if recent >= 100:
        from dataclasses import replace

        zeroed = oracle_attend(replace(case, value_exact=torch.zeros_like(case.value_exact)), layer)
        gap = assert_sensitive(ref, zeroed, base, what="exact values zeroed")
        print(f"  zeroed exact values move the output by {gap:.2e} (relative)", flush=True)


def test_stream_handle_is_torch_current_stream():
    """The launch stream the bindings pass (torch's raw-stream accessor) is torch's current stream,
    also inside a ``torch.cuda.stream`` block."""
    import dkv_hip

    assert dkv_hip.stream_handle() == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert dkv_hip.stream_handle() == side.cuda_stream == torch.cuda.current_stream().cuda_stream
    assert dkv_hip.stream_handle() == torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_attend_exact_tail_in_cache_type(dtype):
    """The exact tail read in the model cache's own type (exact_dtype f16 / bf16, converted to float32
    as the kernels load it) gives the float32 path's output bit for bit, through the C ABI directly and
    through the attention hook, which now passes an fp16 / bf16 cache on as it is."""
    import types

    shape = synth.ModelShape(2, 8, 128, 24, 2048)
    print(f"[case] exact tail in {dtype}: 3B heads, T=900, 305 exact tokens, q_len=2", flush=True)
    case = build_case(shape, 900, seed=4322, query_scale=20.0, q_len=2, sinks=4, recent=300)
    ctx, _, _ = gpu_context(case)
    layer = 1
    q = case.queries[layer].to(DEV).contiguous()
    ke = case.key_exact[layer].to(DEV, dtype).contiguous()
    ve = case.value_exact[layer].to(DEV, dtype).contiguous()
    mask = case.mask.to(DEV).contiguous()
    outs = []
    for k, v in ((ke, ve), (ke.float(), ve.float())):
        out = torch.empty(1, case.q_len, shape.q_heads, shape.head_dim, device=DEV)
        args = ctx.layer_args(layer, q, out, k, v, mask)
        assert args.exact_dtype == (0 if k.dtype == torch.float32 else 1 if k.dtype == torch.float16 else 2)
        ctx.run_layer(args)
        outs.append(out)
    # the hook: key / value as a model cache hands them over ([1, Hkv, E, d]) with an additive mask
    module = types.SimpleNamespace(layer_idx=layer, num_key_value_groups=shape.q_heads // shape.kv_heads)
    hook_out, _ = ctx.attend(module, q.to(dtype), ke[None], ve[None], mask[None, None], None)
    ref_out = torch.empty(1, case.q_len, shape.q_heads, shape.head_dim, dtype=dtype, device=DEV)
    ctx.run_layer(ctx.layer_args(layer, q.to(dtype), ref_out, ke.float(), ve.float(), mask))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]), f"{dtype} exact tail differs from its float32 copy"
    assert torch.equal(hook_out, ref_out), "the hook's cache-type exact tail differs from the float32 path"
    from dataclasses import replace

    rounded = replace(case, key_exact=case.key_exact.to(dtype).float(), value_exact=case.value_exact.to(dtype).float())
    ref = oracle_attend(rounded, layer)  # the oracle over the same (rounded) exact tokens
    err, _ = assert_close(outs[0].cpu().numpy(), ref, what=f"exact tail in {dtype}", base=value_mean_base(case, layer))
    print(f"  bit-identical to float32; max abs err vs oracle {err:.2e}", flush=True)


def test_attend_special_cases():
    """Closed forms: all tokens at 0 planes and no exact part -> output = mean_v;
    a zero query -> the plain average of the decoded values."""
    from oracle import attention_ref

    print("[case] attend special cases", flush=True)
    shape = synth.ModelShape(2, 8, 64, 16, 1024)
    case = build_case(shape, 600, seed=99, zero_frac=1.0, query_scale=50.0)
    ctx, _, _ = gpu_context(case)
    q = case.queries[0].to(DEV).contiguous()
    out = torch.empty(1, 1, shape.q_heads, shape.head_dim, device=DEV)
    args = ctx.layer_args(0, q, out)
    ctx.run_layer(args)
    torch.cuda.synchronize()
    expect = value_mean_base(case, 0)
    assert np.allclose(out.cpu().numpy(), expect, atol=1e-6, rtol=1e-5)
    # zero query: uniform weights over compressed + exact tokens
    case2 = build_case(shape, 600, seed=98, query_scale=0.0)
    ctx2, _, _ = gpu_context(case2)
    got = gpu_attend(case2, ctx2, 1)
    ref = attention_ref.decode_then_attend_f64(
        case2.queries[1].numpy(), case2.coef_hot["key"], case2.coef_hot["value"], case2.layer_slice("key", 1),
        case2.layer_slice("value", 1), case2.mean_slice("key", 1), case2.mean_slice("value", 1),
        case2.cos[case2.positions].numpy(), case2.sin[case2.positions].numpy(), case2.key_exact[1][None].numpy(),
        case2.value_exact[1][None].numpy())
    assert_close(got, ref, what="zero query", base=value_mean_base(case2, 1))


def test_attend_with_no_compressed_tokens():
    """A 36-token conversation (4 sinks + 32 recent) leaves nothing to compress: the kernels skip the
    compressed part and the output is attention over the exact tokens alone."""
    shape = synth.ModelShape(2, 8, 64, 32, 1024)
    print("[case] attend with no compressed tokens", flush=True)
    case = build_case(shape, 36, seed=97, query_scale=40.0)
    assert case.ctx.middle == 0
    ctx, _, _ = gpu_context(case)
    for layer in range(shape.layers):
        got = gpu_attend(case, ctx, layer)
        err, fro = assert_close(got, oracle_attend(case, layer), what=f"all-exact layer {layer}",
                                base=value_mean_base(case, layer))
        print(f"  layer {layer}: max abs err {err:.2e}, rel fro {fro:.2e}", flush=True)


def test_topk_exact():
    import dkv_hip
    from oracle import scoring_ref

    print("[case] topk", flush=True)
    rng = np.random.default_rng(5)
    # 40,000 > 32 x 1,024 elements: the kernel reloads them from memory instead of its register cache
    for n, k in [(16348, 163), (1000, 1), (777, 777), (5000, 64), (40000, 400), (2048, 100)]:
        s = rng.standard_normal(n).astype(np.float32)
        s[rng.integers(0, n, 50)] = s[0]  # ties resolve by lower index
        if n == 2048:
            s[:] = 0.25  # every key equal: the lowest k indices
        out = torch.empty(k, dtype=torch.int32, device=DEV)
        dkv_hip.topk(torch.from_numpy(s).to(DEV), k, out)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), scoring_ref.topk_indices(s, k)), (n, k)
