"""Host-side logic of the Python mirrors (CPU): method-name parsing and its errors
(scripts/methods.py:100-108, 192-213, 227-236), checkpoint/model checks
(scripts/methods.py:134-137, scripts/progressive.py:119-120), the synthetic
checkpoints' consistency with the oracle, and the kvtc compress path (torch,
CPU) against the oracle's quantizer and allocator."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import synth
from oracle import kvtc_ref
from oracle import progressive_ref as pr


def test_budget_of():
    import methods

    assert methods.budget_of("full") == 1.0
    assert methods.budget_of("prog@0.03:r0.01") == 0.03
    assert methods.budget_of("dkvtc@0.02:snap:floor1") == 0.02
    assert methods.budget_of("dkv:0.15:flat") == 0.15
    assert np.isnan(methods.budget_of("pca16/lex8"))


def _small():
    shape = synth.ModelShape(2, 2, 64, 4, 256)
    ctx = synth.make_context(shape, 400, seed=3)
    return shape, ctx


def test_method_errors_follow_reference():
    import methods

    shape, ctx = _small()
    m = methods.Methods("synthetic/llama-3.2", device="cpu", model=synth.RopeModel(shape),
                        kvtc=synth.kvtc_checkpoint(ctx), progressive=synth.order_checkpoint(shape))
    keys, values = synth.prefill_cache(ctx, dtype=torch.float32)
    with pytest.raises(ValueError, match="not served"):
        m.apply("h2o:0.1", keys, values, {})
    with pytest.raises(ValueError, match="Unknown option"):
        m.apply("dkvtc@0.1:bogus", keys, values, {})
    with pytest.raises(ValueError, match="Unknown option"):
        m.apply("prog@0.1:zz", keys, values, {})
    with pytest.raises(ValueError, match="Unknown option"):
        m.apply("kvtc@0.1:ev", keys, values, {})  # :ev only with dkvtc (scripts/methods.py:200)
    other = methods.Methods("another/model", device="cpu", model=synth.RopeModel(shape),
                            kvtc=synth.kvtc_checkpoint(ctx), progressive=synth.order_checkpoint(shape))
    with pytest.raises(RuntimeError, match="was fit for"):
        other.codec("kvtc")
    nomodel = methods.Methods("synthetic/llama-3.2", device="cpu", kvtc=synth.kvtc_checkpoint(ctx))
    with pytest.raises(ValueError, match="model=model"):
        nomodel.codec("kvtc")


def test_progressive_order_mismatch_raises():
    import progressive

    shape, ctx = _small()
    order = synth.order_checkpoint(shape, model_id="other")
    with pytest.raises(RuntimeError, match="was fit for other"):
        progressive.ProgressiveCodec(synth.kvtc_checkpoint(ctx), order, "cpu", synth.RopeModel(shape))


def test_progressive_encode_refuses_a_cpu_codec():
    """The encoder's stages are HIP kernels: a codec built on the CPU says so instead of failing deep
    inside the binding."""
    import progressive

    shape, ctx = _small()
    codec = progressive.ProgressiveCodec(synth.kvtc_checkpoint(ctx), synth.order_checkpoint(shape), "cpu",
                                         synth.RopeModel(shape))
    keys, values = synth.prefill_cache(ctx, dtype=torch.float32)
    with pytest.raises(ValueError, match="runs on the GPU"):
        codec.encode(keys, values, 0.3, 8)


def test_synthetic_checkpoints_match_oracle_tables():
    shape, ctx = _small()
    order = synth.order_checkpoint(shape)["key"]
    ref = pr.plane_major_order(shape.groups)
    assert np.array_equal(order["planes"].numpy(), ref.planes)
    assert np.array_equal(order["prefix_bytes"].numpy().astype(np.int64), ref.prefix_bytes)
    assert order["rungs"] == ref.rungs
    ck = synth.kvtc_checkpoint(ctx)
    for bits, size in zip(ck["key"]["rungs"], ck["key"]["rung_bytes"]):
        assert size == kvtc_ref.rung_bytes(bits.numpy(), 64)


@pytest.mark.parametrize("name", ["kvtc@0.3", "kvtcf@0.3", "dkvtc@0.3:floor1", "dkvtc@0.3:snap:floor1", "dkvtc@0.2:ev"])
def test_kvtc_methods_on_cpu(name):
    """The kvtc family runs the reference's torch arithmetic (CPU here): rebuilt caches equal the
    oracle's quantize-dequantize of the chosen rungs, the budget holds, and exact tokens stay exact."""
    import kvtc
    import methods

    shape, ctx = _small()
    model = synth.RopeModel(shape)
    m = methods.Methods("synthetic/llama-3.2", device="cpu", model=model, kvtc=synth.kvtc_checkpoint(ctx))
    keys, values = synth.prefill_cache(ctx, dtype=torch.float32)
    tokens = keys[0].shape[2]
    scores = {"snap": [torch.rand(shape.kv_heads, tokens, generator=torch.Generator().manual_seed(l))
                       for l in range(shape.layers)]}
    out = m.apply(name, keys, values, scores)
    codec = m.codec("kvtc")
    budget = methods.budget_of(name)
    assert out.used_bytes <= int(budget * tokens * 2 * codec.exact_bytes)
    start, end = codec.last_span
    # bytes counted = exact tokens + every kept (token, stream) at its rung's oracle size
    want_bytes = (tokens - (end - start)) * 2 * codec.exact_bytes
    for kind in ("key", "value"):
        rungs = codec.streams[kind].rungs
        for level in codec.last_choice[kind].tolist():
            if level >= 0:
                want_bytes += (codec.exact_bytes if level == len(rungs)
                               else kvtc_ref.rung_bytes(rungs[level].numpy(), 64))
    assert out.used_bytes == want_bytes
    assert abs(sum(out.histogram.values()) - 1.0) < 1e-12
    assert set(out.histogram) <= {"evict", "exact"} | {f"{s / codec.exact_bytes:.3f}" for kind in ("key", "value")
                                                       for s in codec.streams[kind].rung_bytes}
    for layer in range(shape.layers):
        assert torch.equal(out.keys[layer][..., :start, :], keys[layer][..., :start, :])
        assert torch.equal(out.values[layer][..., end:, :], values[layer][..., end:, :])
    cos, sin = kvtc.rope_tables(model, tokens, "cpu")
    matrix = codec.to_matrix(values, "value", cos, sin)
    stream = codec.streams["value"]
    coef = ((matrix[start:end] - stream.mean) @ stream.basis).numpy()
    choice = codec.last_choice["value"].numpy()
    exact_rung = len(stream.rung_bytes)
    for r in np.unique(choice):
        rows = choice == r
        if r < 0:
            continue
        want = coef[rows] if r == exact_rung else kvtc_ref.quantize_groups(coef[rows], stream.rungs[r].numpy(), 64)
        got = codec.last_coefficients["value"][torch.from_numpy(rows)].numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"rung {r}"
    assert out.token_bytes.shape == (tokens,)


def test_ladder_tables_match_oracle():
    """Ladder segment offsets and rung sizes (scripts/kvtc.py:82-85) and the checks on bad tables."""
    import hot_tier
    from oracle import packing_ref

    bits = synth.ladder_rungs(8)
    sizes = [kvtc_ref.rung_bytes(b.numpy(), 64) for b in bits]
    t = hot_tier.LadderTables(bits, sizes, "cpu")
    assert t.rungs == len(bits) + 1 and t.empty == len(bits)
    assert np.array_equal(t.seg_off.numpy()[:-1], packing_ref.ladder_segment_offsets(bits.numpy()))
    assert np.array_equal(t.sizes64.numpy()[:-1], sizes) and int(t.sizes64[-1]) == 0
    with pytest.raises(ValueError, match="rung_bytes"):
        hot_tier.LadderTables(bits, [s + 4 for s in sizes], "cpu")
    with pytest.raises(ValueError, match="bit widths"):
        hot_tier.LadderTables(bits * 0 + 3, None, "cpu")
    with pytest.raises(ValueError, match="groups of 64"):
        hot_tier.LadderTables(bits, None, "cpu", group=32)


def test_threaded_deflate_is_one_zlib_stream():
    """kvtc_storage.deflate: one thread gives zlib.compress's bytes (the reference's stored form);
    several threads give one zlib stream of the same input, across piece boundaries and for inputs
    of at most one piece, with a size within a fraction of a percent."""
    import zlib

    import kvtc_storage

    rng = np.random.default_rng(3)
    piece = kvtc_storage.DEFLATE_PIECE
    big = (rng.integers(0, 16, 5 * piece + 123, dtype=np.uint8) * rng.integers(0, 2, 5 * piece + 123,
                                                                           dtype=np.uint8)).tobytes()
    assert kvtc_storage.deflate(big) == zlib.compress(big, 6)
    threaded = kvtc_storage.deflate(big, threads=4)
    assert zlib.decompress(threaded) == big
    assert kvtc_storage.inflate(threaded) == big
    assert len(threaded) < 1.002 * len(zlib.compress(big, 6))
    # a long repeat across a piece boundary is still found through the primed window
    rep = rng.integers(0, 256, 20_000, dtype=np.uint8).tobytes()
    crossing = bytes(piece - 10_000) + rep + rep
    assert zlib.decompress(kvtc_storage.deflate(crossing, threads=2)) == crossing
    for n in (0, 1, piece, piece + 1, 2 * piece):
        d = rng.integers(0, 4, n, dtype=np.uint8).tobytes()
        assert zlib.decompress(kvtc_storage.deflate(d, threads=3)) == d


def test_failed_refine_gives_back_slots_and_version():
    """``PackedStream.settle_refine``: the device kernel flags a row outside the stream and merges
    nothing, so the refine slots and the version bump that ``refine_async`` took are given back
    (whichever caller settles: ``refine`` or the question stage's gather of both streams)."""
    from hot_tier import PackedStream

    st = PackedStream.__new__(PackedStream)
    st.pieces = torch.zeros(10, dtype=torch.int16)
    st.refined, st.version = 12, 5  # as refine_async leaves them after taking 4 slots and one version
    with pytest.raises(ValueError, match="refine rows must lie in 0..9"):
        st.settle_refine(torch.tensor([0, 1]), 4)
    assert (st.refined, st.version) == (8, 4)
    assert st.settle_refine(torch.tensor([2176, 0]), 4) == 2176
    assert (st.refined, st.version) == (8, 4)


def test_exact_operand_and_mask_rows():
    """The hook hands the kernels a model cache's exact tokens in their own type when they are
    contiguous and aligned for four-element loads (float32 copies otherwise), and converts the
    additive mask once per mask tensor (again when the tensor changes in place or the key count does)."""
    import types

    from compressed_attention import CompressedContext, _exact_operand

    cache = torch.randn(1, 8, 40, 64, dtype=torch.float16)
    assert _exact_operand(cache[0]) is not None and _exact_operand(cache[0]).data_ptr() == cache.data_ptr()
    bf = cache.to(torch.bfloat16)
    assert _exact_operand(bf[0]).dtype == torch.bfloat16
    strided = cache[0, :, ::2]
    got = _exact_operand(strided)
    assert got.dtype == torch.float32 and got.is_contiguous() and torch.equal(got, strided.float())
    flat = torch.randn(8 * 40 * 64 + 1, dtype=torch.float16)
    shifted = flat[1:].view(8, 40, 64)  # 2-byte offset: not aligned for 8-byte loads
    assert _exact_operand(shifted).dtype == torch.float32
    assert _exact_operand(torch.randn(2, 3, 4, dtype=torch.float64)).dtype == torch.float32

    ctx = types.SimpleNamespace(_mask_cache=None)
    mask = torch.zeros(1, 1, 2, 50, dtype=torch.float16)
    mask[..., -1] = -1e4
    rows = CompressedContext._mask_rows(ctx, mask, 40)
    assert rows.dtype == torch.float32 and rows.shape == (2, 40) and torch.equal(rows, mask[0, 0, :, -40:].float())
    assert CompressedContext._mask_rows(ctx, mask, 40) is rows  # every layer of one forward: converted once
    mask[..., -2] = -1e4  # changed in place: converted again
    again = CompressedContext._mask_rows(ctx, mask, 40)
    assert again is not rows and float(again[0, -2]) == -1e4
    assert CompressedContext._mask_rows(ctx, mask, 41).shape == (2, 41)
    other = mask.clone()
    assert CompressedContext._mask_rows(ctx, other, 41) is not CompressedContext._mask_rows(ctx, mask, 41)


def test_exact_offsets_keep_the_last_few():
    """cu_exact arrays are made once per exact-tail length and only the last eight lengths are kept
    (a long reply adds one length per token)."""
    import types

    from compressed_attention import CompressedContext

    ctx = types.SimpleNamespace(key=types.SimpleNamespace(blob=torch.zeros(1)), _cu_exact={})
    first = CompressedContext._exact_offsets(ctx, (37,))
    assert CompressedContext._exact_offsets(ctx, (37,)) is first
    for n in range(38, 60):
        host, dev = CompressedContext._exact_offsets(ctx, (n,))
        assert host.tolist() == [0, n] and dev.tolist() == [0, n]
    assert len(ctx._cu_exact) == 8 and (37,) not in ctx._cu_exact
    host, _ = CompressedContext._exact_offsets(ctx, (3, 4, 5))
    assert host.tolist() == [0, 3, 7, 12]
