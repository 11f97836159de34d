"""GPU parity of the kvtc-ladder path (the ``dkvtc@`` entry point) against the oracle.

- pack: dkv_pack_ladder's token blobs equal oracle/packing_ref.pack_ladder byte for byte;
- K1: dkv_unpack_dequant over ladder blobs equals code * scale + low (scripts/kvtc.py:78) bit for
  bit in float32 (hence scripts/kvtc.py:62-79 quantize_groups' output), and its fp16 cast (the
  coefficient blocks of scripts/compressed_attention.py:71-77) in float16;
- attention: ``CompressedContext(codec, keys, values, model)`` (scripts/compressed_attention.py:34-89)
  after ``Methods.apply("dkvtc@<b>:snap:floor1")`` matches the oracle's attention over
  ``codec.last_coefficients`` within max-abs 2e-3 / rel 1e-2, with tokens at the exact rung,
  evicted keys (left out) and evicted values (decoding to the mean).
"""

from __future__ import annotations

import types

import numpy as np
import pytest
import torch

import synth
from helpers import assert_close
from oracle import attention_ref, kvtc_ref, packing_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_ladder_pack_and_unpack_bit_exact():
    from hot_tier import LadderStream, LadderTables

    print("[case] ladder pack/unpack G=8 n=777", flush=True)
    rng = np.random.default_rng(21)
    groups, n = 8, 777
    bits = synth.ladder_rungs(groups).numpy()
    rungs = bits.shape[0]
    x = (rng.standard_normal((n, groups * 64)) * np.repeat(np.linspace(4.0, 0.01, groups), 64)).astype(np.float32)
    rung = rng.integers(-1, rungs, n)  # -1: every group dropped
    codes = np.zeros((n, groups, 64), np.uint8)
    low = np.zeros((n, groups), np.float16)
    scale = np.zeros((n, groups), np.float16)
    for r in range(rungs):
        rows = rung == r
        codes[rows], low[rows], scale[rows] = kvtc_ref.quantize_groups_codes(x[rows], bits[r], 64)
    tables = LadderTables(bits, [kvtc_ref.rung_bytes(b, 64) for b in bits], DEV)
    stream = LadderStream.pack(torch.from_numpy(codes).to(DEV), torch.from_numpy(low).to(DEV),
                               torch.from_numpy(scale).to(DEV), torch.from_numpy(rung).to(DEV), tables)
    eff_bits = np.concatenate([bits, np.zeros((1, groups), bits.dtype)])
    eff_rung = np.where(rung < 0, rungs, rung)
    blob, off = packing_ref.pack_ladder(codes, low, scale, eff_rung, eff_bits)
    torch.cuda.synchronize()
    assert np.array_equal(stream.tok_off.cpu().numpy(), off[:-1])
    assert stream.hot_bytes() == int(off[-1])
    assert np.array_equal(stream.blob[: off[-1]].cpu().numpy(), blob)
    want = kvtc_ref.dequantize_codes(codes, low, scale, eff_bits[eff_rung])
    for r in range(rungs):  # the stored codes reproduce the reference quantize-dequantize
        rows = rung == r
        assert np.array_equal(want[rows].view(np.uint32), kvtc_ref.quantize_groups(x[rows], bits[r], 64).view(np.uint32))
    assert not want[rung < 0].any()
    got = stream.dequantize().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = stream.dequantize(dtype=torch.float16).cpu().numpy()
    assert np.array_equal(got16.view(np.uint16), want.astype(np.float16).view(np.uint16))
    part = stream.dequantize(100, 50).cpu().numpy()
    assert np.array_equal(part.view(np.uint32), want[100:150].view(np.uint32))


def _dkvtc_case(name, seed, tokens=1500, edits=False):
    import kvtc
    import methods
    from compressed_attention import CompressedContext

    # 2 layers only, so a token's exact bytes (2 KiB) are small beside the ladder's rungs: the
    # budgets are set high enough for the coarsest rung
    shape = synth.ModelShape(2, 8, 64, 32, 1024)
    ctx = synth.make_context(shape, tokens, seed=seed)
    model = synth.RopeModel(shape, DEV)
    m = methods.Methods("synthetic/llama-3.2", device=DEV, model=model, kvtc=synth.kvtc_checkpoint(ctx))
    keys, values = synth.prefill_cache(ctx, device=DEV, dtype=torch.float16)
    g = torch.Generator("cpu").manual_seed(seed + 1)
    scores = {"snap": [torch.rand(shape.kv_heads, tokens, generator=g).to(DEV) for _ in range(shape.layers)]}
    m.apply(name, keys, values, scores)
    codec = m.codec("kvtc")
    start, end = codec.last_span
    if edits:
        # force the rarer cases: exact-rung keys and values, evicted keys, evicted values
        cos, sin = kvtc.rope_tables(model, tokens, DEV)
        for kind, tensors, rows in (("key", keys, [3, 77, 500]), ("value", values, [77, 901, 1200])):
            stream = codec.streams[kind]
            exact = (codec.to_matrix(tensors, kind, cos, sin)[start:end] - stream.mean) @ stream.basis
            idx = torch.tensor(rows, device=DEV)
            codec.last_coefficients[kind][idx] = exact[idx]
            codec.last_choice[kind][idx] = len(stream.rung_bytes)
        hidden = torch.tensor([10, 11, 640], device=DEV)
        codec.last_choice["key"][hidden] = -1
        codec.last_choice["value"][hidden] = -1
        dropped = torch.tensor([12, 13, 1000], device=DEV)
        codec.last_choice["value"][dropped] = -1
        codec.last_coefficients["value"][dropped] = 0.0
    context = CompressedContext(codec, keys, values, model)
    return shape, ctx, model, codec, keys, values, context


@pytest.mark.parametrize("name,seed,edits", [
    ("dkvtc@0.2:snap:floor1", 31, False),
    ("dkvtc@0.5:snap:floor1", 32, False),  # floor at the finest rung: many exact-rung tokens
    ("dkvtc@0.2:snap:floor1", 33, True),
])
def test_dkvtc_context_matches_oracle(name, seed, edits):
    import kvtc

    print(f"[case] {name} seed={seed} edits={edits}", flush=True)
    shape, ctx, model, codec, keys, values, context = _dkvtc_case(name, seed, edits=edits)
    tokens = keys[0].shape[2]
    start, end = codec.last_span
    choice = {k: codec.last_choice[k].cpu().numpy() for k in ("key", "value")}
    kept = choice["key"] >= 0
    exact_rung = len(codec.streams["key"].rung_bytes)
    promoted = kept & ((choice["key"] == exact_rung) | (choice["value"] == len(codec.streams["value"].rung_bytes)))
    coded = kept & ~promoted
    assert context.key.n == int(coded.sum())
    # byte accounting: each coded token holds its rung's bytes (scripts/kvtc.py:243)
    for kind in ("key", "value"):
        sizes = np.array(codec.streams[kind].rung_bytes + [0])
        c = choice[kind][coded]
        assert context.__dict__[kind].hot_bytes() == int(sizes[np.where(c < 0, len(sizes) - 1, c)].sum())
    if edits:
        assert promoted.sum() >= 5 and (~kept).sum() == 3
    coef = {k: codec.last_coefficients[k].float().cpu().numpy()[kept] for k in ("key", "value")}
    cos, sin = kvtc.rope_tables(model, tokens, DEV)
    pos = np.nonzero(kept)[0] + start
    cos_k, sin_k = cos.cpu().numpy()[pos], sin.cpu().numpy()[pos]
    w = shape.kv_heads * shape.head_dim
    g = torch.Generator("cpu").manual_seed(seed + 2)
    for layer in range(shape.layers):
        q = (torch.randn(1, shape.q_heads, 1, shape.head_dim, generator=g) * 30.0).to(DEV)
        exact = context.exact_cache.layers[layer]
        ke, ve = exact.keys, exact.values  # [1, Hkv, E, d] fp16
        e_len = ke.shape[2]
        mask = torch.zeros(1, 1, 1, e_len, device=DEV)
        mask[..., 1] = -1e9  # one sink hidden by the additive mask
        module = types.SimpleNamespace(layer_idx=layer, num_key_value_groups=shape.gqa)
        out, none = context.attend(module, q, ke, ve, mask, shape.head_dim ** -0.5)
        torch.cuda.synchronize()
        assert none is None and out.shape == (1, 1, shape.q_heads, shape.head_dim)
        basis = {k: codec.streams[k].basis[layer * w:(layer + 1) * w].T.cpu().numpy() for k in ("key", "value")}
        mean = {k: codec.streams[k].mean[layer * w:(layer + 1) * w].cpu().numpy() for k in ("key", "value")}
        ref = attention_ref.attend(q.cpu().numpy(), coef["key"], coef["value"], basis["key"], basis["value"],
                                   mean["key"], mean["value"], cos_k, sin_k, ke.float().cpu().numpy(),
                                   ve.float().cpu().numpy(), mask.cpu().numpy())
        base = np.broadcast_to(np.repeat(mean["value"].reshape(shape.kv_heads, 1, -1), shape.gqa, axis=1)
                               .reshape(1, 1, shape.q_heads, -1), ref.shape)
        err, fro = assert_close(out.float().cpu().numpy(), ref, what=f"{name} layer {layer}", base=base)
        print(f"  layer {layer}: coded {int(coded.sum())}, exact-rung {int(promoted.sum())}, "
              f"max abs err {err:.2e}, rel fro {fro:.2e}", flush=True)


def test_compress_choice_matches_oracle_at_full_size():
    """KVTCCodec.compress's per-token rungs for dkvtc@0.03:snap:floor1 at the 3B shape with 16,384
    tokens (span, budget split, relative errors over the stream energy, snap weights, the floor at
    the finest affordable uniform rung, allocation over the levels from the floor up) against
    oracle.kvtc_ref.compress_choice on the same token matrices and projections.  The two sum
    float32 errors in different orders, so a slot may differ where two upgrade values tie to the
    last bits; those slots are counted and must stay rare."""
    import kvtc
    import methods
    from oracle import kvtc_ref

    shape, tokens = synth.SHAPE_3B, 16384
    print("[case] compress choice, dkvtc@0.03:snap:floor1, 3B shape, 16384 tokens", flush=True)
    ctx = synth.make_context(shape, tokens, 2024, device=DEV)
    model = synth.RopeModel(shape, DEV)
    keys, values = synth.prefill_cache(ctx, device=DEV, dtype=torch.float16, compute_device=DEV)
    g = torch.Generator("cpu").manual_seed(2104)
    scores = {"snap": [torch.rand(shape.kv_heads, tokens, generator=g).to(DEV) for _ in range(shape.layers)]}
    m = methods.Methods("synthetic/llama-3.2", device=DEV, model=model, kvtc=synth.kvtc_checkpoint(ctx))
    m.apply("dkvtc@0.03:snap:floor1", keys, values, scores)
    codec = m.codec("kvtc")
    cos, sin = kvtc.rope_tables(model, tokens, DEV)
    start, end = codec.last_span
    st = codec.streams
    mats, coefs = {}, {}
    for kind, t in (("key", keys), ("value", values)):
        mat = codec.to_matrix(t, kind, cos, sin)
        coefs[kind] = ((mat[start:end] - st[kind].mean) @ st[kind].basis).cpu().numpy()
        mats[kind] = mat.cpu().numpy()
        del mat
    weights = torch.stack(scores["snap"]).sum(dim=(0, 1)).cpu().numpy()
    want = kvtc_ref.compress_choice(
        mats, {k: st[k].mean.cpu().numpy() for k in st}, {k: st[k].basis.cpu().numpy() for k in st},
        {k: st[k].rungs.cpu().numpy() for k in st}, {k: st[k].rung_bytes for k in st}, codec.exact_bytes,
        codec.sinks, m.recent, 0.03, codec.group, weights=weights, floor_share=1.0, coefficients=coefs)
    assert want["span"] == (start, end)
    differ, slots = 0, 0
    for kind in ("key", "value"):
        got = codec.last_choice[kind].cpu().numpy()
        assert (got >= want["first"]).all(), f"{kind}: a token below the floor"
        differ += int((got != want[kind]).sum())
        slots += got.size
    hist = np.bincount(want["key"] + 1)
    print(f"  floor level {want['first']}; oracle key rungs (from -1) {hist.tolist()}; "
          f"{differ} of {slots} slots differ from the oracle", flush=True)
    assert differ <= slots // 200
