"""GPU parity of kvtc byte storage (scripts/kvtc_storage.py) against the oracle.

- ``encode_bytes`` on the GPU equals oracle/storage_ref.encode byte for byte, given the codec's
  coefficients, matrix rows and exact tokens;
- the codes ``decode_bytes`` / ``restore_context`` unpack on the GPU dequantize bit for bit to the
  oracle's decode;
- the reference's own check (FINDINGS.md:468-469): the cache ``decode_bytes`` restores equals the
  one ``KVTCCodec.compress`` returned, bit for bit when no token sits at the exact rung (with
  exact-rung tokens their stored fp16 rows replace the codec's float32 reconstruction, and the other
  tokens agree to float32 rounding);
- ``restore_context`` rebuilds ladder streams byte-identical to the in-memory
  ``CompressedContext``'s and answers identically (bit for bit without exact-rung tokens);
- at the 3b-16k-3pct workload (Llama-3.2-3B shape, 16,384 tokens, dkvtc@0.03:snap:floor1) the bytes survive
  DEFLATE and restore to byte-identical streams; encode / restore timings are printed.
"""

from __future__ import annotations

import time
import types

import numpy as np
import pytest
import torch

import synth
from oracle import storage_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(name: str, seed: int, shape=None, tokens: int = 1500):
    import methods

    shape = shape or synth.ModelShape(2, 8, 64, 32, 1024)
    ctx = synth.make_context(shape, tokens, seed=seed, device=DEV)
    model = synth.RopeModel(shape, DEV)
    m = methods.Methods("synthetic/llama-3.2", device=DEV, model=model, kvtc=synth.kvtc_checkpoint(ctx))
    keys, values = synth.prefill_cache(ctx, device=DEV, dtype=torch.float16, compute_device=DEV)
    g = torch.Generator("cpu").manual_seed(seed + 1)
    scores = {"snap": [torch.rand(shape.kv_heads, tokens, generator=g).to(DEV) for _ in range(shape.layers)]}
    compressed = m.apply(name, keys, values, scores)
    return shape, model, m, m.codec("kvtc"), keys, values, compressed


def _oracle_streams(codec, keys, values, model, recent):
    import kvtc

    tokens = keys[0].shape[2]
    start, end = codec.middle_span(tokens, recent)
    cos, sin = kvtc.rope_tables(model, tokens, DEV)
    streams, metas = [], []
    for kind, tensors in (("key", keys), ("value", values)):
        stream = codec.streams[kind]
        matrix = codec.to_matrix(tensors, kind, cos, sin)
        coef = (matrix[start:end] - stream.mean) @ stream.basis
        exact = kvtc.token_matrix(tensors)
        streams.append({"rungs": codec.last_choice[kind].cpu().numpy(), "bits": stream.rungs.cpu().numpy(),
                        "coefficients": coef.cpu().numpy(), "matrix_rows": matrix[start:end].cpu().numpy(),
                        "exact_tokens": torch.cat([exact[:start], exact[end:]]).cpu().numpy(),
                        "features": matrix.shape[1]})
        metas.append({"bits": stream.rungs.cpu().numpy(), "rank": stream.basis.shape[1], "features": matrix.shape[1]})
    return tokens, start, end, streams, metas


@pytest.mark.parametrize("name,seed", [("dkvtc@0.2:snap:floor1", 41), ("dkvtc@0.5:snap:floor1", 42)])
def test_encode_decode_match_oracle_and_compress(name, seed):
    import kvtc_storage

    print(f"[case] storage {name} seed={seed}", flush=True)
    shape, model, m, codec, keys, values, compressed = _case(name, seed)
    data = kvtc_storage.encode_bytes(codec, keys, values, codec.last_choice, m.recent)
    tokens, start, end, streams, metas = _oracle_streams(codec, keys, values, model, m.recent)
    want = storage_ref.encode(tokens, start, end, streams, codec.group)
    assert len(data) == len(want) == storage_ref.stored_bytes(tokens, end - start, streams, codec.group)
    diff = np.nonzero(np.frombuffer(data, np.uint8) != np.frombuffer(want, np.uint8))[0]
    assert diff.size == 0, f"{diff.size} bytes differ, first at {diff[:5]}"
    # the codes unpacked on the GPU dequantize to the oracle's decode, bit for bit
    parsed = kvtc_storage._Parsed(codec, data)
    ref = storage_ref.decode(data, metas, codec.group)
    for kind, o in zip(("key", "value"), ref["streams"]):
        got = parsed.coefficients(kind).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), o["coefficients"].view(np.uint32)), kind
        assert np.array_equal(parsed.choice[kind].cpu().numpy(), o["rungs"])
    # restored cache vs the codec's compressed cache
    rk, rv = kvtc_storage.decode_bytes(codec, data)
    exact_rung = len(codec.streams["key"].rung_bytes)
    n_exact = {k: int((codec.last_choice[k] == exact_rung).sum()) for k in ("key", "value")}
    print(f"  {len(data)} B, exact-rung tokens {n_exact}, deflated {len(kvtc_storage.deflate(data))} B", flush=True)
    for kind, got, mem in (("key", rk, compressed.keys), ("value", rv, compressed.values)):
        for layer, (a, b) in enumerate(zip(got, mem)):
            assert a.shape == b.shape and a.dtype == b.dtype
            if n_exact["key"] == 0 and n_exact["value"] == 0:
                assert torch.equal(a, b), f"{kind} layer {layer}"
            else:
                err = float((a.float() - b.float()).abs().max())
                assert err <= 2e-2 * float(b.float().abs().max()), f"{kind} layer {layer}: {err}"
            assert torch.equal(a[..., :start, :], b[..., :start, :]) and torch.equal(a[..., end:, :], b[..., end:, :])


@pytest.mark.parametrize("name,seed", [("dkvtc@0.2:snap:floor1", 43), ("dkvtc@0.5:snap:floor1", 44)])
def test_restore_context_matches_in_memory(name, seed):
    import kvtc_storage
    from compressed_attention import CompressedContext

    print(f"[case] restore_context {name} seed={seed}", flush=True)
    shape, model, m, codec, keys, values, compressed = _case(name, seed)
    data = kvtc_storage.encode_bytes(codec, keys, values, codec.last_choice, m.recent)
    mem = CompressedContext(codec, keys, values, model)
    got = kvtc_storage.restore_context(codec, kvtc_storage.inflate(kvtc_storage.deflate(data)), model)
    for kind in ("key", "value"):
        a, b = getattr(got, kind), getattr(mem, kind)
        assert a.n == b.n and a.used == b.used
        assert torch.equal(a.blob[:a.used], b.blob[:b.used]) and torch.equal(a.tok_off, b.tok_off)
        assert torch.equal(a.pieces, b.pieces)
    assert torch.equal(got.positions, mem.positions)
    for layer in range(shape.layers):
        ea, eb = got.exact_cache.layers[layer], mem.exact_cache.layers[layer]
        assert torch.equal(ea.keys, eb.keys) and torch.equal(ea.values, eb.values)
    promoted = (mem.extra is not None)
    g = torch.Generator("cpu").manual_seed(seed + 5)
    for layer in range(shape.layers):
        q = (torch.randn(1, shape.q_heads, 1, shape.head_dim, generator=g) * 20.0).to(DEV)
        module = types.SimpleNamespace(layer_idx=layer, num_key_value_groups=shape.gqa)
        outs = []
        for c in (got, mem):
            ex = c.exact_cache.layers[layer]
            out, _ = c.attend(module, q, ex.keys, ex.values, None, shape.head_dim ** -0.5)
            outs.append(out.float())
        torch.cuda.synchronize()
        err = float((outs[0] - outs[1]).abs().max())
        print(f"  layer {layer}: exact-rung tokens {'yes' if promoted else 'no'}, max diff {err:.2e}", flush=True)
        if not promoted:
            assert err == 0.0
        else:
            assert err <= 1e-2 * float(outs[1].abs().max()) + 1e-3


def test_3b_16k_storage_round_trip():
    import kvtc_storage
    import workloads
    from compressed_attention import CompressedContext

    print("[case] storage full size (3B shape, 16384 tokens, dkvtc@0.03:snap:floor1)", flush=True)
    shape, tokens, budget, _ = workloads.WORKLOADS["3b-16k-3pct"]
    _, model, m, codec, keys, values, _ = _case(f"dkvtc@{budget}:snap:floor1", 2024, shape=shape, tokens=tokens)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    data = kvtc_storage.encode_bytes(codec, keys, values, codec.last_choice, m.recent)
    t1 = time.perf_counter()
    packed = kvtc_storage.deflate(data)
    t2 = time.perf_counter()
    got = kvtc_storage.restore_context(codec, kvtc_storage.inflate(packed), model)
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    mem = CompressedContext(codec, keys, values, model)
    middle = mem.key.n
    start, end = codec.last_span
    features = shape.layers * shape.kv_heads * shape.head_dim
    light = [{"rungs": codec.last_choice[k].cpu().numpy(), "bits": codec.streams[k].rungs.cpu().numpy(),
              "features": features} for k in ("key", "value")]
    assert len(data) == storage_ref.stored_bytes(tokens, end - start, light, codec.group)
    for kind in ("key", "value"):
        a, b = getattr(got, kind), getattr(mem, kind)
        assert a.n == b.n == middle and torch.equal(a.blob[:a.used], b.blob[:b.used])
    fp16 = 2 * 2 * shape.layers * shape.kv_heads * shape.head_dim * tokens
    print(f"  stored {len(data)} B ({len(data) / fp16:.4f} of FP16), deflated {len(packed)} B; encode {1e3 * (t1 - t0):.1f} ms,"
          f" DEFLATE {1e3 * (t2 - t1):.1f} ms, inflate + restore_context {1e3 * (t3 - t2):.1f} ms", flush=True)
