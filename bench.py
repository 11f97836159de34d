"""Benchmark: compressed-cache decode tokens/s on one MI355X.

Workload (default): Llama-3.2-3B shape (28 layers x 8 KV heads x head_dim 128,
24 query heads), a 16,384-token conversation compressed to a 3% budget
(16,348 middle tokens in the packed bit-plane hot tier; 4 sinks + 32 recent +
the new token exact), key and value PCA bases of rank 2048, bf16 decode
query.  One step = one decode token = 28 layers of attention over the codes
(K2 key rebuild + scoring, K3 value weighting + basis), timed with HIP events.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload 3b-16k-3pct|1b-8k-2pct|1b-1500|3b-ragged-32]

Prints one JSON line.  ``roofline`` is for the dominant kernel (K2,
keys_scores): algorithmic MFMA flops per launch / its average duration,
measured with events around every K2 launch in the timed region.
``cpu_baseline`` times the numpy oracle (same algorithm, fp32) on the
host cores for a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT), str(ROOT / "dimmer-kv_amd")]

METRIC = "compressed-cache decode tok/s (3B shape, 16K ctx, 3% budget) + % HBM roofline"
PEAK_F16_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", default="3b-16k-3pct", choices=["1b-1500", "1b-8k-2pct", "3b-16k-3pct", "3b-ragged-32"])
    p.add_argument("--method", default="prog", choices=["prog", "dkvtc"],
                   help="entry point whose cache is decoded: prog@b:r0.01 (bit planes, default) or "
                        "dkvtc@b:snap:floor1 (kvtc ladder codes; 1b-8k-2pct / 3b-16k-3pct)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-question", action="store_true", help="skip the question stage (score, select, gather)")
    p.add_argument("--cold-tier", choices=("device", "host"), default="device",
                   help="where the prog@ cold planes live: device memory, or pinned host memory fetched per question")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on the CPU baseline sample")
    p.add_argument("--traffic-file", default=None,
                   help="rocprofv3 FETCH/WRITE summary of K2 for this workload "
                        "(default profiles/keys_scores_<config>[_dkvtc]_traffic.txt)")
    p.add_argument("--encode", action="store_true",
                   help="time the progressive encoder's stages at the 3B 16K workload; one JSON line")
    p.add_argument("--storage", action="store_true",
                   help="measure kvtc byte storage at 3b-16k-3pct (dkvtc): encode, DEFLATE, restore; one JSON line")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run a plain device copy of MIB MiB (5 launches): the known-size kernel that "
                        "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    p.add_argument("--model", action="store_true",
                   help="time greedy decoding through a random-weight HF Llama-3.2-1B-shaped model over an "
                        "8K-token context compressed by --method (dkvtc@0.02:snap:floor1 or prog@0.02:r0.01), "
                        "direct over the codes and over the rebuilt cache; one JSON line")
    p.add_argument("--new-tokens", type=int, default=32, help="tokens generated per reply in --model")
    p.add_argument("--gemm-reference", action="store_true",
                   help="only time the bare fp16 GEMM of K2's key-rebuild shape at 3b-16k-3pct through "
                        "torch.matmul (hipBLASLt): a library figure beside the fused kernel; one JSON line")
    return p.parse_args()


def copy_calibration(mib: int) -> None:
    import torch

    n = mib * 2**20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)  # first touch of both buffers, outside the timing
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(4):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    seconds = start.elapsed_time(end) / 1e3 / 4
    # the achieved copy rate (bytes read + written per second) is the HBM figure this part reaches
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": 5,
                      "copy_read_plus_write_GBps": round(2 * n / seconds / 1e9, 1)}), flush=True)


def gemm_reference(steps: int = 50) -> None:
    """[16,348 x 2,048] x [2,048 x 1,024] fp16: the decoded key coefficients of one layer times the key
    basis of its 8 KV heads, which K2 computes fused with the decode epilogue (RoPE, QK, softmax
    statistics).  The library GEMM does none of that work, so it bounds what an unfused K2 would cost."""
    import torch

    n, rank, width = 16348, 2048, 1024
    g = torch.Generator(device="cuda").manual_seed(0)
    a = torch.randn(n, rank, device="cuda", dtype=torch.float16, generator=g) * 0.01
    b = torch.randn(rank, width, device="cuda", dtype=torch.float16, generator=g) * 0.01
    c = torch.empty(n, width, device="cuda", dtype=torch.float16)
    for _ in range(10):
        torch.matmul(a, b, out=c)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        torch.matmul(a, b, out=c)
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) / steps * 1e3
    print(json.dumps({"gemm": f"fp16 [{n} x {rank}] x [{rank} x {width}] (torch.matmul)", "launches": steps,
                      "us_per_gemm": round(us, 2), "TFLOPs": round(2 * n * rank * width / us / 1e6, 1)}), flush=True)


def read_traffic(path: str):
    """HBM bytes per K2 launch from a committed rocprofv3 --pmc summary (line 'traffic_bytes_per_launch: N')."""
    try:
        for line in Path(path).read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def host_cores() -> tuple[int, str]:
    """The cores this process may run on (its CPU affinity), capped by OMP_NUM_THREADS when that is set
    (the host's share for this GPU), and a note of how the count was reached.  A cap below the affinity
    is printed as a warning and recorded in the note, since it slows the CPU baseline."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    n, note = affinity, f"CPU affinity {affinity}"
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        note += f", OMP_NUM_THREADS={omp}"
        if int(omp) < affinity:
            n = int(omp)
            print(f"[bench] warning: OMP_NUM_THREADS={omp} caps the CPU baseline below the {affinity} cores of "
                  "this process's affinity", file=sys.stderr, flush=True)
    return max(1, n), note


def _oracle_conversations(w):
    """The oracle's inputs for a workload, one entry per conversation it times: (coefficients per stream
    [n, r] float32, host bases [F, r] per stream, RoPE cos/sin rows [n, d] of its compressed tokens,
    its batch index, exact-token range, its share of the step's compressed tokens).

    prog@ workloads: the K1-decoded coefficients of the packed streams and the synthetic bases.  dkvtc
    (``w.codec``): the codec's own coefficients of the kept tokens with its full-rank bases, as the
    parity tests compare them.  Ragged batches: the shortest, a middle and the longest conversation,
    which together stand for the batch in proportion to their tokens."""
    import numpy as np
    import torch

    s = w.shape

    def rope_rows(positions):
        cos = w.tables.rope_cos.cpu()[positions].numpy()
        sin = w.tables.rope_sin.cpu()[positions].numpy()
        return np.concatenate([cos, cos], -1), np.concatenate([sin, sin], -1)

    if hasattr(w, "codec"):
        codec = w.codec
        start, _ = codec.last_span
        kept = codec.last_choice["key"].cpu().numpy() >= 0
        coef = {k: codec.last_coefficients[k].float().cpu().numpy()[kept] for k in ("key", "value")}
        basis = {k: codec.streams[k].basis.cpu().numpy() for k in ("key", "value")}
        n_extra = 0 if w.context.extra is None else w.context.extra["key"][0].shape[1]
        cos, sin = rope_rows(torch.from_numpy(np.nonzero(kept)[0] + start))
        return [(coef, basis, cos, sin, 0, (n_extra, w.key_exact.shape[2]), 1.0)], "codec coefficients of the kept tokens"
    coef_all = {k: w.streams[k].dequantize(dtype=torch.float32).cpu().numpy() for k in ("key", "value")}
    cu = w.context.cu_host.numpy()
    e_off = np.concatenate([[0], np.cumsum(w.exact_lengths)])
    lengths = np.diff(cu)
    picks = [0] if w.batch == 1 else sorted({int(np.argmin(lengths)), int(np.argsort(lengths)[w.batch // 2]),
                                              int(np.argmax(lengths))})
    convs = []
    for b in picks:
        t0, t1 = int(cu[b]), int(cu[b + 1])
        cos, sin = rope_rows(w.context.positions[t0:t1].long().cpu())
        convs.append(({k: v[t0:t1] for k, v in coef_all.items()}, w.synthetic_basis_host, cos, sin, b,
                      (int(e_off[b]), int(e_off[b + 1])), (t1 - t0) / max(int(cu[-1]), 1)))
    what = "K1-decoded coefficients" if w.batch == 1 else \
        f"K1-decoded coefficients of conversations {picks} ({sum(c[-1] for c in convs):.3f} of the batch's tokens)"
    return convs, what


def cpu_baseline(w, seconds: float):
    """Oracle (numpy fp32) attention of the same workload on every host core this process may use:
    one warm-up layer, then three passes over the layers (all of them when a pass fits a third of
    ``seconds``, else the first k), each pass's mean per-layer time scaled to a step; the reported
    rate is the median of the three passes.  A ragged batch times three of its conversations per
    layer and scales their time by the inverse of their share of the batch's compressed tokens."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import attention_ref

    s = w.shape
    cores, core_note = host_cores()
    convs, what = _oracle_conversations(w)
    share = sum(c[-1] for c in convs)
    wdt = s.kv_heads * s.head_dim
    inputs = {}

    def layer_inputs(layer, conv):
        key = (layer, conv[4])
        if key not in inputs:
            basis, b, (e0, e1) = conv[1], conv[4], conv[5]
            inputs[key] = (w.queries[layer][b:b + 1].float().cpu().numpy(),
                           basis["key"][layer * wdt:(layer + 1) * wdt].T, basis["value"][layer * wdt:(layer + 1) * wdt].T,
                           w.tables.mean_k[layer].cpu().numpy(), w.tables.mean_v[layer].cpu().numpy(),
                           w.key_exact[layer][None, :, e0:e1].cpu().numpy(),
                           w.value_exact[layer][None, :, e0:e1].cpu().numpy())
        return inputs[key]

    def run(layer):
        total = 0.0
        for conv in convs:
            q, bk, bv, mk, mv, ke, ve = layer_inputs(layer, conv)
            coef, cos, sin = conv[0], conv[2], conv[3]
            t0 = time.perf_counter()
            attention_ref.attend(q, coef["key"], coef["value"], bk, bv, mk, mv, cos, sin, ke, ve)
            total += time.perf_counter() - t0
        return total / share  # the whole batch's layer

    with threadpool_limits(limits=cores):
        warm = run(0)
        per_pass = max(1, min(s.layers, int(seconds / 3 / max(warm * share, 1e-6))))
        passes = [float(np.mean([run(layer) for layer in range(per_pass)])) for _ in range(3)]
    per_layer = float(np.median(passes))
    return {"value": w.batch / (per_layer * s.layers), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"numpy fp32 oracle (oracle/attention_ref.attend over {what}) of the same "
                      f"workload on {cores} host cores ({core_note}): one warm-up layer, then 3 passes over {per_pass} of "
                      f"{s.layers} layers; median pass {per_layer * 1e3:.0f} ms/layer (passes "
                      f"{', '.join(f'{p * 1e3:.0f}' for p in passes)} ms), scaled x{s.layers}"}


def held_memory(w) -> dict:
    """GPU memory held for the conversation(s) of a workload, in MiB: the context's parts
    (CompressedContext.held_bytes: packed codes as allocated, the decode workspace) and the exact
    cache the workload keeps beside it (float32 keys and values of the sinks, recent window and new
    token, all layers); apart from them, the extra working memory of a question (the scoring
    workspace and the importance vector, released after it) and the bases (per model).  ``code_bytes`` is the reference's accounting of the packed content
    (scripts/compressed_attention.py:91-94)."""
    ctx = w.context
    parts = ctx.held_bytes()
    parts.pop("total")
    if ctx.exact_cache is None:
        parts["exact_cache"] = sum(t.numel() * t.element_size() for t in (w.key_exact, w.value_exact))
    parts.pop("score_workspace")
    mib = {k: round(v / 2**20, 2) for k, v in parts.items()}
    mib["held_total"] = round(sum(parts.values()) / 2**20, 2)
    q = getattr(w, "question", None)
    if q is not None:  # working memory while a question is scored (released after it)
        mib["question_extra"] = round((q.workspace.numel() + q.importance.numel() * 4 + q.idx.numel() * 4) / 2**20, 2)
    mib["code_bytes_reference_accounting"] = round(ctx.code_bytes() / 2**20, 2)
    mib["bases_per_model"] = round(ctx.basis_bytes() / 2**20, 2)
    mib["unit"] = "MiB"
    return mib


def question_stage(w):
    """The question before the decode (the configuration's first three steps): score the hot tier
    with 64 query tokens using the first 2 planes (28 layers), select the top 1 %, gather their
    cold planes.  Scoring and selection are timed over 10 repetitions after two warm-ups; the gather
    runs once (it changes the cache the decode then reads)."""
    import torch

    q = w.question
    for _ in range(2):
        q.score()
        q.select()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    reps = 10
    ev[0].record()
    for _ in range(reps):
        q.score()
    ev[1].record()
    for _ in range(reps):
        q.select()
    ev[2].record()
    fetched = q.gather()
    ev[3].record()
    torch.cuda.synchronize()
    out = {"query_tokens": int(q.queries.shape[3]), "plane_cap": q.plane_cap, "selected": q.count,
           "score_ms": round(ev[0].elapsed_time(ev[1]) / reps, 3), "topk_ms": round(ev[1].elapsed_time(ev[2]) / reps, 3),
           "gather_ms": round(ev[2].elapsed_time(ev[3]), 3), "fetched_bytes": fetched,
           "cold_tier": "host" if w.streams["key"].cold_on_host else "device"}
    print(f"[bench] question: {out}", file=sys.stderr, flush=True)
    return out


def storage_bench(reps: int = 3, cpu_tokens: int = 1024):
    """kvtc byte storage at the 3b-16k-3pct workload (Llama-3.2-3B shape, 16,384 tokens, dkvtc@0.03:snap:floor1):
    GPU encode (quantize + dkv_wire_pack + one device-to-host copy), the two storage kernels alone
    (HIP events on their stream), host DEFLATE / INFLATE (zlib level 6), ``restore_context`` (one
    host-to-device copy + dkv_wire_unpack + ladder packing) and ``decode_bytes`` (FP16 rebuild).
    CPU baseline: the numpy oracle's encode + decode of the first ``cpu_tokens`` compressed tokens
    of the same cache, scaled to the stored bytes."""
    import numpy as np
    import torch

    import dkv_hip
    import kvtc
    import kvtc_storage
    import methods
    import synth
    import workloads
    from oracle import storage_ref

    dev = "cuda"
    shape, tokens, budget, _ = workloads.WORKLOADS["3b-16k-3pct"]
    ctx = synth.make_context(shape, tokens, 2024, device=dev)
    model = synth.RopeModel(shape, dev)
    m = methods.Methods("synthetic/llama-3.2", device=dev, model=model, kvtc=synth.kvtc_checkpoint(ctx))
    keys, values = synth.prefill_cache(ctx, device=dev, dtype=torch.float16, compute_device=dev)
    g = torch.Generator("cpu").manual_seed(2024 + 80)
    scores = {"snap": [torch.rand(shape.kv_heads, tokens, generator=g).to(dev) for _ in range(shape.layers)]}
    m.apply(f"dkvtc@{budget}:snap:floor1", keys, values, scores)
    codec = m.codec("kvtc")

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            out = fn()
        torch.cuda.synchronize()
        return out, (time.perf_counter() - t0) / reps * 1e3

    data, encode_ms = timed(lambda: kvtc_storage.encode_bytes(codec, keys, values, codec.last_choice, m.recent))
    packed, deflate_ms = timed(lambda: kvtc_storage.deflate(data))
    deflate_threads = min(16, os.cpu_count() or 1)
    packed_mt, deflate_mt_ms = timed(lambda: kvtc_storage.deflate(data, threads=deflate_threads))
    _, inflate_ms = timed(lambda: kvtc_storage.inflate(packed))
    _, restore_ms = timed(lambda: kvtc_storage.restore_context(codec, data, model))
    _, decode_ms = timed(lambda: kvtc_storage.decode_bytes(codec, data))
    # the storage kernels alone, on the values stream (the larger rung mix is the same for keys)
    parsed = kvtc_storage._Parsed(codec, data)
    rungs_np = parsed.choice["value"].cpu().numpy()
    features = shape.layers * shape.kv_heads * shape.head_dim
    base = kvtc_storage.HEADER_BYTES  # section offsets as if values were the first stream (same sizes)
    layout = kvtc_storage._StreamLayout(codec.streams["value"].rungs.cpu().numpy().astype(np.int64), rungs_np,
                                        features, tokens - parsed.middle, base)
    wire = torch.zeros(layout.end, dtype=torch.uint8, device=dev)
    w, keep = layout.device_tables(dev, layout.end)
    ladder = kvtc_storage._full_ladder(codec, "value")
    codes, low, scale = parsed.codes["value"]
    rung16 = parsed.choice["value"].to(torch.int16).contiguous()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    for _ in range(2):
        dkv_hip.wire_pack(codes, low.view(torch.int16), scale.view(torch.int16), rung16, ladder.c_ladder(), w, wire)
        dkv_hip.wire_unpack(wire, rung16, ladder.c_ladder(), w, codes, low.view(torch.int16), scale.view(torch.int16))
    ev[0].record()
    for _ in range(reps):
        dkv_hip.wire_pack(codes, low.view(torch.int16), scale.view(torch.int16), rung16, ladder.c_ladder(), w, wire)
    ev[1].record()
    for _ in range(reps):
        dkv_hip.wire_unpack(wire, rung16, ladder.c_ladder(), w, codes, low.view(torch.int16), scale.view(torch.int16))
    ev[2].record()
    torch.cuda.synchronize()
    pack_us = ev[0].elapsed_time(ev[1]) / reps * 1e3
    unpack_us = ev[1].elapsed_time(ev[2]) / reps * 1e3
    section_bytes = layout.exact_tokens - (base + parsed.middle)
    code_bytes = codes.numel() + 4 * low.numel()
    del keep
    # CPU baseline: the oracle over the first cpu_tokens compressed tokens
    start, end = codec.last_span
    n = min(cpu_tokens, end - start)
    cos, sin = kvtc.rope_tables(model, tokens, dev)
    streams, metas = [], []
    for kind, tensors in (("key", keys), ("value", values)):
        stream = codec.streams[kind]
        matrix = codec.to_matrix(tensors, kind, cos, sin)[start:start + n]
        coef = (matrix - stream.mean) @ stream.basis
        streams.append({"rungs": codec.last_choice[kind][:n].cpu().numpy(), "bits": stream.rungs.cpu().numpy(),
                        "coefficients": coef.cpu().numpy(), "matrix_rows": matrix.cpu().numpy(),
                        "exact_tokens": np.zeros((0, features), np.float32), "features": features})
        metas.append({"bits": stream.rungs.cpu().numpy(), "rank": stream.basis.shape[1], "features": features})
    t0 = time.perf_counter()
    sample = storage_ref.encode(n, 0, n, streams, codec.group)
    t1 = time.perf_counter()
    storage_ref.decode(sample, metas, codec.group)
    t2 = time.perf_counter()
    mb = len(data) / 1e6
    result = {
        "metric": "kvtc byte storage, dkvtc@0.03:snap:floor1 (3B shape, 16K tokens)",
        "value": round(mb / (restore_ms / 1e3), 1), "unit": "MB/s restored into a CompressedContext",
        "higher_is_better": True, "data": "synthetic",
        "stored_bytes": len(data), "fp16_fraction": round(len(data) / (4 * features * tokens), 5),
        "deflated_bytes": len(packed),
        "encode_ms": round(encode_ms, 2), "deflate_ms": round(deflate_ms, 1), "inflate_ms": round(inflate_ms, 1),
        "deflate_threaded": {"threads": deflate_threads, "ms": round(deflate_mt_ms, 1), "bytes": len(packed_mt),
                             "inflates_to_input": kvtc_storage.inflate(packed_mt) == data},
        "restore_context_ms": round(restore_ms, 2), "decode_bytes_ms": round(decode_ms, 2),
        "wire_pack_us": round(pack_us, 1), "wire_unpack_us": round(unpack_us, 1),
        "wire_kernel_bytes": {"sections": int(section_bytes), "codes_and_affine": int(code_bytes),
                              "note": "values stream, per launch"},
        "cpu_baseline": {"value": round(len(sample) / 1e6 / (t2 - t0), 2), "unit": "MB/s encode+decode",
                         "encode_s": round(t1 - t0, 3), "decode_s": round(t2 - t1, 3), "cores": 1, "kind": "port",
                         "sample": f"oracle/storage_ref encode + decode (numpy) of the first {n} compressed tokens "
                                   f"({len(sample)} B) of the same cache"},
    }
    print(json.dumps(result), flush=True)


def model_bench(method: str, new_tokens: int = 32, tokens: int = 8192, question: int = 12, seed: int = 8080):
    """Greedy decoding through a Hugging Face Llama model, the way the reference times its direct
    path (scripts/compressed_attention.py:140-169 ``greedy_answer``; scripts/test_compressed_attention.py):
    a Llama-3.2-1B-shaped model (16 layers, 32 query / 8 KV heads x 64, MLP 8192, vocabulary 128,256)
    with random fp16 weights from a local config (nothing is downloaded), an ``tokens``-token context
    prefilled through the dimmer hook with score capture (dimmer.prefill_with_scores), compressed by
    ``Methods.apply`` at 2 % (``dkvtc@0.02:snap:floor1``, or ``prog@0.02:r0.01``, whose question is
    first scored over the codes and the top 1 % refined), then a question of ``question`` random
    tokens answered with ``new_tokens`` greedy tokens: directly over the codes (CompressedContext
    through the hook) and over the rebuilt cache (the hook's eager attention).  The bases are random
    orthonormal rank-1,024 bases with the prefill's mean (a calibration stand-in), so the
    replies are not meaningful text.  The two paths are compared as the reference does: their
    first-step logits, and how many reply tokens agree (random weights leave the logits of a
    128,256-token vocabulary close together, so replies can part after a few tokens).

    Decode tok/s = new_tokens / (time of a 1 + new_tokens reply - time of the question step alone),
    each the median of 3 after a warm-up, with the host waiting for every token's argmax as
    ``greedy_answer`` does.  A separate instrumented reply splits each decode token's time into the
    attention hook's host time (Python and the C-ABI argument blocks, summed over the layers), its
    device time (HIP events around each call: the exact tail's conversion and the decode kernels)
    and the time outside those kernels (the model's own layers, logits, argmax, host waits)."""
    import statistics

    import torch

    import common
    import dimmer
    import methods
    import synth
    from compressed_attention import CompressedContext, greedy_answer
    from transformers import LlamaForCausalLM

    class Tokenizer:  # ids as text; no special tokens
        eos_token_id = -1
        all_special_ids: list = []

        def decode(self, ids, skip_special_tokens=True):
            return " ".join(str(i) for i in ids)

    dev = "cuda"
    name = {"dkvtc": "dkvtc@0.02:snap:floor1", "prog": "prog@0.02:r0.01"}[method]
    shape = synth.SHAPE_1B
    config = synth.llama_config(shape)
    config.intermediate_size, config.vocab_size, config.tie_word_embeddings = 8192, 128256, True
    torch.manual_seed(seed)
    with torch.device(dev):  # initialise the weights on the GPU
        model = LlamaForCausalLM(config).to(dtype=torch.float16).eval()
    dimmer.install(model)
    g = torch.Generator("cpu").manual_seed(seed + 1)
    ids = torch.randint(0, config.vocab_size, (1, tokens), generator=g).to(dev)
    tail = torch.randint(0, config.vocab_size, (1, question), generator=g).to(dev)
    with torch.no_grad():
        cache, scores = dimmer.prefill_with_scores(model, ids)
    keys, values = common.cache_tensors(cache)
    keys, values = [k.clone() for k in keys], [v.clone() for v in values]
    del cache
    # calibration stand-in: random orthonormal bases, the prefill's mean token vector per stream
    import kvtc

    ck = synth.kvtc_checkpoint(synth.make_context(shape, 64, seed=seed + 2))
    cos, sin = kvtc.rope_tables(model, tokens, dev)
    for kind, tensors in (("key", keys), ("value", values)):
        rows = [kvtc.derotate(t, cos, sin) if kind == "key" else t.float() for t in tensors]
        ck[kind]["mean"] = kvtc.token_matrix(rows).mean(dim=0).cpu()
    m = methods.Methods("synthetic/llama-3.2", device=dev, model=model, kvtc=ck,
                        progressive=synth.order_checkpoint(shape))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    compressed = m.apply(name, keys, values, scores)
    torch.cuda.synchronize()
    compress_s = time.perf_counter() - t0
    refine_ms = fetched = None
    if method == "dkvtc":
        context = CompressedContext(m.codec("kvtc"), keys, values, model)
        exact_kv = ([l.keys for l in context.exact_cache.layers], [l.values for l in context.exact_cache.layers])
        rebuilt_kv = (compressed.keys, compressed.values)
    else:
        stored = compressed.stored
        exact_kv = (stored.exact["key"], stored.exact["value"])
        ask = common.build_cache([t.clone() for t in exact_kv[0]], [t.clone() for t in exact_kv[1]], model)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.no_grad():
            _, _, fetched = compressed.refine(tail[0], tokens, exact_cache=ask)
        torch.cuda.synchronize()
        refine_ms = (time.perf_counter() - t0) * 1e3
        context = stored.context(config.num_attention_heads,
                                 common.build_cache([t.clone() for t in exact_kv[0]], [t.clone() for t in exact_kv[1]],
                                                    model))
        rebuilt_kv = stored.hot()
    tok = Tokenizer()

    def reply(direct: bool, n: int):
        kv = exact_kv if direct else rebuilt_kv
        cache = common.build_cache([t.clone() for t in kv[0]], [t.clone() for t in kv[1]], model)
        torch.cuda.synchronize()
        t = time.perf_counter()
        with torch.no_grad():
            text, logits = greedy_answer(model, tok, context if direct else None, cache, tail, tokens,
                                         max_new_tokens=n, stop_at_eos=False)
        torch.cuda.synchronize()
        return time.perf_counter() - t, text, logits

    out = {}
    for direct in (True, False):
        reply(direct, 2)  # warm-up
        first = statistics.median(reply(direct, 1)[0] for _ in range(3))
        runs = [reply(direct, 1 + new_tokens) for _ in range(3)]
        whole = statistics.median(r[0] for r in runs)
        out[direct] = {"tok_s": new_tokens / (whole - first), "question_ms": first * 1e3, "reply": runs[0][1].split(),
                       "logits": runs[0][2], "ms_per_token": (whole - first) / new_tokens * 1e3}
    # instrumented reply: the attention hook's host and device time per decode token
    plain = context.attend
    calls = []

    def timed(module, query, key, value, attention_mask, scaling):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t = time.perf_counter()
        start.record()
        result = plain(module, query, key, value, attention_mask, scaling)
        end.record()
        calls.append((query.shape[2], time.perf_counter() - t, start, end))
        return result

    context.attend = timed
    try:
        reply(True, 1 + new_tokens)
    finally:
        context.attend = plain
    steps = [c for c in calls if c[0] == 1]
    per = len(steps) / shape.layers
    host_ms = sum(c[1] for c in steps) * 1e3 / per
    device_ms = sum(c[2].elapsed_time(c[3]) for c in steps) / per
    direct = out[True]
    held = {k: round(v / 2**20, 2) for k, v in context.held_bytes().items()}
    result = {
        "metric": f"greedy decode tok/s through HF Llama (1B shape, {tokens}-token context, {name})",
        "value": round(direct["tok_s"], 2), "unit": "tok/s", "higher_is_better": True, "data": "synthetic",
        "model": "Llama-3.2-1B shape, random fp16 weights (local config)",
        "method": name, "context_tokens": tokens, "question_tokens": question, "new_tokens": new_tokens,
        "rebuilt_tok_s": round(out[False]["tok_s"], 2),
        "vs_rebuilt": {
            "first_step_logit_max_diff": round(float((direct["logits"] - out[False]["logits"]).abs().max()), 5),
            "logit_scale": round(float(out[False]["logits"].abs().max()), 3),
            "reply_tokens_agreeing": next((i for i, (a, b) in enumerate(zip(direct["reply"], out[False]["reply"]))
                                           if a != b), new_tokens),
            "reply_tokens": new_tokens},
        "question_ms": {"direct": round(direct["question_ms"], 2), "rebuilt": round(out[False]["question_ms"], 2)},
        "per_token_ms": {"wall": round(direct["ms_per_token"], 3), "attention_host": round(host_ms, 3),
                         "attention_device": round(device_ms, 3),
                         "outside_attention_kernels": round(direct["ms_per_token"] - device_ms, 3),
                         "layers": shape.layers},
        "compress_s": round(compress_s, 2),
        "held_MiB": held,
        "reference_context": "FINDINGS.md:794-798, 927: 38.6-40.5 tok/s direct (22-29 tok/s for "
                             "dkvtc@0.02-0.03), 1B, ~8K tokens, RTX 5060 laptop GPU: other hardware and real "
                             "weights, not a like-for-like comparison",
    }
    if refine_ms is not None:
        result["refine"] = {"ms": round(refine_ms, 2), "fetched_bytes": fetched}
    print(json.dumps(result), flush=True)


def encode_bench(reps: int = 3):
    """The progressive encoder at the 3B 16K workload (Llama-3.2-3B shape, 16,384 tokens, 3 % budget,
    2-plane floor; the reference's ProgressiveCodec.encode with kvtc's floor rule): one JSON line with
    the time of each stage, from HIP events recorded by ProgressiveCodec.encode at its stage
    boundaries (median of ``reps`` encodes after one warm-up).  The stages: the PCA projection of
    each stream (fp32, as the reference), quantize8 with the 9-level error table and the per-rung
    errors (dkv_quantize8), the greedy allocation (sort), packing both tiers (dkv_pack_planes) and
    the exact tokens' copies."""
    import statistics

    import torch

    import progressive
    import synth

    dev = "cuda"
    shape, tokens, budget = synth.SHAPE_3B, 16384, 0.03
    ctx = synth.make_context(shape, tokens, seed=4040, device=dev)
    model = synth.RopeModel(shape, dev)
    codec = progressive.ProgressiveCodec(synth.kvtc_checkpoint(ctx), synth.order_checkpoint(shape), dev, model)
    keys, values = synth.prefill_cache(ctx, device=dev, dtype=torch.float16, compute_device=dev)
    floor = codec.orders["key"].rungs.index(2 * shape.groups)  # every group at 2 planes
    runs = []
    for rep in range(reps + 1):
        marks = []
        stored = codec.encode(keys, values, budget, 32, floor_rung=floor, marks=marks)
        torch.cuda.synchronize()
        if rep:
            runs.append({name: marks[i - 1][1].elapsed_time(ev) for i, (name, ev) in enumerate(marks) if i})
    stages = {name: statistics.median(r[name] for r in runs) for name in runs[0]}
    middle = stored.end - stored.start
    features = shape.layers * shape.kv_heads * shape.head_dim
    proj_ms = stages["key projection"] + stages["value projection"]
    proj_flop = 2 * 2 * middle * features * shape.rank
    total = sum(stages.values())
    result = {
        "metric": "progressive encode ms (3B shape, 16,384 tokens, 3 %, 2-plane floor)",
        "value": round(total, 2), "unit": "ms", "higher_is_better": False, "data": "synthetic",
        "stages_ms": {k: round(v, 3) for k, v in stages.items()},
        "from_coefficients_ms": round(total - proj_ms - stages["exact tokens"], 2),
        "projection": {"tflop": round(proj_flop / 1e12, 3), "achieved_tflops": round(proj_flop / proj_ms / 1e9, 1),
                       "peak_tflops": 157.3, "dtype": "fp32",
                       "frac": round(proj_flop / proj_ms / 1e9 / 157.3, 3)},
        "middle_tokens": middle, "encodes": reps,
    }
    print(json.dumps(result), flush=True)


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gemm_reference:
        gemm_reference()
        return
    if args.storage:
        storage_bench()
        return
    if args.encode:
        encode_bench()
        return
    if args.model:
        model_bench(args.method, args.new_tokens)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}): this build runs the decode path on a "
              "single GPU; sharding tokens across GPUs is a design, not a measured configuration.", file=sys.stderr)
        sys.exit(2)
    import torch

    import workloads

    torch.manual_seed(0)
    dev = "cuda"
    if args.traffic_file is None:
        suffix = "_dkvtc" if args.method == "dkvtc" else ""
        args.traffic_file = str(ROOT / "profiles" / f"keys_scores_{args.workload}{suffix}_traffic.txt")
    t_build = time.perf_counter()
    if args.method == "dkvtc":
        if args.workload not in ("1b-8k-2pct", "3b-16k-3pct"):
            print("--method dkvtc runs at 1b-8k-2pct or 3b-16k-3pct", file=sys.stderr)
            sys.exit(2)
        w = workloads.build_dkvtc(args.workload, device=dev)
    elif args.workload == "3b-ragged-32":
        w = workloads.build_ragged(device=dev, keep_host_basis=not args.no_cpu_baseline)
    else:
        w = workloads.build_decode(args.workload, device=dev, keep_host_basis=not args.no_cpu_baseline,
                                   refine_fraction=0.01 if args.workload == "3b-16k-3pct" and not args.no_question else 0.0,
                                   cold_tier=args.cold_tier)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t_build
    print(f"[bench] built {args.workload} in {build_s:.1f}s: {w.middle_total} compressed tokens, "
          f"{w.hot_code_bytes() / 2**20:.1f} MiB hot codes", file=sys.stderr, flush=True)
    question = question_stage(w) if hasattr(w, "question") else None

    for _ in range(args.warmup):
        w.step_split()
    torch.cuda.synchronize()

    # eager pass: K decode steps launched one kernel at a time, with HIP events around every K2 launch
    # on its launch stream (the roofline's per-launch duration; events cannot sit inside a graph)
    L = len(w.args)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(L * args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(L * args.steps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for k in range(args.steps):
        w.step_split(starts[k * L:(k + 1) * L], ends[k * L:(k + 1) * L])
    t1.record()
    torch.cuda.synchronize()
    eager_ms = t0.elapsed_time(t1) / args.steps
    k2_ms = sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / len(starts)

    # timed region: K decode steps replayed from one HIP graph holding the whole step (the K1 decode and
    # every layer's kernels), as a serving loop runs it; bracketed by device synchronisation
    graph = w.capture()
    for _ in range(args.warmup):
        graph.replay()
    g0 = torch.cuda.Event(enable_timing=True)
    g1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    g0.record()
    for _ in range(args.steps):
        graph.replay()
    g1.record()
    torch.cuda.synchronize()
    ms_step = g0.elapsed_time(g1) / args.steps
    print(f"[bench] {ms_step:.3f} ms/step (HIP graph replay); eager {eager_ms:.3f} ms/step with K2 "
          f"{k2_ms * 1e3:.1f} us/launch", file=sys.stderr, flush=True)

    k2_flops = w.k2_flops_per_layer()
    achieved = k2_flops / (k2_ms * 1e-3) / 1e12
    bytes_step = w.bytes_per_layer() * L
    flops_step = w.flops_per_layer() * L
    t_hbm = bytes_step / (PEAK_HBM_GBS * 1e9)
    t_mfma = flops_step / (PEAK_F16_TFLOPS * 1e12)
    step_s = ms_step * 1e-3
    result = {
        "metric": METRIC,
        "value": round(w.batch / step_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": {"3b-16k-3pct": "Llama-3.2-3B shape, 16384-token context at 3% budget, 28-layer decode",
                         "1b-8k-2pct": "Llama-3.2-1B shape, 8192-token context at 2% budget, 16-layer decode",
                         "1b-1500": "Llama-3.2-1B shape, 1500-token context, 16-layer decode",
                         "3b-ragged-32": "32 ragged Llama-3.2-3B conversations U[2K,16K] at 3%, one varlen decode"}[args.workload]
                        + (f", {w.name.split(':', 1)[1]} (kvtc ladder codes)" if args.method == "dkvtc" else ""),
            "name": args.workload,
            "method": "dkvtc@b:snap:floor1" if args.method == "dkvtc" else "prog@b:r0.01",
            "compressed_tokens": w.middle_total,
            "exact_tokens_per_seq": list(w.exact_lengths)[:4],
            "batch": w.batch,
            "layers": L,
            "rank": w.tables.rank,
            "hot_code_bytes": w.hot_code_bytes(),
            "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": "keys_scores (K2: fp16 MFMA key rebuild from the decoded codes + RoPE + QK)",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_F16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_F16_TFLOPS, 4),
            "traffic": read_traffic(args.traffic_file),
            "avg_launch_us": round(k2_ms * 1e3, 2),
            "flops_per_launch": k2_flops,
        },
        "eager_ms_per_step": round(eager_ms, 4),
        "step_roofline": {
            "algorithmic_bytes_per_step": bytes_step,
            "algorithmic_flops_per_step": flops_step,
            "hbm_frac": round(t_hbm / step_s, 4),
            "mfma_frac": round(t_mfma / step_s, 4),
            "binding_frac": round(max(t_hbm, t_mfma) / step_s, 4),
        },
        "cpu_baseline": None,
    }
    if question is not None:
        result["question"] = question
    result["memory"] = held_memory(w)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
