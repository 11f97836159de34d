"""GPU-resident synthetic decode workloads for the benchmark, the smoke test and the
full-size parity properties.

One ``DecodeWorkload`` is a compressed conversation (or a ragged batch of
them) packed on the GPU plus, per layer, the decode query, the exact cache
(sinks, recent window and the new token, RoPE applied) and a preallocated
output, with the C-ABI argument blocks built once so a decode step is just
``n_layers`` calls of ``dkv_attend_layer``.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

import dkv_hip
import synth
from compressed_attention import CompressedContext, ModelTables
from hot_tier import OrderTables, PackedStream
from progressive import plane_major_order, quantize8

WORKLOADS = {
    # name: (shape, tokens, budget, query dtype); the ragged batch is "3b-ragged-32" (build_ragged)
    "1b-1500": (synth.SHAPE_1B, 1500, None, torch.float32),
    "1b-8k-2pct": (synth.SHAPE_1B, 8192, 0.02, torch.bfloat16),
    "3b-16k-3pct": (synth.SHAPE_3B, 16384, 0.03, torch.bfloat16),
}
# At 8K tokens the 36 exact tokens alone take 22 % of a 2 % budget, which leaves less than the
# 2-plane floor (640 B/token K+V at rank 1024); the 1B 8K workload quotes its budget per compressed token
# (655.36 B/token = the floor plus top-ups), so its plane maps are drawn against that.
BUDGET_OVER_MIDDLE = {"1b-8k-2pct"}


@dataclass
class DecodeWorkload:
    name: str
    shape: synth.ModelShape
    context: CompressedContext
    tables: ModelTables
    streams: dict
    queries: torch.Tensor        # [L, B, Hq, q_len, d]
    key_exact: torch.Tensor      # [L, Hkv, E_total, d] f32
    value_exact: torch.Tensor
    outs: torch.Tensor           # [L, B, q_len, Hq, d]
    args: list = field(default_factory=list)
    workspace: torch.Tensor | None = None
    tokens: int = 0
    middle: int = 0
    exact_lengths: tuple = ()
    batch: int = 1
    q_len: int = 1

    def step(self) -> None:
        """One decode step: K1 decode of the key codes, then every layer of compressed attention."""
        dkv_hip.attend_prepare(self.args[0], self.workspace)
        for a in self.args:
            dkv_hip.attend_layer(a, self.workspace)

    def step_split(self, starts=None, ends=None) -> None:
        """Same work as ``step`` with K2 and K3 launched separately and optional timing
        events recorded around each K2 launch (on the launch stream)."""
        dkv_hip.attend_prepare(self.args[0], self.workspace)
        for i, a in enumerate(self.args):
            if starts is not None:
                starts[i].record()
            dkv_hip.attend_scores(a, self.workspace)
            if ends is not None:
                ends[i].record()
            dkv_hip.attend_values(a, self.workspace)

    def capture(self):
        """Record one decode step (K1 decode + every layer) in a HIP graph; replaying it removes the
        per-launch host overhead.  The step allocates nothing and records no memset."""
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            self.step()  # warm-up on the capture stream
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self.step()
        torch.cuda.synchronize()
        self.graph = graph
        return graph

    # ---- algorithmic work of one decode step (all layers) ----
    def hot_code_bytes(self) -> int:
        """Packed code bytes the step reads (bit-plane prefixes, or ladder rung blobs)."""
        return sum(int(s.tables.prefix64[s.pieces.long()].sum()) if isinstance(s, PackedStream) else s.hot_bytes()
                   for s in self.streams.values())

    def bytes_per_layer(self) -> int:
        s = self.shape
        basis = 2 * self.tables.rank * s.kv_heads * s.head_dim * 2  # fp16 key + value basis slices
        return self.hot_code_bytes() + basis

    def k2_flops_per_layer(self) -> int:
        s = self.shape
        n = self.middle_total
        return 2 * n * self.tables.rank * s.kv_heads * s.head_dim + 2 * n * s.q_heads * self.q_len * s.head_dim

    def flops_per_layer(self) -> int:
        s = self.shape
        n = self.middle_total
        rows = s.q_heads * self.q_len
        r = self.tables.rank
        return self.k2_flops_per_layer() + 2 * rows * n * r + 2 * rows * self.batch * r * s.head_dim

    @property
    def middle_total(self) -> int:
        return self.context.key.n


class QuestionStage:
    """Question-time work of the progressive entry point (scripts/methods.py:244-248): score the
    hot tier with the question's query tokens using each group's first ``plane_cap`` planes, pick
    the top ``fraction`` of the compressed tokens, fetch their cold planes."""

    def __init__(self, w, queries, key_exact, key_question, fraction, plane_cap=2):
        self.w, self.queries, self.key_exact, self.key_question = w, queries, key_exact, key_question
        self.fraction, self.plane_cap = fraction, plane_cap
        self.count = max(1, int(round(fraction * w.context.key.n)))
        self.idx = torch.empty(self.count, dtype=torch.int32, device=queries.device)
        self.args = []
        s = w.shape
        scratch = torch.empty(1, queries.shape[3], s.q_heads, s.head_dim, dtype=queries.dtype, device=queries.device)
        for layer in range(s.layers):
            self.args.append(w.context.layer_args(layer, queries[layer], scratch, key_exact[layer], key_exact[layer],
                                                  None, (key_exact.shape[2],)))
        self._scratch = scratch
        self.workspace = torch.zeros(dkv_hip.score_workspace_bytes(self.args[0]), dtype=torch.uint8,
                                     device=queries.device)
        self.importance = torch.empty(w.context.key.n, dtype=torch.float32, device=queries.device)

    @classmethod
    def build(cls, w, ctx, seed, fraction, q_len=64, query_scale=1.0):
        """``q_len`` question tokens of N(0, query_scale^2) bf16 queries per layer, random question keys."""
        s = w.shape
        device = w.queries.device
        queries = synth.make_queries(s, q_len, seed, device, torch.bfloat16, query_scale)
        g = torch.Generator("cpu").manual_seed(seed + 1)
        key_question = (torch.randn(s.layers, s.kv_heads, q_len, s.head_dim, generator=g) * 0.5).to(device)
        e_ctx = w.key_exact.shape[2] - w.q_len  # context exact tokens (sinks + recent)
        key_exact = w.key_exact[:, :, :e_ctx].contiguous()
        return cls(w, queries, key_exact, key_question.contiguous(), fraction)

    def score(self) -> torch.Tensor:
        """K1 (first plane_cap planes) + K4a over every layer -> importance [n]."""
        dkv_hip.score_begin(self.importance)
        dkv_hip.attend_prepare(self.args[0], self.workspace, self.plane_cap, values=False)
        for layer, a in enumerate(self.args):
            dkv_hip.score_layer(a, self.key_question[layer], self.importance, self.workspace)
        return self.importance

    def select(self) -> torch.Tensor:
        dkv_hip.topk(self.importance, self.count, self.idx)
        return self.idx

    def gather(self) -> int:
        """K4c on both streams; returns the bytes fetched (progressive.py:232).  With device cold
        tiers both streams refine on the device and one read brings back both byte counts."""
        streams = [self.w.streams[k] for k in ("key", "value")]
        if any(st.cold_on_host for st in streams):
            rows = self.idx.long()
            return sum(st.refine(rows) for st in streams)
        k = self.idx.numel()
        counts = torch.stack([st.refine_async(self.idx) for st in streams]).cpu()  # one synchronisation
        fetched, error = 0, None
        for st, c in zip(streams, counts):
            try:
                fetched += st.settle_refine(c, k)
            except ValueError as e:  # settle the other stream too before raising
                error = e
        if error is not None:
            raise error
        return fetched


def _pack_streams(coefs: dict, planes: dict, shape: synth.ModelShape, device, refine_capacity: int = 0,
                  cold_tier: str = "device") -> dict:
    order = plane_major_order(shape.groups)
    otab = OrderTables(order.planes, order.prefix_bytes, device)
    streams = {}
    for kind in ("key", "value"):
        codes, low, span = quantize8(coefs[kind].to(device), 64)
        pieces = torch.from_numpy(planes[kind] * shape.groups).to(device)
        streams[kind] = PackedStream.pack(codes, low, span, pieces, otab, refine_capacity=refine_capacity,
                                          with_cold=refine_capacity > 0, cold_tier=cold_tier)
        del codes, low, span
    return streams


def build_decode(name: str = "3b-16k-3pct", seed: int = 2024, device="cuda", q_len: int = 1, query_scale: float = 1.0,
                 shape: synth.ModelShape | None = None, tokens: int | None = None, budget: float | None = None,
                 query_dtype: torch.dtype | None = None, keep_host_basis: bool = False,
                 refine_fraction: float = 0.0, cold_tier: str = "device", budget_shape: synth.ModelShape | None = None,
                 question_scale: float = 1.0) -> DecodeWorkload:
    """A single-conversation decode workload (a ``WORKLOADS`` entry, or any shape and length).
    ``keep_host_basis`` keeps float32 host copies of the bases (for the CPU baseline);
    ``refine_fraction`` > 0 keeps a cold tier (in device memory, or pinned host memory with
    ``cold_tier="host"``) and room to refine that fraction of the tokens, and builds the question
    stage (64 bf16 query tokens of N(0, question_scale^2)).  ``budget_shape`` draws the plane maps
    for that model's budget (a few-layer slice of a larger model)."""
    if name in WORKLOADS:
        s0, t0, b0, qd0 = WORKLOADS[name]
        shape, tokens = shape or s0, tokens or t0
        budget = b0 if budget is None else budget
        query_dtype = query_dtype or qd0
    ctx = synth.make_context(shape, tokens, seed, budget=budget, device=device,
                             budget_over_middle=name in BUDGET_OVER_MIDDLE, budget_shape=budget_shape)
    capacity = int(round(refine_fraction * ctx.middle)) + 1 if refine_fraction > 0 else 0
    streams = _pack_streams(ctx.coef, ctx.planes, shape, device, capacity, cold_tier)
    cos, sin = synth.rope_tables(shape, tokens + max(q_len, 64), device)
    tables = ModelTables(ctx.basis["key"], ctx.basis["value"], ctx.mean["key"], ctx.mean["value"], shape.layers,
                         shape.kv_heads, shape.head_dim, cos, sin)
    positions = torch.arange(ctx.start, ctx.end, dtype=torch.int32)
    context = CompressedContext(tables, streams["key"], streams["value"], positions, shape.q_heads)
    new_coef = {kind: synth.coefficients(q_len, shape.rank, seed + 50 + i, device)
                for i, kind in enumerate(("key", "value"))}
    exact_coef = {kind: torch.cat([ctx.exact_coef[kind], new_coef[kind]]) for kind in ("key", "value")}
    exact_pos = torch.cat([ctx.exact_positions(), torch.arange(tokens, tokens + q_len)]).to(device)
    key_exact, value_exact = synth.decode_exact(ctx, exact_coef, exact_pos, cos, sin)
    queries = synth.make_queries(shape, q_len, seed + 60, device, query_dtype, query_scale)
    outs = torch.empty(shape.layers, 1, q_len, shape.q_heads, shape.head_dim, dtype=query_dtype, device=device)
    mask = None
    if q_len > 1:
        mask = synth.causal_mask(q_len, tokens - ctx.middle, device)[0, 0].contiguous()
    w = DecodeWorkload(name, shape, context, tables, streams, queries, key_exact, value_exact, outs,
                       tokens=tokens, middle=ctx.middle, exact_lengths=(key_exact.shape[2],), q_len=q_len)
    w.args = [context.layer_args(l, queries[l], outs[l], key_exact[l], value_exact[l], mask) for l in range(shape.layers)]
    w.workspace = context.workspace(w.args[0])
    if keep_host_basis:
        w.synthetic_basis_host = {k: v.cpu().numpy() for k, v in ctx.basis.items()}
    if refine_fraction > 0:
        w.question = QuestionStage.build(w, ctx, seed + 70, refine_fraction, query_scale=question_scale)
    # drop the float32 device bases now that the fp16 kernel layouts exist
    ctx.basis.clear()
    w.synthetic = ctx
    return w


def build_dkvtc(name: str = "3b-16k-3pct", seed: int = 2024, device="cuda", budget: float | None = None,
                method: str | None = None, query_dtype: torch.dtype | None = None,
                query_scale: float = 1.0) -> DecodeWorkload:
    """The ``dkvtc@<budget>:snap:floor1`` decode workload at a config's shape, built through the
    reference entry points: a synthetic prefill cache (fp16), ``Methods.apply`` (KVTCCodec.compress
    with per-token rungs, synthetic snap importance, floor at the finest affordable uniform rung),
    then ``CompressedContext(codec, keys, values, model)`` over the packed ladder codes.  The exact
    cache of each layer is the middle tokens kept at the exact rung, the sinks and recent window,
    and one new token."""
    import methods

    shape, tokens, b0, qd0 = WORKLOADS[name]
    budget = b0 if budget is None else budget
    query_dtype = query_dtype or qd0
    method = method or f"dkvtc@{budget}:snap:floor1"
    ctx = synth.make_context(shape, tokens, seed, device=device)
    model = synth.RopeModel(shape, device)
    kvtc_ck = synth.kvtc_checkpoint(ctx)
    keys, values = synth.prefill_cache(ctx, device=device, dtype=torch.float16, compute_device=device)
    g = torch.Generator("cpu").manual_seed(seed + 80)
    scores = {"snap": [torch.rand(shape.kv_heads, tokens, generator=g).to(device) for _ in range(shape.layers)]}
    m = methods.Methods("synthetic/llama-3.2", device=device, model=model, kvtc=kvtc_ck)
    m.apply(method, keys, values, scores)
    codec = m.codec("kvtc")
    context = CompressedContext(codec, keys, values, model)
    del keys, values
    cos, sin = synth.rope_tables(shape, tokens + 1, device)
    new_coef = {kind: synth.coefficients(1, shape.rank, seed + 50 + i, device)
                for i, kind in enumerate(("key", "value"))}
    new_k, new_v = synth.decode_exact(ctx, new_coef, torch.tensor([tokens], device=device), cos, sin)
    ke, ve = [], []
    for layer in range(shape.layers):
        exact = context.exact_cache.layers[layer]
        parts_k = [exact.keys[0].float(), new_k[layer]]
        parts_v = [exact.values[0].float(), new_v[layer]]
        if context.extra is not None:
            parts_k.insert(0, context.extra["key"][layer])
            parts_v.insert(0, context.extra["value"][layer])
        ke.append(torch.cat(parts_k, dim=1))
        ve.append(torch.cat(parts_v, dim=1))
    key_exact = torch.stack(ke).contiguous()
    value_exact = torch.stack(ve).contiguous()
    queries = synth.make_queries(shape, 1, seed + 60, device, query_dtype, query_scale)
    outs = torch.empty(shape.layers, 1, 1, shape.q_heads, shape.head_dim, dtype=query_dtype, device=device)
    streams = {"key": context.key, "value": context.value}
    w = DecodeWorkload(name + ":" + method, shape, context, context.tables, streams, queries, key_exact, value_exact,
                       outs, tokens=tokens, middle=context.key.n, exact_lengths=(key_exact.shape[2],))
    w.args = [context.layer_args(l, queries[l], outs[l], key_exact[l], value_exact[l]) for l in range(shape.layers)]
    w.workspace = context.workspace(w.args[0])
    w.codec = codec
    w.synthetic = ctx
    return w


def build_ragged(count: int = 32, lo: int = 2048, hi: int = 16384, budget: float = 0.03, seed: int = 3033,
                 device="cuda", shape: synth.ModelShape = synth.SHAPE_3B,
                 query_dtype: torch.dtype = torch.bfloat16, query_scale: float = 1.0,
                 keep_host_basis: bool = False) -> DecodeWorkload:
    """``count`` conversations with lengths U[lo, hi] (32 ragged 3B conversations of 2K-16K tokens
    at 3 % by default), independent plane maps, one packed buffer per stream and cu_seqlens
    offsets; one fused varlen decode step covers all of them.  Conversation b's query is the
    shared N(0, query_scale^2) draw times 0.5 + b / (count - 1).  ``keep_host_basis`` keeps
    float32 host copies of the bases."""
    lengths = synth.ragged_lengths(count, lo, hi, seed)
    basis = {"key": synth.orthonormal_basis(shape.features, shape.rank, seed + 1, device),
             "value": synth.orthonormal_basis(shape.features, shape.rank, seed + 2, device)}
    coefs = {"key": [], "value": []}
    planes = {"key": [], "value": []}
    positions, cu, exact_k, exact_v, exact_len = [], [0], [], [], []
    cos, sin = synth.rope_tables(shape, max(lengths) + 1, device)
    mean = None
    for b, tokens in enumerate(lengths):
        ctx = synth.make_context(shape, tokens, seed + 100 * (b + 1), budget=budget, device=device, basis=basis)
        if mean is None:
            mean = ctx.mean
        ctx.mean = mean
        for kind in ("key", "value"):
            coefs[kind].append(ctx.coef[kind])
            planes[kind].append(ctx.planes[kind])
        positions.append(torch.arange(ctx.start, ctx.end, dtype=torch.int32))
        cu.append(cu[-1] + ctx.middle)
        new_coef = {kind: synth.coefficients(1, shape.rank, seed + 100 * (b + 1) + 50 + i, device)
                    for i, kind in enumerate(("key", "value"))}
        exact_coef = {kind: torch.cat([ctx.exact_coef[kind], new_coef[kind]]) for kind in ("key", "value")}
        exact_pos = torch.cat([ctx.exact_positions(), torch.tensor([tokens])]).to(device)
        ke, ve = synth.decode_exact(ctx, exact_coef, exact_pos, cos, sin)
        exact_k.append(ke)
        exact_v.append(ve)
        exact_len.append(ke.shape[2])
    coefs = {kind: torch.cat(v) for kind, v in coefs.items()}
    planes = {kind: np.concatenate(v) for kind, v in planes.items()}
    streams = _pack_streams(coefs, planes, shape, device)
    del coefs
    tables = ModelTables(basis["key"], basis["value"], mean["key"], mean["value"], shape.layers, shape.kv_heads,
                         shape.head_dim, cos, sin)
    host_basis = {k: v.cpu().numpy() for k, v in basis.items()} if keep_host_basis else None
    basis.clear()
    cu_t = torch.tensor(cu, dtype=torch.int32)
    context = CompressedContext(tables, streams["key"], streams["value"], torch.cat(positions), shape.q_heads,
                                cu_seqlens=cu_t)
    key_exact = torch.cat(exact_k, dim=2).contiguous()  # [L, Hkv, E_total, d]
    value_exact = torch.cat(exact_v, dim=2).contiguous()
    queries = synth.make_queries(shape, 1, seed + 7, device, query_dtype, query_scale).expand(-1, count, -1, -1, -1)
    queries = (queries * torch.linspace(0.5, 1.5, count, device=device).to(query_dtype)[None, :, None, None, None])
    queries = queries.contiguous()
    outs = torch.empty(shape.layers, count, 1, shape.q_heads, shape.head_dim, dtype=query_dtype, device=device)
    w = DecodeWorkload("3b-ragged-32", shape, context, tables, streams, queries, key_exact, value_exact, outs,
                       tokens=sum(lengths), middle=cu[-1], exact_lengths=tuple(exact_len), batch=count)
    w.args = [context.layer_args(l, queries[l], outs[l], key_exact[l], value_exact[l], None, tuple(exact_len))
              for l in range(shape.layers)]
    w.workspace = context.workspace(w.args[0])
    w.lengths = lengths
    w.budget = budget
    if host_basis is not None:
        w.synthetic_basis_host = host_basis
    return w
