"""Attention over the compressed cache, without rebuilding the FP16 cache (MI355X HIP path).

Mirror of scripts/compressed_attention.py (SrikanthBalaaji/Dimmer-KV).  The
maths is the reference's (:1-19): keys are rebuilt one layer at a time from
coefficients x that layer's basis slice + mean, RoPE'd at their positions,
scored and discarded; values stay in coefficient space,
``sum_n p_n v_n = (sum_n p_n c_n) @ B_v + mean_v * sum_n p_n``; one softmax
spans the compressed tokens and a small exact cache (sinks, recent window,
new tokens).

What changes is where it runs: every step is a hand-written HIP kernel in
libdimmerkv_hip.so (include/dimmerkv.h).  Once per decode step (and again
after a refine) the packed hot tier (hot_tier.PackedStream) is decoded into a
per-conversation workspace: the key coefficients as fp16 MFMA operands and the
value codes as 8-bit codes with one affine pair per (token, group).  Every
layer then rebuilds its keys from that operand buffer on MFMA, RoPE'd and
scored in registers, so no layer's keys (the FP16 key cache) ever reach
memory; the values are weighted in coefficient space.

Both of the reference's entry points build a context: ``prog@`` through
``ProgressiveCache.context`` (packed bit planes), and ``dkvtc@`` through the
reference's own constructor ``CompressedContext(codec, keys, values, model,
dtype)`` (:34-89) after ``KVTCCodec.compress``, which here packs the chosen
ladder codes (hot_tier.LadderStream) instead of fp16 coefficient blocks.

``CompressedContext.attend`` keeps the reference's contract (:113-137):
(module, query [B, Hq, q_len, d], key/value [B, Hkv, T_exact, d] exact cache
after ``update``, additive attention_mask or None, scaling) ->
(output [B, q_len, Hq, d] contiguous, None).
"""

from __future__ import annotations

import torch

import dkv_hip
from hot_tier import LadderStream, LadderTables

# Exact tokens one sequence may hold in the shared softmax (the kernels' exact-token split).
MAX_EXACT_TOKENS = 1024


class ModelTables:
    """Per-model device tables shared by every conversation (the reference's basis/mean,
    scripts/compressed_attention.py:45-54): fp16 key/value bases in the kernels' layouts,
    float32 means [L, Hkv*d] and the RoPE half-tables [P, d/2] (cos/sin of
    scripts/kvtc.py:32-37; the two halves of HF's emb are equal)."""

    def __init__(self, basis_k: torch.Tensor, basis_v: torch.Tensor, mean_k: torch.Tensor, mean_v: torch.Tensor,
                 layers: int, kv_heads: int, head_dim: int, cos: torch.Tensor, sin: torch.Tensor):
        if not basis_k.is_cuda:
            raise ValueError("ModelTables needs GPU tensors (the HIP path has no CPU fallback)")
        features, rank = basis_k.shape
        if features != layers * kv_heads * head_dim or rank % 128:
            raise ValueError(f"basis [{features}, {rank}] does not match L*Hkv*d = {layers * kv_heads * head_dim}"
                             " with a rank that is a multiple of 128")
        self.layers, self.kv_heads, self.head_dim, self.rank = layers, kv_heads, head_dim, rank
        device = basis_k.device
        self.key_basis = torch.empty(layers * rank * kv_heads * head_dim, dtype=torch.float16, device=device)
        self.value_basis = torch.empty_like(self.key_basis)
        dkv_hip.prepare_key_basis(basis_k.float().contiguous(), layers, kv_heads, head_dim, rank, self.key_basis)
        dkv_hip.prepare_value_basis(basis_v.float().contiguous(), layers, kv_heads, head_dim, rank,
                                    self.value_basis)
        self.mean_k = mean_k.float().reshape(layers, kv_heads * head_dim).contiguous()
        self.mean_v = mean_v.float().reshape(layers, kv_heads * head_dim).contiguous()
        half = head_dim // 2
        self.rope_cos = cos[:, :half].float().contiguous()
        self.rope_sin = sin[:, :half].float().contiguous()

    def basis_bytes(self) -> int:
        return (self.key_basis.numel() + self.value_basis.numel()) * 2


class CompressedContext:
    """Compressed middle tokens of one or more conversations, attended to directly.

    Two constructors:

    - ``CompressedContext(codec, keys, values, model, dtype=torch.float16)``, the reference's
      (scripts/compressed_attention.py:34-89), after ``codec.compress`` (the ``dkvtc@`` /
      ``kvtc@`` entry points): the compressed tokens' ladder codes are packed per token;
    - ``CompressedContext(tables, key, value, positions, q_heads, cu_seqlens=None,
      exact_cache=None)`` over packed streams (``prog@``, and ragged batches): ``cu_seqlens``
      (int32 [B+1]) splits the streams into B conversations for a fused varlen decode.
    """

    def __init__(self, *args, **kwargs):
        from kvtc import KVTCCodec

        if args and isinstance(args[0], KVTCCodec):
            self._init_kvtc(*args, **kwargs)
        else:
            self._init_streams(*args, **kwargs)

    def _init_streams(self, tables: ModelTables, key, value, positions: torch.Tensor, q_heads: int,
                      cu_seqlens: torch.Tensor | None = None, exact_cache=None, extra=None):
        if key.n != value.n:
            raise ValueError("key and value streams hold different token counts")
        self.tables, self.key, self.value = tables, key, value
        self.q_heads = q_heads
        device = key.blob.device
        self.positions = positions.to(device=device, dtype=torch.int32).contiguous()
        if not self.positions.numel():  # no compressed token: still a non-null pointer for the C ABI
            self.positions = torch.zeros(1, dtype=torch.int32, device=device)[:0]
        elif int(positions.min()) < 0 or int(positions.max()) >= tables.rope_cos.shape[0]:
            raise ValueError(f"positions {int(positions.min())}..{int(positions.max())} fall outside the "
                             f"{tables.rope_cos.shape[0]} rows of the RoPE tables")
        if cu_seqlens is None:
            cu_seqlens = torch.tensor([0, key.n], dtype=torch.int32)
        self.cu_host = cu_seqlens.to(torch.int32).cpu().contiguous()
        self.cu = self.cu_host.to(device)
        self.batch = self.cu_host.numel() - 1
        self.exact_cache = exact_cache
        self._workspace = None
        self._prepared = None  # (plane_cap, stream versions) decoded into the workspace
        self._score_workspace = None
        self._score_prepared = None
        self._cu_exact = {}
        self._mask_cache = None  # (mask tensor, its version, keys, float32 rows) of the last forward
        self._args_static = None  # (key stream, value stream, their array addresses, the shared argument fields)
        self.importance = None  # float32 [n] while a question is being scored
        # Middle tokens held exactly (kvtc's exact rung), per layer float32 [Hkv, E_x, d] (keys RoPE'd);
        # they join the exact tokens of every softmax.
        self.extra = extra

    def _init_kvtc(self, codec, keys: list[torch.Tensor], values: list[torch.Tensor], model, dtype=torch.float16):
        """The reference constructor (scripts/compressed_attention.py:34-89) over ``codec``'s last
        compress: tokens whose key was evicted are left out (:50); the others are packed at their
        rungs into ladder streams over the union of the groups they use (:53-54), an evicted value
        decoding to the mean; tokens with a key or value at the exact rung are rebuilt once
        (inverse transform, RoPE) and attended as exact tokens.  The exact cache holds the sinks
        and the recent window (:85-88).  ``dtype`` is the reference's coefficient dtype; the
        kernels decode keys to fp16 MFMA operands and value codes exactly whatever it is."""
        from kvtc import inverse_transform

        start, end = codec.last_span
        streams = codec.streams
        choice = {k: codec.last_choice[k].to(codec.device) for k in ("key", "value")}

        def promoted_rows(kind, idx):
            return inverse_transform(codec.last_coefficients[kind][idx].float(), streams[kind], codec.group)

        exact_keys = [torch.cat([k[..., :start, :], k[..., end:, :]], dim=2) for k in keys]
        exact_values = [torch.cat([v[..., :start, :], v[..., end:, :]], dim=2) for v in values]
        self._init_ladder(codec, model, dtype, start, end, keys[0].shape[2], choice, codec.last_codes, promoted_rows,
                          exact_keys, exact_values)

    def _init_ladder(self, codec, model, dtype, start: int, end: int, tokens: int, choice: dict, codes: dict,
                     promoted_rows, exact_keys: list, exact_values: list):
        """Context over kvtc ladder codes: ``choice`` holds each middle token's rung per stream
        (-1 evicted, len(rung_bytes) exact), ``codes`` per stream (codes u8 [middle, G, 64], fp16
        shifts and scales [middle, G]) at those rungs, ``promoted_rows(kind, idx)`` the pre-RoPE
        matrix rows [len(idx), features] of middle tokens attended exactly, and ``exact_keys`` /
        ``exact_values`` the per-layer sinks + recent window."""
        from common import build_cache
        from kvtc import rerotate, rope_tables

        device = codec.device
        layers, heads, dim, group = codec.layers, codec.heads, codec.head_dim, codec.group
        streams = codec.streams
        exact_rung = {k: len(streams[k].rung_bytes) for k in ("key", "value")}
        kept = choice["key"] >= 0
        promoted = kept & ((choice["key"] == exact_rung["key"]) | (choice["value"] == exact_rung["value"]))
        coded = kept & ~promoted
        rows = coded.nonzero().flatten()
        # groups any coded token uses in either stream, padded to a multiple of 4 with empty groups
        groups = streams["key"].rungs.shape[1]
        used = torch.zeros(groups, dtype=torch.bool, device=device)
        for kind in ("key", "value"):
            r = choice[kind][rows]
            r = r[(r >= 0) & (r < exact_rung[kind])].unique()
            if r.numel():
                used |= (streams[kind].rungs.to(device)[r] > 0).any(dim=0)
        cols = used.nonzero().flatten()
        padded = max(4, -(-cols.numel() // 4) * 4)
        cos, sin = rope_tables(model, tokens, device)
        packed, bases = {}, {}
        for kind in ("key", "value"):
            rungs = torch.zeros(streams[kind].rungs.shape[0], padded, dtype=torch.long)
            rungs[:, :cols.numel()] = streams[kind].rungs.cpu()[:, cols.cpu()]
            table = LadderTables(rungs, None, device, group)
            code, low, scale = codes[kind]
            c = torch.zeros(rows.numel(), padded, group, dtype=torch.uint8, device=device)
            lo = torch.zeros(rows.numel(), padded, dtype=torch.float16, device=device)
            sc = torch.zeros_like(lo)
            c[:, :cols.numel()] = code[rows][:, cols]
            lo[:, :cols.numel()] = low[rows][:, cols]
            sc[:, :cols.numel()] = scale[rows][:, cols]
            packed[kind] = LadderStream.pack(c, lo, sc, choice[kind][rows], table)
            basis = torch.zeros(streams[kind].basis.shape[0], padded * group, device=device)
            col_idx = (cols[:, None] * group + torch.arange(group, device=device)).flatten()
            basis[:, :col_idx.numel()] = streams[kind].basis[:, col_idx]
            bases[kind] = basis
        tables = ModelTables(bases["key"], bases["value"], streams["key"].mean, streams["value"].mean, layers, heads,
                             dim, cos, sin)
        extra = None
        exact_tokens = tokens - (end - start)
        idx = promoted.nonzero().flatten()
        if exact_tokens + idx.numel() > MAX_EXACT_TOKENS:
            raise ValueError(f"{exact_tokens} exact and {idx.numel()} exact-rung tokens exceed the "
                             f"{MAX_EXACT_TOKENS} exact tokens a sequence may hold")
        if idx.numel():
            extra = {}
            for kind in ("key", "value"):
                per_layer = promoted_rows(kind, idx).view(-1, layers, heads, dim)
                parts = []
                for layer in range(layers):
                    part = per_layer[:, layer].transpose(0, 1)  # [heads, E_x, d]
                    if kind == "key":
                        part = rerotate(part, cos[start + idx], sin[start + idx])
                    parts.append(part.float().contiguous())
                extra[kind] = parts
        self._init_streams(tables, packed["key"], packed["value"], rows + start,
                           model.config.num_attention_heads, exact_cache=build_cache(exact_keys, exact_values, model),
                           extra=extra)
        self.codec, self.model, self.dtype = codec, model, dtype
        self.start, self.end, self.context_tokens = start, end, tokens

    def _with_extra(self, layer: int, key_exact, value_exact, mask, q_len: int):
        """Prepends the exact-rung middle tokens (never masked) to a batch-1 exact cache."""
        if self.extra is None:
            return key_exact, value_exact, mask
        ek, ev = self.extra["key"][layer], self.extra["value"][layer]
        if key_exact is None:
            return ek, ev, None
        key_exact = torch.cat([ek, key_exact], dim=1)
        value_exact = torch.cat([ev, value_exact], dim=1)
        if mask is not None:
            mask = torch.cat([mask.new_zeros(q_len, ek.shape[1]), mask], dim=1).contiguous()
        return key_exact, value_exact, mask

    # ----- memory accounting (scripts/compressed_attention.py:91-102) -----
    def code_bytes(self) -> int:
        """Bytes held for the compressed tokens: the packed hot tiers (reference accounting), plus
        the float32 rows of exact-rung tokens."""
        extra = 0
        if self.extra is not None:
            extra = sum(t.numel() * t.element_size() for kind in ("key", "value") for t in self.extra[kind])
        return self.key.hot_bytes() + self.value.hot_bytes() + extra

    def basis_bytes(self) -> int:
        return self.tables.basis_bytes()

    def exact_bytes(self) -> int:
        if self.exact_cache is None:
            return 0
        layers = self.exact_cache.layers
        return sum((l.keys.numel() + l.values.numel()) * l.keys.element_size() for l in layers)

    def workspace_bytes(self) -> int:
        """The working memory this context keeps once allocated: the per-step decode workspace (key
        operands, value codes and affine pairs decoded once per step, per-layer probabilities and
        partials; dkv_attend_workspace_bytes) and, after a question, the scoring workspace
        (dkv_score_workspace_bytes)."""
        return sum(t.numel() for t in (self._workspace, self._score_workspace) if t is not None)

    def held_bytes(self) -> dict:
        """GPU memory held for this conversation, in parts (bytes): ``codes`` the packed streams as
        allocated (``code_bytes`` is the reference's accounting of their content), ``exact_rung``
        float32 rows of exact-rung tokens, ``exact_cache`` the sinks and recent window kept here,
        ``decode_workspace`` and, while a question is scored, ``score_workspace`` (see
        ``workspace_bytes``), and ``total``.  The bases (``basis_bytes``) are per model and not
        included."""
        extra = 0
        if self.extra is not None:
            extra = sum(t.numel() * t.element_size() for kind in ("key", "value") for t in self.extra[kind])
        parts = {
            "codes": self.key.device_bytes() + self.value.device_bytes() + self.cu.numel() * 4
                     + self.positions.numel() * self.positions.element_size(),
            "exact_rung": extra,
            "exact_cache": self.exact_bytes(),
            "decode_workspace": 0 if self._workspace is None else self._workspace.numel(),
            "score_workspace": 0 if self._score_workspace is None else self._score_workspace.numel(),
        }
        parts["total"] = sum(parts.values())
        return parts

    # ----- attention -----
    def _mask_rows(self, attention_mask: torch.Tensor, keys: int) -> torch.Tensor:
        """float32 [q_len, keys]: the additive mask's rows over the exact cache.  A forward passes the
        same mask tensor to every layer, so its conversion is kept while that tensor is (the strong
        reference keeps its memory from being reused by another mask meanwhile)."""
        key = (attention_mask, attention_mask._version, keys)
        cached = self._mask_cache
        if cached is None or cached[0] is not attention_mask or cached[1:3] != key[1:]:
            rows = attention_mask[0, 0, :, -keys:].float().contiguous()
            self._mask_cache = cached = (attention_mask, attention_mask._version, keys, rows)
        return cached[3]

    def _exact_offsets(self, lengths: tuple[int, ...]):
        """cu_exact (host and device) for these exact-tail lengths.  The tail grows by a token per decode
        step, so only the last few are kept (a dropped device array goes back to torch's allocator in
        stream order, after the kernels queued on the stream that read it)."""
        if lengths not in self._cu_exact:
            host = torch.zeros(len(lengths) + 1, dtype=torch.int32)
            host[1:] = torch.cumsum(torch.tensor(lengths, dtype=torch.int32), 0)
            while len(self._cu_exact) >= 8:
                self._cu_exact.pop(next(iter(self._cu_exact)))
            self._cu_exact[lengths] = (host, host.to(self.key.blob.device))
        return self._cu_exact[lengths]

    def layer_args(self, layer: int, query: torch.Tensor, out: torch.Tensor, key_exact: torch.Tensor | None = None,
                   value_exact: torch.Tensor | None = None, mask: torch.Tensor | None = None,
                   exact_lengths: tuple[int, ...] | None = None, scaling: float | None = None):
        """Build the C-ABI argument block of one layer.  query [B, Hq, q_len, d] (f32/f16/bf16);
        out [B, q_len, Hq, d]; key/value_exact [Hkv, E_total, d] (RoPE applied), both float32, float16
        or bfloat16 (one type; the kernels convert to float32 exactly as they load);
        mask float32 [q_len, E] (B == 1)."""
        t = self.tables
        batch, q_heads, q_len, dim = query.shape
        if batch != self.batch or q_heads != self.q_heads or dim != t.head_dim:
            raise ValueError(f"query {tuple(query.shape)} does not match the context "
                             f"(batch {self.batch}, {self.q_heads} heads, head_dim {t.head_dim})")
        a = dkv_hip.AttendArgs.from_buffer_copy(self._static_args())
        a.q_len, a.layer, a.q_heads = q_len, layer, q_heads
        a.scaling = dim ** -0.5 if scaling is None else float(scaling)
        a.query, a.query_dtype = dkv_hip.ptr(query), dkv_hip.dtype_code(query.dtype)
        if key_exact is not None and key_exact.shape[1] > 0:
            lengths = exact_lengths if exact_lengths is not None else (key_exact.shape[1],)
            host, dev = self._exact_offsets(tuple(int(x) for x in lengths))
            a.cu_exact, a.cu_exact_host = dev.data_ptr(), host.data_ptr()
            if value_exact.dtype != key_exact.dtype:
                raise ValueError(f"exact keys ({key_exact.dtype}) and values ({value_exact.dtype}) differ in type")
            a.key_exact, a.value_exact = dkv_hip.ptr(key_exact), dkv_hip.ptr(value_exact)
            a.exact_dtype = dkv_hip.dtype_code(key_exact.dtype)
            a.mask = dkv_hip.ptr(mask) if mask is not None else None
        a.out, a.out_dtype = dkv_hip.ptr(out), dkv_hip.dtype_code(out.dtype)
        return a

    def _static_args(self) -> dkv_hip.AttendArgs:
        """The fields of the argument block that every layer shares (shapes, streams, bases, tables),
        built again only when a stream's arrays move (a refine that grows the hot blob)."""
        ptrs = tuple(x.data_ptr() for s in (self.key, self.value) for x in (s.blob, s.tok_off, s.pieces))
        cached = self._args_static
        if cached is None or cached[0] is not self.key or cached[1] is not self.value or cached[2] != ptrs:
            t = self.tables
            a = dkv_hip.AttendArgs()
            a.batch = self.batch
            a.layers, a.kv_heads, a.head_dim, a.rank = t.layers, t.kv_heads, t.head_dim, t.rank
            a.key, a.value = self.key.c_stream(), self.value.c_stream()
            a.cu_seqlens = self.cu.data_ptr()
            a.cu_seqlens_host = self.cu_host.data_ptr()
            a.positions = dkv_hip.addr(self.positions)
            a.key_basis, a.value_basis = t.key_basis.data_ptr(), t.value_basis.data_ptr()
            a.mean_k, a.mean_v = t.mean_k.data_ptr(), t.mean_v.data_ptr()
            a.rope_cos, a.rope_sin, a.rope_rows = t.rope_cos.data_ptr(), t.rope_sin.data_ptr(), t.rope_cos.shape[0]
            self._args_static = cached = (self.key, self.value, ptrs, a)
        return cached[3]

    def workspace(self, args) -> torch.Tensor:
        need = dkv_hip.attend_workspace_bytes(args)
        if self._workspace is None or self._workspace.numel() < need:
            self._workspace = torch.zeros(need, dtype=torch.uint8, device=self.key.blob.device)
            self._prepared = None
        return self._workspace

    def prepare(self, args, plane_cap: int = 8) -> None:
        """K1: decode the key codes into the workspace (once per decode step; the layers reuse it)."""
        dkv_hip.attend_prepare(args, self.workspace(args), plane_cap)
        self._prepared = (plane_cap, self.key.version, self.value.version)

    def run_layer(self, args) -> None:
        """One layer through the C ABI; the key codes are decoded again at layer 0 (the start of
        every forward) and whenever the key stream changed since the last decode."""
        workspace = self.workspace(args)
        if args.layer == 0 or self._prepared != (8, self.key.version, self.value.version):
            self.prepare(args)
        dkv_hip.attend_layer(args, workspace)

    def attend(self, module, query, key, value, attention_mask, scaling):
        """Same contract as an HF attention function: returns (output [B, T, H, D], None)."""
        layer = module.layer_idx
        if module.num_key_value_groups * self.tables.kv_heads != query.shape[1]:
            raise ValueError("module.num_key_value_groups does not match the context's GQA grouping")
        query = query.contiguous()
        batch, q_heads, q_len, dim = query.shape
        out = torch.empty(batch, q_len, q_heads, dim, dtype=query.dtype, device=query.device)
        key_exact = value_exact = mask = None
        lengths = None
        if key is not None and key.shape[2] > 0:
            if batch != 1:
                raise ValueError("exact caches with batch > 1 go through layer_args(exact_lengths=...)")
            key_exact, value_exact = _exact_operand(key[0]), _exact_operand(value[0])
            if self.extra is not None or key_exact.dtype != value_exact.dtype:
                key_exact, value_exact = key_exact.float().contiguous(), value_exact.float().contiguous()
            lengths = (key.shape[2],)
            if attention_mask is not None:
                mask = self._mask_rows(attention_mask, key.shape[2])
        if self.extra is not None:
            if batch != 1:
                raise ValueError("a context with exact-rung tokens takes one conversation")
            key_exact, value_exact, mask = self._with_extra(layer, key_exact, value_exact, mask, q_len)
            lengths = (key_exact.shape[1],)
        args = self.layer_args(layer, query, out, key_exact, value_exact, mask, lengths, scaling)
        self.run_layer(args)
        if self.importance is not None:
            self._score(layer, query, key, scaling)
        return out, None

    # ----- question scoring over the hot codes (K4a) -----
    def begin_scoring(self, plane_cap: int = 8) -> None:
        """Start accumulating the attention the compressed tokens receive (dimmer.py:60-66 scoring);
        the question's keys are rebuilt from the first ``plane_cap`` planes of each group."""
        self.importance = torch.empty(self.key.n, dtype=torch.float32, device=self.key.blob.device)
        self.score_plane_cap = plane_cap
        self._score_prepared = None
        dkv_hip.score_begin(self.importance)

    def end_scoring(self) -> torch.Tensor:
        """The importance vector; the scoring workspace goes back to the allocator, so a context holds
        it only while a question is scored."""
        importance, self.importance = self.importance, None
        self._score_workspace = None
        self._score_prepared = None
        return importance

    def _score(self, layer: int, query: torch.Tensor, key: torch.Tensor, scaling) -> None:
        """Adds this layer's attention mass on each compressed token, summed over the question
        tokens and all query heads; the softmax spans the compressed tokens, the exact cache
        before the question and the question's own keys (causal)."""
        if self.batch != 1:
            raise ValueError("question scoring takes one conversation")
        q_len = query.shape[2]
        if key is None or key.shape[2] < q_len:
            raise ValueError("scoring needs the question's keys in the exact cache")
        past = key.shape[2] - q_len
        key_question = key[0, :, past:].float().contiguous()
        key_exact = value_exact = None
        lengths = None
        if past > 0:
            key_exact = key[0, :, :past].float().contiguous()
            value_exact = key_exact  # values are not read by the scoring kernels
        key_exact, value_exact, _ = self._with_extra(layer, key_exact, value_exact, None, q_len)
        if key_exact is not None:
            lengths = (key_exact.shape[1],)
        scratch = torch.empty(1, q_len, query.shape[1], query.shape[3], dtype=query.dtype, device=query.device)
        args = self.layer_args(layer, query, scratch, key_exact, value_exact, None, lengths, scaling)
        need = dkv_hip.score_workspace_bytes(args)
        if self._score_workspace is None or self._score_workspace.numel() < need:
            self._score_workspace = torch.zeros(need, dtype=torch.uint8, device=query.device)
            self._score_prepared = None
        state = (self.score_plane_cap, self.key.version)
        if self._score_prepared != state:
            dkv_hip.attend_prepare(args, self._score_workspace, self.score_plane_cap, values=False)
            self._score_prepared = state
        dkv_hip.score_layer(args, key_question, self.importance, self._score_workspace)


def _exact_operand(t: torch.Tensor) -> torch.Tensor:
    """A cache's [Hkv, E, d] exact tokens as the kernels take them: float32, float16 or bfloat16 as they
    are when contiguous and aligned for their four-element loads (a model's fp16 cache needs no
    conversion), a float32 copy otherwise."""
    if t.dtype in (torch.float16, torch.bfloat16, torch.float32) and t.is_contiguous():
        if dkv_hip.addr(t) % (16 if t.dtype == torch.float32 else 8) == 0:
            return t
    return t.float().contiguous()


def _stops(token: int, tokenizer) -> bool:
    return token == tokenizer.eos_token_id or token in tokenizer.all_special_ids


def greedy_answer(model, tokenizer, context: CompressedContext | None, cache, input_ids: torch.Tensor,
                  start_position: int, max_new_tokens: int = 12, evicted=None, stop_at_eos: bool = True):
    """Greedy decoding on top of a prefilled cache (scripts/compressed_attention.py:140-169): at most
    ``max_new_tokens`` forward passes, the first over ``input_ids`` (the question) at positions from
    ``start_position``, each later one over the token the previous pass chose; an end-of-sequence or
    special token ends the reply without being part of it (unless ``stop_at_eos`` is False).

    With ``context`` set, every attention call of the model runs over the compressed tokens directly
    (the HIP decode kernels) and ``cache`` must be ``context.exact_cache``; otherwise ``cache`` is a
    full cache with optional per-layer ``evicted`` masks.  Returns (text, first-step logits)."""
    import dimmer

    device = input_ids.device
    reply: list[int] = []
    first_logits = None
    dimmer.STATE.compressed = context
    dimmer.set_eviction(evicted)
    try:
        feed, position = input_ids, start_position
        for _ in range(max_new_tokens):
            width = feed.shape[1]
            step_positions = torch.arange(position, position + width, device=device).unsqueeze(0)
            last = model(input_ids=feed, past_key_values=cache, position_ids=step_positions,
                         use_cache=True).logits[0, -1]
            if first_logits is None:
                first_logits = last.float()
            token = int(torch.argmax(last))
            if stop_at_eos and _stops(token, tokenizer):
                break
            reply.append(token)
            feed, position = torch.full((1, 1), token, dtype=torch.long, device=device), position + width
    finally:
        dimmer.STATE.compressed = None
        dimmer.set_eviction(None)
    return tokenizer.decode(reply, skip_special_tokens=True).strip(), first_logits


__all__ = ["ModelTables", "CompressedContext", "greedy_answer"]
