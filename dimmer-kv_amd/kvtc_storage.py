"""Byte storage of kvtc / DimmerKV-TC caches (the interface of scripts/kvtc_storage.py:
``encode_bytes`` :42-79 and ``decode_bytes`` :82-135, same byte layout and errors), built for
the GPU: the codes are quantized by the codec's torch arithmetic on the device and moved
between per-token codes and the storage sections by two HIP kernels (``dkv_wire_pack`` /
``dkv_wire_unpack``); the host sees one device-to-host copy of the finished byte string on
encode and one host-to-device copy on restore.  DEFLATE runs on the host with zlib (level 6,
the reference's setting, scripts/bench_serving.py:131-134).

Layout (per stream: keys, then values): an int32 header (tokens, start, end); the rung id of
every compressed token (1 byte); for every rung present, in increasing order, either the fp16
pre-RoPE matrix rows of its tokens (the exact rung) or, for each width 2, 4, 8 the rung uses,
the LSB-first codes of (its tokens x the groups of that width), then their fp16 shifts, then
their fp16 scales; last the sinks and recent window as fp16 token-matrix rows.

Besides the reference's two functions, ``restore_context`` answers straight from the bytes: it
unpacks the codes into a ``CompressedContext`` (no FP16 cache is rebuilt), and ``deflate`` /
``inflate`` wrap zlib for the stored form.
"""

from __future__ import annotations

import zlib

import numpy as np
import torch

import dkv_hip
from hot_tier import LADDER_GROUP, LadderTables

WIDTHS = (2, 4, 8)
HEADER_BYTES = 12  # int32 tokens, start, end


DEFLATE_PIECE = 1 << 20  # bytes per independently compressed piece of the threaded DEFLATE
DEFLATE_WINDOW = 1 << 15  # DEFLATE's back-reference window


def deflate(data: bytes, level: int = 6, threads: int = 1) -> bytes:
    """zlib stream of ``data``.  ``threads`` = 1 is ``zlib.compress(data, level)`` itself, the
    reference's bytes.  ``threads`` > 1 compresses 1 MiB pieces on that many threads (zlib releases
    the GIL) and joins them into one zlib stream: each piece is raw DEFLATE primed with the
    preceding 32 KiB as its window, ended by a sync flush (the last by the final block), behind the
    standard header and before the adler32 of the whole input.  ``zlib.decompress`` reads it like
    any zlib stream; its bytes differ from the one-thread form (blocks end at piece boundaries)."""
    if threads <= 1 or len(data) <= DEFLATE_PIECE:
        return zlib.compress(data, level)
    from concurrent.futures import ThreadPoolExecutor

    view = memoryview(data)
    starts = range(0, len(data), DEFLATE_PIECE)

    def piece(start: int) -> bytes:
        end = min(start + DEFLATE_PIECE, len(data))
        if start:
            c = zlib.compressobj(level, zlib.DEFLATED, -15, zdict=view[max(0, start - DEFLATE_WINDOW):start])
        else:
            c = zlib.compressobj(level, zlib.DEFLATED, -15)
        return c.compress(view[start:end]) + c.flush(zlib.Z_FINISH if end == len(data) else zlib.Z_SYNC_FLUSH)

    with ThreadPoolExecutor(max_workers=threads) as pool:
        body = b"".join(pool.map(piece, starts))
    header = zlib.compress(b"", level)[:2]  # CMF/FLG of a zlib stream at this level
    return header + body + zlib.adler32(data).to_bytes(4, "big")


def inflate(data: bytes) -> bytes:
    return zlib.decompress(data)


class _StreamLayout:
    """Where one stream's pieces lie in the byte string, from its rung ids (host arithmetic)."""

    def __init__(self, bits: np.ndarray, rungs: np.ndarray, features: int, exact_tokens: int, base: int):
        R, G = bits.shape
        if rungs.size and (rungs.min() < 0 or rungs.max() > R):
            raise ValueError(f"rung ids must lie in 0..{R} (got {int(rungs.min())}..{int(rungs.max())})")
        self.rung_ids = base
        counts = np.bincount(rungs, minlength=R + 1).astype(np.int64)
        self.count = counts
        # position of every token among the tokens of its rung
        order = np.argsort(rungs, kind="stable")
        first = np.concatenate([[0], np.cumsum(counts)[:-1]])
        self.rank = np.empty(rungs.size, np.int32)
        self.rank[order] = (np.arange(rungs.size) - first[rungs[order]]).astype(np.int32)
        # rows R (the exact rung) and R + 1 (LadderTables' empty rung) carry no sections
        self.section = np.full((R + 2, 3), -1, np.int64)
        self.nwidth = np.zeros((R + 2, 3), np.int16)
        self.slot = np.full((R + 2, G), -1, np.int16)
        for r in range(R):
            for wi, w in enumerate(WIDTHS):
                cols = np.nonzero(bits[r] == w)[0]
                self.nwidth[r, wi] = cols.size
                self.slot[r, cols] = np.arange(cols.size)
        off = base + rungs.size
        self.exact_rows = None
        for r in np.unique(rungs):
            if r == R:
                self.exact_rows = off
                off += int(counts[R]) * features * 2
                continue
            for wi, w in enumerate(WIDTHS):
                nw = int(self.nwidth[r, wi])
                if nw:
                    self.section[r, wi] = off
                    off += int(counts[r]) * nw * (LADDER_GROUP * w // 8 + 4)
        self.exact_tokens = off
        self.end = off + exact_tokens * features * 2

    def device_tables(self, device, total: int):
        t = {
            "section": torch.as_tensor(self.section).to(device),
            "count": torch.as_tensor(np.concatenate([self.count, [0]]).astype(np.int32)).to(device),
            "rank": torch.as_tensor(self.rank).to(device),
            "slot": torch.as_tensor(self.slot).to(device),
            "nwidth": torch.as_tensor(self.nwidth).to(device),
        }
        t["rank"] = torch.zeros(1, dtype=torch.int32, device=device)[:0] if not self.rank.size else t["rank"]
        wire = dkv_hip.Wire(t["section"].data_ptr(), t["count"].data_ptr(), dkv_hip.addr(t["rank"]),
                            t["slot"].data_ptr(), t["nwidth"].data_ptr(), total)
        return wire, t  # the tensors must outlive the kernel launch


def _full_ladder(codec, kind: str) -> LadderTables:
    stream = codec.streams[kind]
    return LadderTables(stream.rungs, stream.rung_bytes, codec.device, codec.group)


def _fp16_bytes(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.float16).contiguous().view(torch.uint8).reshape(-1)


def _fp16_rows(wire: torch.Tensor, at: int, rows: int, features: int) -> torch.Tensor:
    """fp16 [rows, features] stored at byte ``at`` (copied out: ``at`` may be odd)."""
    return wire[at:at + rows * features * 2].clone().view(torch.float16).view(rows, features)


def encode_bytes(codec, keys, values, choice: dict, exact_recent: int) -> bytes:
    """Serialize a compressed cache; ``choice`` is ``codec.last_choice`` (scripts/kvtc_storage.py:42-79)."""
    from kvtc import quantize_groups_codes, rope_tables, token_matrix

    device = codec.device
    tokens = keys[0].shape[2]
    start, end = codec.middle_span(tokens, exact_recent)
    middle = end - start
    features = codec.layers * codec.heads * codec.head_dim
    cos, sin = rope_tables(codec._model, tokens, device)
    prepared, base = [], HEADER_BYTES
    for kind, tensors in (("key", keys), ("value", values)):
        rungs = choice[kind].to(device)
        if bool((rungs < 0).any()):
            raise NotImplementedError("Byte storage does not support evicted tokens yet.")
        stream = codec.streams[kind]
        bits = stream.rungs.cpu().numpy().astype(np.int64)
        layout = _StreamLayout(bits, rungs.cpu().numpy().astype(np.int64), features, tokens - middle, base)
        prepared.append((kind, tensors, rungs, layout))
        base = layout.end
    wire = torch.empty(base, dtype=torch.uint8, device=device)
    wire[:HEADER_BYTES] = torch.tensor(np.asarray([tokens, start, end], "<i4").view(np.uint8), device=device)
    for kind, tensors, rungs, layout in prepared:
        stream = codec.streams[kind]
        coefficients = codec.centered(tensors, kind, cos, sin, start, end) @ stream.basis  # compress's arithmetic
        wire[layout.rung_ids:layout.rung_ids + middle] = rungs.to(torch.uint8)
        groups = coefficients.shape[1] // codec.group
        codes = torch.zeros(middle, groups, codec.group, dtype=torch.uint8, device=device)
        low = torch.zeros(middle, groups, dtype=torch.float16, device=device)
        scale = torch.zeros_like(low)
        exact_rung = len(stream.rung_bytes)
        for rung in sorted(rungs.unique().tolist()):
            if rung == exact_rung:
                continue
            rows = rungs == rung
            codes[rows], low[rows], scale[rows] = quantize_groups_codes(coefficients[rows], stream.rungs[rung],
                                                                        codec.group)
        ladder = _full_ladder(codec, kind)
        w, keep = layout.device_tables(device, base)
        dkv_hip.wire_pack(codes, low.view(torch.int16), scale.view(torch.int16), rungs.to(torch.int16).contiguous(),
                          ladder.c_ladder(), w, wire)
        # the token-matrix rows of the tokens stored as they are (the exact rung's, in token order, then the sinks
        # and the recent window), converted from those tokens only: the conversion is per token
        if layout.exact_rows is not None:
            idx = start + torch.nonzero(rungs == exact_rung).flatten()
            rows = codec.to_matrix([t.index_select(2, idx) for t in tensors], kind, cos[idx], sin[idx])
            rows_bytes = _fp16_bytes(rows)
            wire[layout.exact_rows:layout.exact_rows + rows_bytes.numel()] = rows_bytes
        outside = [torch.cat([t[:, :, :start], t[:, :, end:]], dim=2) for t in tensors]
        tail = _fp16_bytes(token_matrix(outside))
        wire[layout.exact_tokens:layout.end] = tail
        del keep
    host = torch.empty(base, dtype=torch.uint8, pin_memory=True)
    host.copy_(wire)
    return host.numpy().tobytes()


class _Parsed:
    """The pieces of a byte string on the device: per stream the rung ids, the codes at those
    rungs, the exact-rung rows and the exact tokens."""

    def __init__(self, codec, data: bytes):
        device = codec.device
        if len(data) < HEADER_BYTES:
            raise ValueError(f"Decoded 0 of {len(data)} bytes.")
        self.tokens, self.start, self.end = (int(v) for v in np.frombuffer(data, "<i4", 3))
        self.middle = self.end - self.start
        if not 0 <= self.start <= self.end <= self.tokens:
            raise ValueError(f"bad storage header (tokens={self.tokens}, start={self.start}, end={self.end})")
        features = codec.layers * codec.heads * codec.head_dim
        layouts, base = [], HEADER_BYTES
        for kind in ("key", "value"):
            if base + self.middle > len(data):
                raise ValueError(f"Decoded {base} of {len(data)} bytes.")
            rungs = np.frombuffer(data, np.uint8, self.middle, base).astype(np.int64)
            bits = codec.streams[kind].rungs.cpu().numpy().astype(np.int64)
            layout = _StreamLayout(bits, rungs, features, self.tokens - self.middle, base)
            layouts.append((kind, rungs, layout))
            base = layout.end
        if base != len(data):
            raise ValueError(f"Decoded {base} of {len(data)} bytes.")
        host = torch.empty(len(data), dtype=torch.uint8, pin_memory=True)
        host.numpy()[:] = np.frombuffer(data, np.uint8)
        wire = host.to(device, non_blocking=True)
        self.choice, self.codes, self.exact_rows, self.exact_tokens = {}, {}, {}, {}
        for kind, rungs_np, layout in layouts:
            stream = codec.streams[kind]
            rungs = torch.as_tensor(rungs_np).to(device)
            groups = stream.basis.shape[1] // codec.group
            codes = torch.zeros(self.middle, groups, codec.group, dtype=torch.uint8, device=device)
            low = torch.zeros(self.middle, groups, dtype=torch.float16, device=device)
            scale = torch.zeros_like(low)
            w, keep = layout.device_tables(device, len(data))
            dkv_hip.wire_unpack(wire, rungs.to(torch.int16).contiguous(), _full_ladder(codec, kind).c_ladder(), w,
                                codes, low.view(torch.int16), scale.view(torch.int16))
            del keep
            exact_rung = len(stream.rung_bytes)
            idx = (rungs == exact_rung).nonzero().flatten()
            rows = None
            if layout.exact_rows is not None:
                rows = _fp16_rows(wire, layout.exact_rows, idx.numel(), features).float()
            self.choice[kind] = rungs
            self.codes[kind] = (codes, low, scale)
            self.exact_rows[kind] = (idx, rows)
            self.exact_tokens[kind] = _fp16_rows(wire, layout.exact_tokens, self.tokens - self.middle, features)

    def coefficients(self, kind: str) -> torch.Tensor:
        """code * scale + shift in float32 (scripts/kvtc_storage.py:119), zeros where nothing is stored."""
        codes, low, scale = self.codes[kind]
        values = codes.float() * scale.float().unsqueeze(2) + low.float().unsqueeze(2)
        return values.reshape(codes.shape[0], -1)


def decode_bytes(codec, data: bytes, dtype=torch.float16):
    """Rebuild per-layer keys and values [1, heads, tokens, dim] from ``encode_bytes`` output
    (scripts/kvtc_storage.py:82-135)."""
    from kvtc import inverse_transform, rope_tables, split_token_matrix

    p = _Parsed(codec, data)
    features = codec.layers * codec.heads * codec.head_dim
    cos, sin = rope_tables(codec._model, p.tokens, codec.device)
    out = {}
    for kind in ("key", "value"):
        stream = codec.streams[kind]
        matrix = torch.empty(p.tokens, features, device=codec.device)
        matrix[p.start:p.end] = inverse_transform(p.coefficients(kind), stream, codec.group)
        idx, rows = p.exact_rows[kind]
        if rows is not None:
            middle_rows = matrix[p.start:p.end]
            middle_rows[idx] = rows
        rebuilt = codec.from_matrix(matrix, kind, cos, sin, dtype)
        exact_layers = split_token_matrix(p.exact_tokens[kind], codec.layers, codec.heads, codec.head_dim)
        for layer, original in enumerate(exact_layers):
            rebuilt[layer][..., :p.start, :] = original[..., :p.start, :].to(dtype)
            rebuilt[layer][..., p.end:, :] = original[..., p.start:, :].to(dtype)
        out[kind] = rebuilt
    return out["key"], out["value"]


def restore_context(codec, data: bytes, model, dtype=None):
    """A ``CompressedContext`` straight from the bytes: the codes are unpacked on the GPU into
    ladder streams and attended to directly; the exact-rung tokens (their stored fp16 rows) and
    the sinks and recent window join the exact tokens, whose cache takes ``dtype`` (default: the
    model's parameter dtype, so that the model can append to it)."""
    from compressed_attention import CompressedContext
    from kvtc import inverse_transform, split_token_matrix

    p = _Parsed(codec, data)

    def promoted_rows(kind, idx):
        rows = inverse_transform(p.coefficients(kind)[idx], codec.streams[kind], codec.group)
        stored_idx, stored = p.exact_rows[kind]
        if stored is not None and stored_idx.numel():
            # exact-rung tokens of this stream: their stored rows, placed among ``idx``
            pos = torch.searchsorted(idx, stored_idx)
            rows[pos] = stored
        return rows

    if dtype is None:
        weight = next(model.parameters(), None)
        dtype = torch.float16 if weight is None else weight.dtype
    exact = {}
    for kind in ("key", "value"):
        layers = split_token_matrix(p.exact_tokens[kind], codec.layers, codec.heads, codec.head_dim)
        exact[kind] = [t.to(dtype).contiguous() for t in layers]
    ctx = CompressedContext.__new__(CompressedContext)
    ctx._init_ladder(codec, model, dtype, p.start, p.end, p.tokens, p.choice, p.codes, promoted_rows,
                     exact["key"], exact["value"])
    return ctx


__all__ = ["encode_bytes", "decode_bytes", "restore_context", "deflate", "inflate"]
