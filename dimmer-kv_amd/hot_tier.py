"""Packed hot/cold bit-plane tiers of one stream on the GPU.

The reference keeps progressive codes unpacked in a ``TokenStore``
(scripts/progressive.py:103-110) and only counts their bytes
(:185-194).  Here the bytes exist: a token's hot blob holds, for every group
with m > 0 planes, ``[low f16][span f16][m plane words]`` and is exactly
``order.prefix_bytes[pieces[t]]`` bytes; its cold blob holds the remaining
pieces (``prefix_bytes[-1] - prefix_bytes[pieces[t]]`` bytes, the
reference's ``fetched``, :232).  The plane-word bit order is fixed by
include/dimmerkv.h / oracle/packing_ref.py.

``PackedStream.refine`` is the cold-plane gather (K4c): selected tokens get
full blobs in a refine area at the end of the hot allocation, and their
offsets/piece counts are redirected there, so the attention kernels see the
refined tokens with no other change.  The cold tier lives in device memory, or
(``cold_tier="host"``) in pinned host memory, from which a refine copies only
the chosen tokens' cold blobs.

``LadderStream`` holds the kvtc ladder codes of the ``dkvtc@`` entry point
(scripts/kvtc.py:62-79, scripts/kvtc_storage.py:21-75) in the same
token-addressed form: one blob per token at its rung, ``[low f16][scale f16]
[64 codes of b bits, LSB-first]`` for every group with b > 0 bits, so the
same attention kernels decode either format.
"""

from __future__ import annotations

import numpy as np
import torch

import dkv_hip

HEADER_BYTES = 4
PIECE_BYTES = 8
RUNG_ID_BYTES = 1


class OrderTables:
    """Device copies of one stream's order plus the derived segment-offset tables."""

    def __init__(self, planes, prefix_bytes, device):
        planes = np.asarray(torch.as_tensor(planes).cpu(), dtype=np.int64)
        prefix = np.asarray(torch.as_tensor(prefix_bytes).cpu(), dtype=np.int64)
        self.groups = planes.shape[1]
        self.pieces = planes.shape[0] - 1
        m = planes
        m_full = planes[-1][None, :]
        seg = np.where(m > 0, HEADER_BYTES + PIECE_BYTES * m, 0)
        seg_off = np.zeros_like(seg)
        seg_off[:, 1:] = np.cumsum(seg[:, :-1], axis=1)
        cold = np.where((m == 0) & (m_full > 0), HEADER_BYTES, 0) + PIECE_BYTES * np.maximum(m_full - m, 0)
        cold_off = np.zeros_like(cold)
        cold_off[:, 1:] = np.cumsum(cold[:, :-1], axis=1)
        if not np.array_equal(seg.sum(axis=1), prefix):
            raise ValueError("order prefix_bytes do not match its plane table (8 B/piece + 4 B/first plane)")
        self.prefix_np = prefix
        self.planes = torch.as_tensor(planes.astype(np.uint8)).to(device)
        self.seg_off = torch.as_tensor(seg_off.astype(np.int32)).to(device)
        self.cold_off = torch.as_tensor(cold_off.astype(np.int32)).to(device)
        self.prefix = torch.as_tensor(prefix.astype(np.int32)).to(device)
        self.prefix64 = torch.as_tensor(prefix).to(device)
        self.full_bytes = int(prefix[-1])

    def c_order(self) -> dkv_hip.Order:
        return dkv_hip.Order(self.groups, self.pieces, self.planes.data_ptr(), self.seg_off.data_ptr(),
                             self.cold_off.data_ptr(), self.prefix.data_ptr())


def _nonnull(t: torch.Tensor) -> torch.Tensor:
    """``t`` itself, or for an empty tensor an empty view of a one-element allocation: the C ABI takes
    every array as a non-null pointer, and an empty torch tensor has none."""
    return t if t.numel() else torch.zeros(1, dtype=t.dtype, device=t.device)[:0]


def _nbytes(*tensors) -> int:
    """Bytes of the device allocations among ``tensors`` (None and host tensors count 0)."""
    return sum(t.numel() * t.element_size() for t in tensors if t is not None and t.is_cuda)


def _exclusive_cumsum(sizes: torch.Tensor) -> tuple[torch.Tensor, int]:
    off = _nonnull(torch.zeros(sizes.numel(), dtype=torch.int64, device=sizes.device))
    if sizes.numel() > 1:
        off[1:] = torch.cumsum(sizes[:-1], 0)
    total = int(sizes.sum()) if sizes.numel() else 0
    return off, total


class PackedStream:
    """Hot + cold tiers of one stream (keys or values) for n tokens."""

    def __init__(self, tables: OrderTables, blob, tok_off, pieces, cold, cold_off, hot_used: int, refine_capacity: int):
        self.tables = tables
        self.blob, self.tok_off, self.pieces = blob, tok_off, pieces
        self.cold, self.cold_off = cold, cold_off
        self.hot_used = hot_used
        self.refine_capacity = refine_capacity
        self.refined = 0
        self.version = 0  # bumped whenever tokens change (refine), so decoded copies know to refresh
        self.initial_pieces = pieces.clone()
        # host mirrors of each token's piece count and of the prefix sizes, for the host cold tier's
        # refine (it needs the rows on the host anyway); the device tier counts bytes on the device
        self._pieces_h = pieces.cpu().numpy().astype(np.int64)
        self._prefix_h = tables.prefix64.cpu().numpy()
        self._owner = None  # device tier: per-token first-entry tags of dkv_refine_rows (never cleared)
        self._refine_calls = 0
        self._stage_off = None  # host cold tier: device offsets of the staged cold blobs, by token
        self._stage_host = None  # host cold tier: pinned staging buffer, reused by every refine
        self._stage_dev = None   # ... its device copy
        self._stage_done = None  # ... an event after the last copy out of it

    @property
    def cold_on_host(self) -> bool:
        return self.cold is not None and not self.cold.is_cuda

    def move_cold_to_host(self) -> None:
        """Keep the cold tier in pinned host memory (frees its device copy); ``refine`` then copies
        only the selected tokens' cold blobs to the device."""
        if self.cold is None or self.cold_on_host:
            return
        host = torch.empty(self.cold.numel(), dtype=torch.uint8, pin_memory=True)
        host.copy_(self.cold)
        self.cold = host
        self.cold_off = self.cold_off.cpu()
        self._cold_size0 = (self.tables.full_bytes - self.tables.prefix64[self.initial_pieces.long()]).cpu()
        self._stage_off = torch.zeros(self.n, dtype=torch.int64, device=self.blob.device)
        # staging for refine, sized for the refine capacity now so that a question allocates nothing
        room = max(self.refine_capacity * self.tables.full_bytes, 16)
        self._stage_host = torch.empty(room, dtype=torch.uint8, pin_memory=True)
        self._stage_dev = torch.empty(room, dtype=torch.uint8, device=self.blob.device)

    @property
    def n(self) -> int:
        return self.pieces.numel()

    @classmethod
    def pack(cls, codes: torch.Tensor, low: torch.Tensor, span: torch.Tensor, pieces: torch.Tensor,
             tables: OrderTables, refine_capacity: int = 0, with_cold: bool = True,
             cold_tier: str = "device") -> "PackedStream":
        """codes u8 [n, G, 64], low/span f16 [n, G], pieces [n] -> packed tiers (GPU pack kernel).
        ``cold_tier`` "host" keeps the cold planes in pinned host memory."""
        if cold_tier not in ("device", "host"):
            raise ValueError(f"cold_tier must be 'device' or 'host' (got {cold_tier!r})")
        device = codes.device
        n = codes.shape[0]
        pieces = _nonnull(pieces.to(device=device, dtype=torch.int16).contiguous())
        p64 = pieces.long()
        hot_sizes = tables.prefix64[p64] if n else torch.zeros(0, dtype=torch.int64, device=device)
        tok_off, hot_total = _exclusive_cumsum(hot_sizes)
        capacity = hot_total + refine_capacity * tables.full_bytes
        blob = torch.zeros(max(capacity, 16), dtype=torch.uint8, device=device)
        cold = cold_off = None
        if with_cold:
            cold_sizes = tables.full_bytes - hot_sizes
            cold_off, cold_total = _exclusive_cumsum(cold_sizes)
            cold = torch.zeros(max(cold_total, 16), dtype=torch.uint8, device=device)
        if n:
            dkv_hip.pack_planes(codes.contiguous(), low.contiguous().view(torch.int16),
                                span.contiguous().view(torch.int16), pieces, tables.c_order(), blob, tok_off,
                                cold, cold_off)
        stream = cls(tables, blob, tok_off, pieces, cold, cold_off, hot_total, refine_capacity)
        if cold_tier == "host":
            stream.move_cold_to_host()
        return stream

    def c_stream(self) -> dkv_hip.Stream:
        return dkv_hip.Stream(self.blob.data_ptr(), dkv_hip.addr(self.tok_off), dkv_hip.addr(self.pieces),
                              self.tables.c_order(), dkv_hip.DKV_FMT_PLANES)

    def dequantize(self, t0: int = 0, nt: int | None = None, dtype=torch.float32) -> torch.Tensor:
        """K1: coefficients [nt, 64G] of tokens t0.. at their hot prefix (bit-exact in float32)."""
        nt = self.n - t0 if nt is None else nt
        out = torch.empty(nt, 64 * self.tables.groups, dtype=dtype, device=self.blob.device)
        if nt:
            dkv_hip.unpack_dequant(self.c_stream(), t0, nt, out)
        return out

    def hot_bytes(self) -> int:
        """Reference accounting of this stream's hot tier (progressive.py:185-188, without exact tokens)."""
        return int(self.tables.prefix64[self.pieces.long()].sum()) + RUNG_ID_BYTES * self.n

    def cold_bytes(self) -> int:
        return int((self.tables.full_bytes - self.tables.prefix64[self.pieces.long()]).sum())

    def device_bytes(self) -> int:
        """GPU memory this stream holds: the hot blob as allocated (with the room for refined tokens),
        the per-token offsets and piece counts, a device cold tier and its offsets, and the refine
        bookkeeping (first-entry tags, the host tier's device staging)."""
        return _nbytes(self.blob, self.tok_off, self.pieces, self.cold, self.cold_off, self._owner, self._stage_off,
                       self._stage_dev)

    def refine(self, rows: torch.Tensor) -> int:
        """K4c: fetch the cold pieces of ``rows`` (stream-local) -> bytes fetched (progressive.py:232).

        The fetched count is taken over ``rows`` as given, a repeated row counting each time as in
        the reference's formula; each distinct row is merged once.  Rows already at full precision
        cost nothing (their cold blob is empty) and are merged like the others.  Rows outside the
        stream raise ValueError and change nothing."""
        if rows.numel() == 0:
            return 0
        if self.cold is None:
            raise ValueError("this stream was packed without a cold tier")
        if self.cold_on_host:
            return self._refine_host(rows)
        return self.settle_refine(self.refine_async(rows).cpu(), rows.numel())

    def settle_refine(self, counts: torch.Tensor, k: int) -> int:
        """The result of a ``refine_async`` of ``k`` rows, once its counts are on the host: the bytes
        fetched, or, when a row lay outside the stream (the kernel then merged nothing), the ``k``
        slots and the version bump given back and ValueError raised.  Every caller of
        ``refine_async`` settles its counts here."""
        if int(counts[1]):
            self.refined -= k
            self.version -= 1
            raise ValueError(f"refine rows must lie in 0..{self.n - 1}")
        return int(counts[0])

    def refine_async(self, rows: torch.Tensor) -> torch.Tensor:
        """Device cold tier: ``refine`` without a host round trip (dkv_refine_rows).  Returns a device
        int64 [2]: the bytes fetched and a flag set when a row lies outside the stream (then nothing
        was merged); the caller reads it (its synchronisation) and passes it to ``settle_refine``.
        Each distinct row's full blob goes to the slot of its first entry, so the refined area grows
        by ``rows.numel()`` slots (the host tier's ``refine`` uses one slot per distinct row)."""
        if self.cold is None or self.cold_on_host:
            raise ValueError("refine_async needs a device cold tier")
        device = self.blob.device
        k = rows.numel()
        if self.refined + k > self.refine_capacity:
            raise ValueError(f"refine capacity {self.refine_capacity} tokens exceeded")
        if self._owner is None:
            self._owner = torch.zeros(max(self.n, 1), dtype=torch.int64, device=device)
        self._refine_calls += 1
        counts = torch.zeros(2, dtype=torch.int64, device=device)
        if k:
            rows32 = rows.to(device=device, dtype=torch.int32).contiguous()
            base = self.hot_used + self.refined * self.tables.full_bytes
            dkv_hip.refine_rows(self.c_stream(), self.n, self.cold, self.cold_off, rows32, base, self.blob,
                                self.tok_off, self.pieces, self._owner, self._refine_calls, counts)
            self.refined += k
            self.version += 1
        return counts

    def _refine_host(self, rows: torch.Tensor) -> int:
        """Host cold tier: the rows come to the host (the cold blobs are gathered there); the byte
        count comes from the host mirror of the pieces; the gather runs over the distinct rows."""
        device = self.blob.device
        rows_h = rows.detach().to("cpu", torch.int64).numpy()
        if rows_h.min() < 0 or rows_h.max() >= self.n:
            raise ValueError(f"refine rows must lie in 0..{self.n - 1} (got {rows_h.min()}..{rows_h.max()})")
        fetched = int((self.tables.full_bytes - self._prefix_h[self._pieces_h[rows_h]]).sum())
        rows_np = np.unique(rows_h)  # rows_np and rows list the same tokens in the same order
        if rows_np.size != rows_h.size:
            rows = torch.from_numpy(rows_np.astype(np.int32)).to(device)
        else:
            rows_np = rows_h
            rows = rows.to(device=device, dtype=torch.int32).contiguous()
        k = rows.numel()
        if self.refined + k > self.refine_capacity:
            raise ValueError(f"refine capacity {self.refine_capacity} tokens exceeded")
        base = self.hot_used + self.refined * self.tables.full_bytes
        cold, cold_off = self._stage_cold(rows_np, rows)
        dkv_hip.gather_cold(self.c_stream(), cold, cold_off, rows, base, self.blob, self.tok_off, self.pieces)
        self._pieces_h[rows_np] = self.tables.pieces
        self.refined += k
        self.version += 1
        return fetched

    def _stage_cold(self, rows_np: np.ndarray, rows: torch.Tensor):
        """Host cold tier: gather the cold blobs of the distinct ``rows`` (host copy ``rows_np``, in
        the same order) into the pinned staging buffer, copy it to the device (one host-to-device
        transfer), and point each row's cold offset into the copy.  The buffers are kept and grow
        only when a refine needs more; before the host writes the pinned buffer again it waits for
        the previous copy out of it."""
        rows_h = torch.from_numpy(np.ascontiguousarray(rows_np, dtype=np.int64))
        start = self.cold_off[rows_h].numpy()
        size = self._cold_size0[rows_h].numpy()
        dst = np.zeros(size.size + 1, np.int64)
        np.cumsum(size, out=dst[1:])
        used = int(dst[-1])
        device = self.blob.device
        if self._stage_host is None or self._stage_host.numel() < max(used, 16):
            self._stage_host = torch.empty(max(used, 16), dtype=torch.uint8, pin_memory=True)
            self._stage_dev = torch.empty(max(used, 16), dtype=torch.uint8, device=device)
        elif self._stage_done is not None:
            self._stage_done.synchronize()
        if used:
            # one block copy per row (the pinned cold tier is best read in whole runs, not byte by byte)
            cold_np, staged_np = self.cold.numpy(), self._stage_host.numpy()
            for a, d, n in zip(start.tolist(), dst[:-1].tolist(), size.tolist()):
                staged_np[d:d + n] = cold_np[a:a + n]
            self._stage_dev[:used].copy_(self._stage_host[:used], non_blocking=True)
        self._stage_done = torch.cuda.Event()
        self._stage_done.record()
        self._stage_off[rows.long()] = torch.from_numpy(dst[:-1]).to(device, non_blocking=True)
        return self._stage_dev, self._stage_off


LADDER_GROUP = 64
LADDER_WIDTHS = (0, 2, 4, 8)


class LadderTables:
    """Device copies of one stream's kvtc rung ladder (scripts/kvtc.py:100-105 ``rungs`` [R, G]
    bit widths and ``rung_bytes``) plus each rung's segment offsets.  One more row, ``empty``
    (index R), has every group at 0 bits: the rung of a token whose coefficients are all dropped
    (an evicted value decodes to the mean, scripts/kvtc.py:245-247)."""

    def __init__(self, rungs, rung_bytes, device, group: int = LADDER_GROUP):
        if group != LADDER_GROUP:
            raise ValueError(f"the ladder kernels take groups of {LADDER_GROUP} components (got {group})")
        bits = np.asarray(torch.as_tensor(rungs).cpu(), dtype=np.int64)
        if bits.ndim != 2 or not np.isin(bits, LADDER_WIDTHS).all():
            raise ValueError(f"ladder bit widths must be a [rungs, groups] table over {LADDER_WIDTHS}")
        seg = np.where(bits > 0, HEADER_BYTES + bits * group // 8, 0)
        sizes = seg.sum(axis=1)
        if rung_bytes is not None and not np.array_equal(sizes, np.asarray(rung_bytes, dtype=np.int64)):
            raise ValueError("rung_bytes do not match the ladder (8b bytes + 4 B per group with b > 0)")
        bits = np.concatenate([bits, np.zeros((1, bits.shape[1]), np.int64)])
        seg = np.concatenate([seg, np.zeros((1, seg.shape[1]), np.int64)])
        seg_off = np.zeros_like(seg)
        seg_off[:, 1:] = np.cumsum(seg[:, :-1], axis=1)
        self.groups = bits.shape[1]
        self.rungs = bits.shape[0]
        self.empty = self.rungs - 1
        self.bits_np = bits
        self.bits = torch.as_tensor(bits.astype(np.uint8)).to(device)
        self.seg_off = torch.as_tensor(seg_off.astype(np.int32)).to(device)
        self.sizes64 = torch.as_tensor(seg.sum(axis=1)).to(device)
        self.rung_bytes = self.sizes64.to(torch.int32)

    def c_ladder(self) -> dkv_hip.Ladder:
        return dkv_hip.Ladder(self.groups, self.rungs, self.bits.data_ptr(), self.seg_off.data_ptr(),
                              self.rung_bytes.data_ptr())


class LadderStream:
    """kvtc ladder codes of one stream (keys or values) for n tokens (the ``dkvtc@`` hot tier)."""

    def __init__(self, tables: LadderTables, blob, tok_off, rung, used: int):
        self.tables = tables
        self.blob, self.tok_off, self.pieces = blob, tok_off, rung  # ``pieces`` holds each token's rung
        self.used = used
        self.version = 0

    @property
    def n(self) -> int:
        return self.pieces.numel()

    @classmethod
    def pack(cls, codes: torch.Tensor, low: torch.Tensor, scale: torch.Tensor, rung: torch.Tensor,
             tables: LadderTables) -> "LadderStream":
        """codes u8 [n, G, 64], low/scale f16 [n, G], rung [n] (-1 = every group dropped) -> one blob
        per token (GPU pack kernel)."""
        device = codes.device
        rung = rung.to(device=device, dtype=torch.int64)
        if rung.numel() and (int(rung.min()) < -1 or int(rung.max()) >= tables.empty):
            raise ValueError(f"rung ids must lie in -1..{tables.empty - 1}")
        rung = _nonnull(torch.where(rung < 0, torch.full_like(rung, tables.empty), rung).to(torch.int16).contiguous())
        sizes = tables.sizes64[rung.long()] if rung.numel() else torch.zeros(0, dtype=torch.int64, device=device)
        tok_off, total = _exclusive_cumsum(sizes)
        blob = torch.zeros(max(total, 16), dtype=torch.uint8, device=device)
        if rung.numel():
            dkv_hip.pack_ladder(codes.contiguous(), low.contiguous().view(torch.int16),
                                scale.contiguous().view(torch.int16), rung, tables.c_ladder(), blob, tok_off)
        return cls(tables, blob, tok_off, rung, total)

    def c_stream(self) -> dkv_hip.Stream:
        return dkv_hip.Stream(self.blob.data_ptr(), dkv_hip.addr(self.tok_off), dkv_hip.addr(self.pieces), dkv_hip.Order(),
                              dkv_hip.DKV_FMT_LADDER, self.tables.c_ladder())

    def dequantize(self, t0: int = 0, nt: int | None = None, dtype=torch.float32) -> torch.Tensor:
        """K1: coefficients [nt, 64G] of tokens t0.. (bit-exact with scripts/kvtc.py:78 in float32)."""
        nt = self.n - t0 if nt is None else nt
        out = torch.empty(nt, LADDER_GROUP * self.tables.groups, dtype=dtype, device=self.blob.device)
        if nt:
            dkv_hip.unpack_dequant(self.c_stream(), t0, nt, out)
        return out

    def hot_bytes(self) -> int:
        """Bytes held for this stream's tokens: the rung sizes (scripts/kvtc.py:243 accounting)."""
        return self.used

    def device_bytes(self) -> int:
        """GPU memory this stream holds: the blob as allocated, the per-token offsets and rungs."""
        return _nbytes(self.blob, self.tok_off, self.pieces)

    def refine(self, rows: torch.Tensor) -> int:
        raise ValueError("kvtc ladder streams have no cold tier to refine from")
