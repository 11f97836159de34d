"""Packed hot/cold bit-plane layout (oracle; test infrastructure only).

The reference keeps progressive codes unpacked (scripts/progressive.py:103-110)
and only *counts* their bytes: 8 B per (group, plane) piece plus a 4 B fp16
offset/range header with a group's first plane (progressive.py:12-13, 32-34,
87-90, 185-194).  This build stores exactly those bytes.  This module is the
numpy statement of that layout, used to check the GPU packer and unpacker
bit for bit.

Layout of one stream ("DKV1"):

* Token ``t`` keeps the first ``k_t`` pieces of its stream's order in the hot
  tier, so group ``g`` holds ``m = order.planes[k_t, g]`` planes.
* Hot token blob = for every group with m > 0, in group order, a segment
  ``[low f16][span f16][m plane words of 8 B, plane 0 (the MSB) first]``.
  Its size is ``order.prefix_bytes[k_t]`` exactly.
* Cold token blob = for every group with m < m_full (m_full = the group's
  planes in the order's full state, 8 for a complete order), in group order,
  ``[low f16][span f16, only if m == 0][plane words m..m_full-1]``; its size is
  ``prefix_bytes[-1] - prefix_bytes[k_t]`` (the reference's ``fetched``).
* A plane word is two little-endian u32 halves; half h holds coefficients
  32h..32h+31.  Coefficient ``32h + 4w + i`` (w in 0..7, i in 0..3) of plane p
  sits at bit ``(8i + w + 7 - p) mod 32`` of its half, and the bit is bit
  ``7 - p`` of that coefficient's 8-bit code.  This permutation lets a GPU
  lane rebuild four 8-bit codes with one AND-OR per plane and one rotate
  (rotr(OR_p(word_p & mask(p, w)), w) has byte i = code of coefficient 4w+i
  truncated to the present planes).

kvtc ladder streams (the ``dkvtc@`` entry point; ``pack_ladder``): token t at
rung r has one blob of ``rung_bytes[r]`` bytes: for every group with b > 0
bits, in group order, ``[low f16][scale f16][64 codes of b bits]``, the codes
LSB-first (code j at bit b*j of the code bytes: the bit order of
scripts/kvtc_storage.py:21-27 ``_pack``, applied to one (token, group) at a
time, which is whole bytes since 64b is a multiple of 8).

Pins (tests/test_oracle_kvtc_scoring_packing.py): per-plane bit positions are
a bijection, pack/unpack round-trips, both tiers' byte sizes equal the
reference's counts, and the lane formula above rebuilds the truncated codes;
ladder code bytes against hand-computed bytes and numpy.packbits(bitorder=
"little") of each code's bits, blob sizes against kvtc_ref.rung_bytes.
"""

from __future__ import annotations

import numpy as np

from .progressive_ref import HEADER_BYTES, PIECE_BYTES, Order


def bit_position(coef: np.ndarray, plane: int) -> np.ndarray:
    """Bit index (0..63) inside the 64-bit plane word of a coefficient index (0..63)."""
    coef = np.asarray(coef)
    half, j = coef // 32, coef % 32
    w, i = j // 4, j % 4
    return half * 32 + (8 * i + w + 7 - plane) % 32


def plane_word(codes64: np.ndarray, plane: int) -> np.uint64:
    """64 codes (u8) -> the 8-byte word of bit-plane ``plane`` (0 = MSB)."""
    bits = (codes64.astype(np.uint64) >> np.uint64(7 - plane)) & np.uint64(1)
    pos = bit_position(np.arange(64), plane).astype(np.uint64)
    return np.uint64(np.bitwise_or.reduce(bits << pos))


def word_codes(word: int, plane: int) -> np.ndarray:
    """Inverse of ``plane_word`` for one plane: 64 bits (0/1) in coefficient order."""
    pos = bit_position(np.arange(64), plane).astype(np.uint64)
    return ((np.uint64(word) >> pos) & np.uint64(1)).astype(np.uint8)


def segment_offsets(order: Order) -> np.ndarray:
    """seg_off[k, g]: byte offset of group g's hot segment in a token blob with k hot pieces."""
    m = order.planes.astype(np.int64)
    seg = np.where(m > 0, HEADER_BYTES + PIECE_BYTES * m, 0)
    off = np.zeros_like(seg)
    off[:, 1:] = np.cumsum(seg[:, :-1], axis=1)
    return off.astype(np.int32)


def cold_segment_offsets(order: Order) -> np.ndarray:
    """cold_off[k, g]: byte offset of group g's cold segment in a cold blob (k hot pieces)."""
    m = order.planes.astype(np.int64)
    m_full = m[-1][None, :]
    seg = np.where((m == 0) & (m_full > 0), HEADER_BYTES, 0) + PIECE_BYTES * np.maximum(m_full - m, 0)
    off = np.zeros_like(seg)
    off[:, 1:] = np.cumsum(seg[:, :-1], axis=1)
    return off.astype(np.int32)


def _header_bytes(low, span) -> bytes:
    return np.array([low], dtype=np.float16).tobytes() + np.array([span], dtype=np.float16).tobytes()


def pack(codes: np.ndarray, low: np.ndarray, span: np.ndarray, pieces: np.ndarray, order: Order):
    """codes u8 [T, G, 64], low/span f16 [T, G], pieces [T] -> (hot blob, hot offsets[T+1], cold blob, cold offsets[T+1])."""
    tokens, groups, _ = codes.shape
    hot, cold = bytearray(), bytearray()
    hot_off, cold_off = [0], [0]
    m_full = order.planes[-1]
    for t in range(tokens):
        m_all = order.planes[int(pieces[t])]
        for g in range(groups):
            m = int(m_all[g])
            if m > 0:
                hot += _header_bytes(low[t, g], span[t, g])
                for p in range(m):
                    hot += int(plane_word(codes[t, g], p)).to_bytes(8, "little")
        for g in range(groups):
            m, mf = int(m_all[g]), int(m_full[g])
            if m == 0 and mf > 0:
                cold += _header_bytes(low[t, g], span[t, g])
            for p in range(m, mf):
                cold += int(plane_word(codes[t, g], p)).to_bytes(8, "little")
        hot_off.append(len(hot))
        cold_off.append(len(cold))
    return (np.frombuffer(bytes(hot), dtype=np.uint8), np.array(hot_off, dtype=np.int64),
            np.frombuffer(bytes(cold), dtype=np.uint8), np.array(cold_off, dtype=np.int64))


def plane_words(codes: np.ndarray) -> np.ndarray:
    """codes u8 [..., 64] -> the eight plane words [..., 8] (uint64, plane 0 = MSB first), vectorised
    ``plane_word``."""
    c = codes.astype(np.uint64)
    words = np.zeros(codes.shape[:-1] + (8,), dtype=np.uint64)
    members = np.arange(64)
    for p in range(8):
        bits = (c >> np.uint64(7 - p)) & np.uint64(1)
        words[..., p] = np.bitwise_or.reduce(bits << bit_position(members, p).astype(np.uint64), axis=-1)
    return words


def pack_fast(codes: np.ndarray, low: np.ndarray, span: np.ndarray, pieces: np.ndarray, order: Order):
    """``pack`` vectorised over tokens (same four results): every (token, group) is laid out as
    [low][span][8 plane words] (68 bytes) and the bytes of each tier are selected from it in
    (token, group, byte) order."""
    tokens, groups, _ = codes.shape
    full = np.empty((tokens, groups, HEADER_BYTES + 8 * PIECE_BYTES), dtype=np.uint8)
    full[..., 0:2] = np.ascontiguousarray(low, dtype=np.float16).view(np.uint8).reshape(tokens, groups, 2)
    full[..., 2:4] = np.ascontiguousarray(span, dtype=np.float16).view(np.uint8).reshape(tokens, groups, 2)
    full[..., 4:] = plane_words(codes).astype("<u8").view(np.uint8).reshape(tokens, groups, 8 * PIECE_BYTES)
    m = order.planes[np.asarray(pieces, dtype=np.int64)].astype(np.int64)[..., None]  # [T, G, 1]
    mf = order.planes[-1].astype(np.int64)[None, :, None]
    b = np.arange(full.shape[-1])
    plane = (b - HEADER_BYTES) // PIECE_BYTES  # plane of a word byte (negative for the header)
    is_header = b < HEADER_BYTES
    hot_mask = (m > 0) & (is_header | (plane < m))
    cold_mask = (is_header & (m == 0) & (mf > 0)) | (~is_header & (plane >= m) & (plane < mf))
    hot, cold = full[hot_mask], full[cold_mask]
    hot_off = np.zeros(tokens + 1, dtype=np.int64)
    cold_off = np.zeros(tokens + 1, dtype=np.int64)
    np.cumsum(hot_mask.reshape(tokens, -1).sum(axis=1), out=hot_off[1:])
    np.cumsum(cold_mask.reshape(tokens, -1).sum(axis=1), out=cold_off[1:])
    return hot, hot_off, cold, cold_off


def unpack(blob: np.ndarray, offsets: np.ndarray, pieces: np.ndarray, order: Order, groups: int):
    """Hot blob -> (codes u8 [T,G,64] truncated to the hot planes, low f16, span f16, planes [T,G])."""
    tokens = len(pieces)
    codes = np.zeros((tokens, groups, 64), dtype=np.uint8)
    low = np.zeros((tokens, groups), dtype=np.float16)
    span = np.zeros((tokens, groups), dtype=np.float16)
    seg = segment_offsets(order)
    raw = blob.tobytes()
    for t in range(tokens):
        k = int(pieces[t])
        for g in range(groups):
            m = int(order.planes[k, g])
            if m == 0:
                continue
            base = int(offsets[t]) + int(seg[k, g])
            low[t, g] = np.frombuffer(raw[base:base + 2], dtype=np.float16)[0]
            span[t, g] = np.frombuffer(raw[base + 2:base + 4], dtype=np.float16)[0]
            acc = np.zeros(64, dtype=np.uint8)
            for p in range(m):
                word = int.from_bytes(raw[base + 4 + 8 * p: base + 12 + 8 * p], "little")
                acc |= (word_codes(word, p) << (7 - p)).astype(np.uint8)
            codes[t, g] = acc
    return codes, low, span, order.planes[np.asarray(pieces, dtype=np.int64)]


def ladder_segment_offsets(bits: np.ndarray, group: int = 64) -> np.ndarray:
    """Byte offset of group g's segment in a token blob at rung r: [R, G]."""
    seg = np.where(bits > 0, HEADER_BYTES + bits * group // 8, 0).astype(np.int64)
    off = np.zeros_like(seg)
    off[:, 1:] = np.cumsum(seg[:, :-1], axis=1)
    return off


def pack_ladder_codes(codes64: np.ndarray, width: int) -> bytes:
    """64 codes of ``width`` bits, LSB-first: code j occupies bits width*j .. width*j+width-1."""
    out = bytearray(len(codes64) * width // 8)
    for j, c in enumerate(codes64.astype(np.int64)):
        bit = width * j
        out[bit // 8] |= (int(c) & ((1 << width) - 1)) << (bit % 8)
    return bytes(out)


def pack_ladder(codes: np.ndarray, low: np.ndarray, scale: np.ndarray, rung: np.ndarray, bits: np.ndarray,
                group: int = 64):
    """codes u8 [n, G, 64], low/scale f16 [n, G], rung [n] (rows of ``bits`` [R, G]) -> (blob u8,
    offsets int64 [n+1])."""
    parts, offsets = [], [0]
    for t in range(codes.shape[0]):
        row = bits[rung[t]]
        blob = bytearray()
        for g in np.nonzero(row > 0)[0]:
            blob += _header_bytes(low[t, g], scale[t, g])
            blob += pack_ladder_codes(codes[t, g], int(row[g]))
        parts.append(bytes(blob))
        offsets.append(offsets[-1] + len(blob))
    return np.frombuffer(b"".join(parts), np.uint8).copy(), np.asarray(offsets, np.int64)
