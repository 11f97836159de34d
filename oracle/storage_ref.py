"""kvtc byte storage restated in numpy (oracle; test infrastructure only).

Follows scripts/kvtc_storage.py of the reference:
- ``pack_codes`` / ``unpack_codes`` / ``packed_length``  :21-38 (``_pack``, ``_unpack``,
  ``_packed_length``): codes below 2^w, 8 // w per byte, code k of a byte at bit w*k
  (LSB-first), the last byte zero-padded
- ``encode``  :42-79 (``encode_bytes``) on arrays: an int32 header (tokens, start, end), then
  per stream (keys, values) the rung id of every compressed token (1 byte), then for each rung
  present, in increasing order, either the fp16 matrix rows of its tokens (the exact rung) or,
  for each width 2, 4, 8 the rung uses, the packed codes of (its tokens x the groups of that
  width), their fp16 shifts and their fp16 scales; then the exact tokens (sinks and recent
  window) as fp16 rows
- ``decode``  :82-135 (``decode_bytes``) down to the dequantized coefficients (code * scale +
  shift in float32, zeros for dropped groups and exact-rung rows), the exact-rung rows and the
  exact tokens; the inverse transform and RoPE are the codec's and are left to the caller
- ``stored_bytes``: the length ``encode`` writes, from the rung sizes (scripts/kvtc.py:82-85)

The quantizer is ``kvtc_ref.quantize_groups_codes`` (pinned there).  Pins
(tests/test_oracle_storage.py): a hand-written byte string for a small cache (header, rung ids,
rung and width order, LSB-first packing, fp16 byte order, exact rows and tokens), hand-computed
packings, decode(encode(x)) equal to kvtc_ref.quantize_groups bit for bit (the reference's own
check: the restored cache equals the in-memory compressed one, FINDINGS.md:468-469), the byte
count against the closed form, and numpy's own bit packing for width 1 layouts.
"""

from __future__ import annotations

import numpy as np

from . import kvtc_ref

WIDTHS = (2, 4, 8)
HEADER = np.dtype("<i4")


def packed_length(count: int, width: int) -> int:
    per = 8 // width
    return (count + per - 1) // per


def pack_codes(codes: np.ndarray, width: int) -> bytes:
    """Flat codes below 2^width -> bytes, code k of each byte at bit width*k."""
    per = 8 // width
    flat = np.asarray(codes, dtype=np.uint32).ravel()
    flat = np.concatenate([flat, np.zeros((-flat.size) % per, np.uint32)]).reshape(-1, per)
    shifts = (np.arange(per, dtype=np.uint32) * width)[None, :]
    return (flat << shifts).sum(axis=1).astype(np.uint8).tobytes()


def unpack_codes(data: bytes, width: int, count: int) -> np.ndarray:
    per = 8 // width
    packed = np.frombuffer(data, dtype=np.uint8).astype(np.uint32)
    shifts = (np.arange(per, dtype=np.uint32) * width)[None, :]
    return ((packed[:, None] >> shifts) & np.uint32(2**width - 1)).ravel()[:count].astype(np.uint8)


def _stream_parts(rungs: np.ndarray, bits: np.ndarray, coefficients: np.ndarray, matrix_rows: np.ndarray,
                  exact_tokens: np.ndarray, group: int) -> list[bytes]:
    rungs = np.asarray(rungs, dtype=np.int64)
    if (rungs < 0).any():
        raise NotImplementedError("Byte storage does not support evicted tokens yet.")
    exact_rung = bits.shape[0]
    parts = [rungs.astype(np.uint8).tobytes()]
    for rung in np.unique(rungs):
        rows = rungs == rung
        if rung == exact_rung:
            parts.append(matrix_rows[rows].astype(np.float16).tobytes())
            continue
        row_bits = bits[rung]
        codes, low, scale = kvtc_ref.quantize_groups_codes(coefficients[rows], row_bits, group)
        for width in WIDTHS:
            chosen = np.nonzero(row_bits == width)[0]
            if chosen.size == 0:
                continue
            parts += [pack_codes(codes[:, chosen], width), low[:, chosen].astype("<f2").tobytes(),
                      scale[:, chosen].astype("<f2").tobytes()]
    parts.append(exact_tokens.astype("<f2").tobytes())
    return parts


def encode(tokens: int, start: int, end: int, streams: list[dict], group: int) -> bytes:
    """``streams`` = [keys, values], each a dict with ``rungs`` [middle] (0..R, R = the exact
    rung), ``bits`` [R, groups], ``coefficients`` float32 [middle, rank], ``matrix_rows`` float32
    [middle, features] (the codec's pre-RoPE token matrix rows) and ``exact_tokens`` float32
    [tokens - middle, features] (token matrix rows of the sinks and the recent window)."""
    parts = [np.asarray([tokens, start, end], dtype=HEADER).tobytes()]
    for s in streams:
        parts += _stream_parts(s["rungs"], np.asarray(s["bits"]), np.asarray(s["coefficients"], np.float32),
                               np.asarray(s["matrix_rows"], np.float32), np.asarray(s["exact_tokens"], np.float32),
                               group)
    return b"".join(parts)


def decode(data: bytes, metas: list[dict], group: int) -> dict:
    """Inverse of ``encode`` down to codes: ``metas`` = [keys, values] with ``bits`` [R, groups],
    ``rank`` and ``features``.  Returns {"header": (tokens, start, end), "streams": [per stream
    {"rungs", "coefficients" float32 [middle, rank], "exact_rows" (indices, fp16 rows),
    "exact_tokens" fp16 [tokens - middle, features]}]}; raises ValueError if bytes are left."""
    offset = 0

    def read(dtype, count):
        nonlocal offset
        arr = np.frombuffer(data, dtype=dtype, count=count, offset=offset)
        offset += arr.nbytes
        return arr

    tokens, start, end = (int(v) for v in read(HEADER, 3))
    middle = end - start
    out = []
    for meta in metas:
        bits, rank, features = np.asarray(meta["bits"]), int(meta["rank"]), int(meta["features"])
        exact_rung = bits.shape[0]
        rungs = read(np.uint8, middle).astype(np.int64)
        coefficients = np.zeros((middle, rank), np.float32)
        exact_rows = (np.zeros(0, np.int64), np.zeros((0, features), np.float16))
        for rung in np.unique(rungs):
            rows = np.nonzero(rungs == rung)[0]
            count = rows.size
            if rung == exact_rung:
                exact_rows = (rows, read("<f2", count * features).reshape(count, features).copy())
                continue
            groups = rank // group
            codes = np.zeros((count, groups, group), np.uint8)
            low = np.zeros((count, groups), np.float16)
            scale = np.zeros((count, groups), np.float16)
            row_bits = bits[rung]
            for width in WIDTHS:
                chosen = np.nonzero(row_bits == width)[0]
                if chosen.size == 0:
                    continue
                n_codes = count * chosen.size * group
                packed = read(np.uint8, packed_length(n_codes, width)).tobytes()
                codes[:, chosen] = unpack_codes(packed, width, n_codes).reshape(count, chosen.size, group)
                low[:, chosen] = read("<f2", count * chosen.size).reshape(count, chosen.size)
                scale[:, chosen] = read("<f2", count * chosen.size).reshape(count, chosen.size)
            coefficients[rows] = kvtc_ref.dequantize_codes(codes, low, scale, row_bits)
        exact_tokens = read("<f2", (tokens - middle) * features).reshape(tokens - middle, features).copy()
        out.append({"rungs": rungs, "coefficients": coefficients, "exact_rows": exact_rows,
                    "exact_tokens": exact_tokens})
    if offset != len(data):
        raise ValueError(f"Decoded {offset} of {len(data)} bytes.")
    return {"header": (tokens, start, end), "streams": out}


def stored_bytes(tokens: int, middle: int, streams: list[dict], group: int) -> int:
    """12 header bytes + per stream: one rung id per compressed token, each token's rung size
    (scripts/kvtc.py:82-85; 2 bytes per feature at the exact rung) and the fp16 exact tokens.
    Holds when 64 codes of every width fill whole bytes (group * width % 8 == 0)."""
    total = HEADER.itemsize * 3
    for s in streams:
        bits, features = np.asarray(s["bits"]), int(s["features"])
        rungs = np.asarray(s["rungs"], np.int64)
        sizes = [kvtc_ref.rung_bytes(bits[r], group) for r in range(bits.shape[0])] + [2 * features]
        total += middle + sum(sizes[r] for r in rungs) + (tokens - middle) * features * 2
    return total
