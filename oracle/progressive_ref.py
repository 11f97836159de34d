"""Progressive bit-plane codec restated in numpy (oracle; test infrastructure only).

Follows scripts/progressive.py of the reference:
- ``quantize8``   :37-44
- ``dequantize``  :47-55
- ``Order``       :58-64 (planes / prefix_bytes / rungs); the synthetic plane-major order
                  replaces ``build_order`` :67-100 (calibration, needs a model download)
- byte accounting of ``ProgressiveCache`` :185-194 (hot_bytes / cold_bytes) and
  ``refine``'s ``fetched`` :232
- ``encode`` error table + rung errors :150-166 (used by the config-4 encoder checks)

fp32 operation order is kept exactly: dequantize is
``low + ((idx + 0.5) * span) / 2**m`` with every product and sum rounded
separately (no fused multiply-add), which numpy float32 arithmetic does.

Pins (tests/test_oracle_progressive.py): exhaustive dequantize over all
256 codes x m in 0..8 on sampled fp16 (low, span) against exact rational
arithmetic rounded once per operation; quantize8 against its closed-form
bin property and nesting; byte totals against hand-computed formulas.
"""

from __future__ import annotations

import numpy as np

PLANES = 8
HEADER_BYTES = 4
RUNG_ID_BYTES = 1
PIECE_BYTES = 8


def quantize8(coefficients: np.ndarray, group: int = 64):
    """[tokens, features] f32 -> codes u8 [tokens, groups, group], low f16, span f16 [tokens, groups].

    progressive.py:37-44.  A degenerate group whose fp16 span rounds to 0
    gives 0/0 = NaN in the reference and an undefined uint8 cast; the
    build defines that case as code 0 (parity unpinned for it).
    """
    x = np.ascontiguousarray(coefficients, dtype=np.float32)
    tokens, features = x.shape
    grouped = x.reshape(tokens, features // group, group)
    low = grouped.min(axis=-1).astype(np.float16)
    span = np.maximum(grouped.max(axis=-1) - low.astype(np.float32), np.float32(1e-8)).astype(np.float16)
    with np.errstate(divide="ignore", invalid="ignore"):
        scaled = ((grouped - low.astype(np.float32)[..., None]) / span.astype(np.float32)[..., None]) * np.float32(256)
    scaled = np.floor(scaled)
    scaled = np.where(np.isnan(scaled), 0.0, np.clip(scaled, 0, 255))
    return scaled.astype(np.uint8), low, span


def dequantize(codes: np.ndarray, low: np.ndarray, span: np.ndarray, planes: np.ndarray) -> np.ndarray:
    """progressive.py:47-55.  ``planes`` is [tokens or 1, groups]; 0 planes -> 0.0."""
    m = planes.astype(np.int32)[..., None]
    shift = np.clip(PLANES - m, 0, PLANES)
    index = codes.astype(np.int32) >> shift
    bins = np.power(np.float32(2), m.astype(np.float32)).astype(np.float32)
    prod = ((index.astype(np.float32) + np.float32(0.5)) * span.astype(np.float32)[..., None]).astype(np.float32)
    value = (low.astype(np.float32)[..., None] + (prod / bins).astype(np.float32)).astype(np.float32)
    out = np.where(m > 0, value, np.float32(0)).astype(np.float32)
    return out.reshape(codes.shape[0], codes.shape[1] * codes.shape[2])


class Order:
    """progressive.py:58-64: planes [pieces+1, groups], prefix_bytes [pieces+1], rungs."""

    def __init__(self, planes: np.ndarray, prefix_bytes: np.ndarray, rungs: list[int]):
        self.planes = planes.astype(np.uint8)
        self.prefix_bytes = prefix_bytes.astype(np.int64)
        self.rungs = list(rungs)

    @property
    def groups(self) -> int:
        return self.planes.shape[1]

    @property
    def pieces(self) -> int:
        return self.planes.shape[0] - 1


def order_from_sequence(sequence: list[int], groups: int, rungs: list[int] | None = None) -> Order:
    """Order for a (group) sequence: piece k adds one plane to group sequence[k].

    Byte prefix follows progressive.py:87,90 (8 B per piece, +4 B on a group's
    first plane)."""
    level = np.zeros(groups, dtype=np.int64)
    planes, sizes = [level.copy()], [0]
    for g in sequence:
        sizes.append(sizes[-1] + PIECE_BYTES + (HEADER_BYTES if level[g] == 0 else 0))
        level[g] += 1
        if level[g] > PLANES:
            raise ValueError("group gets more than 8 planes")
        planes.append(level.copy())
    if rungs is None:
        rungs = list(range(len(sequence) + 1))
    return Order(np.stack(planes), np.array(sizes, dtype=np.int64), rungs)


def plane_major_order(groups: int) -> Order:
    """Synthetic order: plane 0 of every group, then plane 1, ... (planes[k,g] = k//G + (g < k%G))."""
    sequence = [g for _ in range(PLANES) for g in range(groups)]
    return order_from_sequence(sequence, groups, rungs=[groups * m for m in range(1, PLANES + 1)])


def token_planes(order: Order, pieces: np.ndarray) -> np.ndarray:
    """Per-token plane map [tokens, groups] = order.planes[pieces] (progressive.py:200)."""
    return order.planes[np.asarray(pieces, dtype=np.int64)]


def hot_bytes(orders: dict, pieces: dict, exact_tokens: int, exact_bytes: int) -> int:
    """progressive.py:185-188."""
    return exact_tokens * 2 * exact_bytes + sum(
        int(orders[kind].prefix_bytes[pieces[kind]].sum()) + RUNG_ID_BYTES * len(pieces[kind]) for kind in pieces)


def cold_bytes(orders: dict, pieces: dict) -> int:
    """progressive.py:191-194."""
    return sum(int((orders[kind].prefix_bytes[-1] - orders[kind].prefix_bytes[pieces[kind]]).sum()) for kind in pieces)


def fetched_bytes(orders: dict, pieces: dict, rows: np.ndarray) -> int:
    """progressive.py:232 summed over both streams."""
    return sum(int((orders[kind].prefix_bytes[-1] - orders[kind].prefix_bytes[pieces[kind][rows]]).sum())
               for kind in pieces)


def error_table(coefficients: np.ndarray, codes, low, span, group: int = 64) -> np.ndarray:
    """progressive.py:152-158: squared error of every (token, group) at 0..8 planes, [tokens, groups, 9] f32.

    fp32 sums over the 64 members follow numpy's pairwise order, which can
    differ from torch's in the last bit (parity unpinned at near-ties)."""
    tokens = coefficients.shape[0]
    grouped = coefficients.reshape(tokens, -1, group).astype(np.float32)
    groups = grouped.shape[1]
    out = np.empty((tokens, groups, PLANES + 1), dtype=np.float32)
    for m in range(PLANES + 1):
        rebuilt = dequantize(codes, low, span, np.full((1, groups), m)).reshape(grouped.shape)
        out[..., m] = np.square(grouped - rebuilt).sum(axis=-1, dtype=np.float32)
    return out


def rung_errors(coefficients: np.ndarray, table: np.ndarray, order: Order, weights: np.ndarray | None = None):
    """progressive.py:149-164: each token's error at every rung of ``order`` = the table's entries at
    the rung's plane counts summed over the groups, over the stream's mean token energy (float32,
    floored at 1e-12), times weights / mean(weights) when weights are given -> [tokens, rungs]."""
    x = np.asarray(coefficients, dtype=np.float32)
    energy = max(np.float32(np.square(x).sum(axis=1, dtype=np.float32).mean(dtype=np.float32)), np.float32(1e-12))
    rung_planes = order.planes[np.asarray(order.rungs)].astype(np.int64)  # [rungs, groups]
    groups = table.shape[1]
    picked = table[:, np.arange(groups)[None, :], rung_planes]  # [tokens, rungs, groups]
    out = (picked.sum(axis=2, dtype=np.float32) / energy).astype(np.float32)
    if weights is not None:
        w = np.asarray(weights, dtype=np.float32)
        out = (out * (w / max(np.float32(w.mean(dtype=np.float32)), np.float32(1e-12)))[:, None]).astype(np.float32)
    return out


def level_bytes(order: Order) -> list[int]:
    """progressive.py:166: bytes of each rung of ``order`` including the rung id."""
    return [int(order.prefix_bytes[k]) + RUNG_ID_BYTES for k in order.rungs]
