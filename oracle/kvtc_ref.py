"""kvtc ladder quantizer and the DimmerKV greedy allocator, restated in numpy
(oracle; test infrastructure only).

Follows scripts/kvtc.py of the reference:
- ``quantize_groups`` :62-79 (round half to even, fp16 low/scale)
- ``rung_bytes``      :82-85
- ``allocate_rungs``  :277-298 (fp64 values, cummin along levels, *stable*
  descending sort, take the sorted prefix whose cumulative cost fits)

Pins (tests/test_oracle_kvtc_scoring_packing.py): allocate_rungs against an exhaustive
brute force of the same greedy rule on tiny inputs, against the invariants
(budget respected, per-slot upgrades form a prefix), and against torch's
stable sort on random inputs; quantize_groups against its closed-form grid.
"""

from __future__ import annotations

import numpy as np

GROUP_BYTES_OVERHEAD = 4
BIT_OPTIONS = (0, 2, 4, 8)


def quantize_groups(coefficients: np.ndarray, bits: np.ndarray, group: int) -> np.ndarray:
    """kvtc.py:62-79 quantize-dequantize with per-group bit widths (0 = dropped)."""
    x = coefficients.astype(np.float32)
    tokens, features = x.shape
    grouped = x.reshape(tokens, features // group, group)
    out = np.zeros_like(grouped)
    for width in BIT_OPTIONS[1:]:
        chosen = np.nonzero(bits == width)[0]
        if chosen.size == 0:
            continue
        part = grouped[:, chosen]
        low = part.min(axis=-1, keepdims=True).astype(np.float16).astype(np.float32)
        scale = np.maximum((part.max(axis=-1, keepdims=True) - low) / np.float32(2**width - 1),
                           np.float32(1e-8)).astype(np.float16).astype(np.float32)
        q = np.clip(np.rint((part - low) / scale), 0, 2**width - 1).astype(np.float32)
        out[:, chosen] = (q * scale).astype(np.float32) + low
    return out.reshape(tokens, features)


def rung_bytes(bits: np.ndarray, group: int) -> int:
    """kvtc.py:82-85."""
    used = bits > 0
    return int((bits.astype(np.float32) * group / 8).sum() + GROUP_BYTES_OVERHEAD * used.sum())


def allocate_rungs(errors: np.ndarray, level_bytes: np.ndarray, middle: int, budget: int) -> np.ndarray:
    """kvtc.py:277-298.  errors [slots, levels] (first ``middle`` slots keys, then values),
    level_bytes = key levels then value levels.  Returns per-slot upgrade counts."""
    slots, levels = errors.shape
    sizes = np.repeat(np.asarray(level_bytes, dtype=np.float64).reshape(2, levels), middle, axis=0)
    base = int(sizes[:, 0].sum())
    if base > budget:
        raise ValueError("Budget cannot cover the coarsest rung for every token.")
    err = errors.astype(np.float32)
    gains = np.maximum(err[:, :-1] - err[:, 1:], np.float32(0)).astype(np.float64)
    costs = sizes[:, 1:] - sizes[:, :-1]
    value = np.minimum.accumulate(gains / costs, axis=1)
    # Stable descending sort: ties keep index order.  argsort of the negated
    # values with a stable kind gives the same permutation.
    order = np.argsort(-value.reshape(-1), kind="stable")
    taken = order[np.cumsum(costs.reshape(-1)[order]) <= budget - base]
    counts = np.zeros(slots, dtype=np.int64)
    np.add.at(counts, taken // (levels - 1), 1)
    return counts
