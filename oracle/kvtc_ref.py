"""kvtc ladder quantizer and the DimmerKV greedy allocator, restated in numpy
(oracle; test infrastructure only).

Follows scripts/kvtc.py of the reference:
- ``quantize_groups`` :62-79 (round half to even, fp16 low/scale), split into
  ``quantize_groups_codes`` (the integer codes and fp16 low/scale that
  scripts/kvtc_storage.py:63-73 stores) and ``dequantize_codes``
  (code * scale + low, scripts/kvtc.py:78 and kvtc_storage.py:119)
- ``rung_bytes``      :82-85
- ``allocate_rungs``  :277-298 (fp64 values, cummin along levels, *stable*
  descending sort, take the sorted prefix whose cumulative cost fits)
- ``compress_choice`` :157-233 (``KVTCCodec.compress`` up to the rung choice:
  span, budget split, per-token relative errors over the stream's energy,
  importance weights, key weight, the eviction level, the floor, allocation
  over the levels from the floor up)

Pins (tests/test_oracle_kvtc_scoring_packing.py, tests/test_oracle_compress_choice.py):
compress_choice against a per-token plain-Python statement, the floor against
enumeration of the uniform rungs, and invariants that a dropped term breaks
(key-only rescaling by a power of two leaves the choice unchanged only with the
energy normalisation; zero-importance tokens stay at the floor; evicted keys
evict their values; bytes within the budget); allocate_rungs against an exhaustive
brute force of the same greedy rule on tiny inputs, against the invariants
(budget respected, per-slot upgrades form a prefix), and against torch's
stable sort on random inputs; quantize_groups against its closed-form grid
and against dequantize_codes(quantize_groups_codes(.)) bit for bit.
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


def quantize_groups_codes(coefficients: np.ndarray, bits: np.ndarray, group: int):
    """The integer side of kvtc.py:62-79: codes u8 [tokens, groups, group], low and scale f16
    [tokens, groups] (scripts/kvtc_storage.py:70-73); groups with 0 bits get zeros."""
    x = coefficients.astype(np.float32)
    tokens, features = x.shape
    groups = features // group
    grouped = x.reshape(tokens, groups, group)
    codes = np.zeros((tokens, groups, group), np.uint8)
    low16 = np.zeros((tokens, groups), np.float16)
    scale16 = np.zeros((tokens, groups), np.float16)
    for width in BIT_OPTIONS[1:]:
        chosen = np.nonzero(bits == width)[0]
        if chosen.size == 0:
            continue
        part = grouped[:, chosen]
        lo = part.min(axis=-1, keepdims=True).astype(np.float16)
        sc = np.maximum((part.max(axis=-1, keepdims=True) - lo.astype(np.float32)) / np.float32(2**width - 1),
                        np.float32(1e-8)).astype(np.float16)
        q = np.clip(np.rint((part - lo.astype(np.float32)) / sc.astype(np.float32)), 0, 2**width - 1)
        codes[:, chosen] = q.astype(np.uint8)
        low16[:, chosen] = lo[..., 0]
        scale16[:, chosen] = sc[..., 0]
    return codes, low16, scale16


def dequantize_codes(codes: np.ndarray, low: np.ndarray, scale: np.ndarray, bits: np.ndarray) -> np.ndarray:
    """code * scale + low in float32, product and sum rounded separately (kvtc.py:78); 0 where a
    group has 0 bits.  ``bits`` is [groups] or [tokens, groups]."""
    c = codes.astype(np.float32)
    prod = (c * scale.astype(np.float32)[..., None]).astype(np.float32)
    out = (prod + low.astype(np.float32)[..., None]).astype(np.float32)
    b = np.broadcast_to(bits, low.shape)
    out[b == 0] = 0.0
    return out.reshape(codes.shape[0], codes.shape[1] * codes.shape[2])


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


def compress_choice(matrices: dict, means: dict, bases: dict, rungs: dict, rung_bytes: dict, exact_bytes: int,
                    sinks: int, exact_recent: int, budget: float, group: int = 64, weights=None, evict: bool = False,
                    floor_share: float = 0.0, key_weight: float = 1.0, coefficients: dict | None = None) -> dict:
    """The per-token rung choice of ``KVTCCodec.compress(..., per_token=True)`` (kvtc.py:157-233).

    ``matrices[kind]`` float32 [tokens, features] are the token matrices (keys already without
    RoPE, kvtc.py:188), ``means``/``bases`` the stream calibration, ``rungs[kind]`` [R, groups] bit
    widths and ``rung_bytes[kind]`` their sizes.  ``coefficients[kind]`` [middle, rank], when given,
    replaces the projection (X - mean) @ basis of the middle tokens (kvtc.py:189), so a caller can
    feed the exact values another implementation projected.  Returns {"key", "value": int64
    [middle] rungs (-1 evicted, R = exact), "span": (start, end), "budget_bytes", "remaining",
    "first" (the floor level), "errors": float32 [2 * middle, levels]}."""
    tokens = matrices["key"].shape[0]
    start = min(sinks, tokens)  # kvtc.py:177-180
    end = max(start, tokens - exact_recent)
    middle = end - start
    budget_bytes = int(budget * tokens * 2 * exact_bytes)  # kvtc.py:182-183
    remaining = budget_bytes - (tokens - middle) * 2 * exact_bytes
    errors = []
    for kind in ("key", "value"):
        centred = (matrices[kind][start:end].astype(np.float32) - means[kind].astype(np.float32)).astype(np.float32)
        coef = coefficients[kind] if coefficients is not None else (centred @ bases[kind].astype(np.float32))
        coef = np.asarray(coef, dtype=np.float32)
        energy = np.float32(np.square(centred).sum(axis=1, dtype=np.float32).mean(dtype=np.float32)) if middle else \
            np.float32(0)  # :190-191
        per_rung = [np.square(coef - quantize_groups(coef, bits, group)).sum(axis=1, dtype=np.float32)
                    for bits in np.asarray(rungs[kind])]
        columns = [(np.stack(per_rung, axis=1) / energy).astype(np.float32), np.zeros((middle, 1), np.float32)]
        if evict:  # :195-197, the whole centred vector is lost
            columns.insert(0, (np.square(coef).sum(axis=1, dtype=np.float32) / energy)[:, None].astype(np.float32))
        err = np.concatenate(columns, axis=1)
        if weights is not None:  # :198-201
            w = np.asarray(weights, dtype=np.float32)[start:end]
            err = (err * (w / max(np.float32(w.mean(dtype=np.float32)), np.float32(1e-12)))[:, None]).astype(np.float32)
        if kind == "key":  # :202-203
            err = (err * np.float32(key_weight)).astype(np.float32)
        errors.append(err)
    level_bytes = {kind: list(rung_bytes[kind]) + [exact_bytes] for kind in ("key", "value")}  # :206
    evict_bytes = [0] if evict else []
    first = 0
    if floor_share > 0:  # :209-214
        fits = [r for r in range(len(level_bytes["key"]))
                if middle * (level_bytes["key"][r] + level_bytes["value"][r]) <= floor_share * remaining]
        first = len(evict_bytes) + (max(fits) if fits else 0)
    levels = np.concatenate([np.asarray(evict_bytes + level_bytes[kind], dtype=np.float64)[first:]
                             for kind in ("key", "value")])
    all_errors = np.concatenate([e[:, first:] for e in errors])
    chosen = allocate_rungs(all_errors, levels, middle, remaining) + first - len(evict_bytes)  # :215-219
    key, value = chosen[:middle].copy(), chosen[middle:].copy()
    value[key < 0] = -1  # :220-221
    return {"key": key, "value": value, "span": (start, end), "budget_bytes": budget_bytes, "remaining": remaining,
            "first": first, "errors": np.concatenate(errors)}
