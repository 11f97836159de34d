"""Pins of oracle/kvtc_ref.compress_choice, the per-token rung choice of KVTCCodec.compress
(scripts/kvtc.py:157-233), on the CPU.

- A per-token plain-Python statement (float64 errors, one token at a time, the greedy rule
  as a sorted item list) gives the same choices on small random caches, with and without
  importance weights, key weight, eviction level and floor.
- The floor is the finest uniform rung whose bytes fit floor_share of the remaining budget,
  found by enumeration, and no slot lies below it.
- Rescaling only the keys around their mean by a power of two leaves the choice unchanged
  (errors and energy scale alike); the same statement without the energy normalisation
  changes it, so a dropped normalisation would fail.
- Tokens of zero importance are never upgraded above the floor under a tight budget.
- With eviction, an evicted key evicts its value, and evicted slots cost nothing.
- Every choice fits the budget left after the exact tokens.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import kvtc_ref

GROUP = 64


def _setup(seed: int, tokens: int = 40, features: int = 128, rank: int = 128):
    rng = np.random.default_rng(seed)
    bases, means, matrices = {}, {}, {}
    scale = (np.arange(1, rank + 1) ** -0.75).astype(np.float32)
    for i, kind in enumerate(("key", "value")):
        q, _ = np.linalg.qr(rng.standard_normal((features, features)))
        bases[kind] = q[:, :rank].astype(np.float32)
        means[kind] = (rng.standard_normal(features) * 0.05).astype(np.float32)
        coef = rng.standard_normal((tokens, rank)).astype(np.float32) * scale * (1.0 + 0.5 * i)
        matrices[kind] = (means[kind] + coef @ bases[kind].T).astype(np.float32)
    groups = rank // GROUP
    ladder = np.array([[2, 0], [4, 0], [4, 2], [8, 4], [8, 8]][: 5], dtype=np.int64)[:, :groups]
    rungs = {kind: ladder for kind in ("key", "value")}
    rung_bytes = {kind: [kvtc_ref.rung_bytes(b, GROUP) for b in ladder] for kind in ("key", "value")}
    return matrices, means, bases, rungs, rung_bytes, 2 * features


def _plain(matrices, means, bases, rungs, rung_bytes, exact_bytes, sinks, recent, budget, weights=None,
           evict=False, floor_share=0.0, key_weight=1.0, normalise=True):
    """One token at a time in float64, the greedy rule as an explicit sorted item list."""
    tokens = matrices["key"].shape[0]
    start = min(sinks, tokens)
    end = max(start, tokens - recent)
    middle = end - start
    budget_bytes = int(budget * tokens * 2 * exact_bytes)
    remaining = budget_bytes - (tokens - middle) * 2 * exact_bytes
    errs = {}
    for kind in ("key", "value"):
        rows = []
        centred = [matrices[kind][start + t].astype(np.float64) - means[kind] for t in range(middle)]
        energy = np.mean([float(np.dot(c, c)) for c in centred]) if normalise else 1.0
        for t in range(middle):
            coef = (centred[t] @ bases[kind].astype(np.float64)).astype(np.float32)[None]
            row = []
            if evict:
                row.append(float(np.sum(coef.astype(np.float64) ** 2)) / energy)
            for bits in rungs[kind]:
                rebuilt = kvtc_ref.quantize_groups(coef, bits, GROUP)
                row.append(float(np.sum((coef.astype(np.float64) - rebuilt) ** 2)) / energy)
            row.append(0.0)
            if weights is not None:
                w = np.asarray(weights, np.float64)[start:end]
                row = [x * w[t] / max(w.mean(), 1e-12) for x in row]
            if kind == "key":
                row = [x * key_weight for x in row]
            rows.append(row)
        errs[kind] = rows
    sizes = {kind: ([0] if evict else []) + list(rung_bytes[kind]) + [exact_bytes] for kind in ("key", "value")}
    first = 0
    if floor_share > 0:
        plain_sizes = {kind: list(rung_bytes[kind]) + [exact_bytes] for kind in ("key", "value")}
        best = 0
        for r in range(len(plain_sizes["key"])):
            if middle * (plain_sizes["key"][r] + plain_sizes["value"][r]) <= floor_share * remaining:
                best = r
        first = (1 if evict else 0) + best
    slots = [(kind, t) for kind in ("key", "value") for t in range(middle)]
    base = sum(sizes[kind][first] for kind, _ in slots)
    items = []
    for i, (kind, t) in enumerate(slots):
        run = float("inf")
        e, s = errs[kind][t], sizes[kind]
        for l in range(first, len(s) - 1):
            run = min(run, max(e[l] - e[l + 1], 0.0) / (s[l + 1] - s[l]))
            items.append((-run, i * (len(s) - 1 - first) + (l - first), i, s[l + 1] - s[l]))
    items.sort(key=lambda x: (x[0], x[1]))
    counts, spent = [0] * len(slots), 0
    for _, _, i, cost in items:
        if spent + cost > remaining - base:
            break
        spent += cost
        counts[i] += 1
    chosen = np.array(counts) + first - (1 if evict else 0)
    key, value = chosen[:middle].copy(), chosen[middle:].copy()
    value[key < 0] = -1
    return key, value, first, remaining


def _bytes(choice, rung_bytes, exact_bytes):
    total = 0
    for kind in ("key", "value"):
        sizes = list(rung_bytes[kind]) + [exact_bytes]
        total += sum(sizes[r] for r in choice[kind] if r >= 0)
    return total


CASES = [
    dict(budget=0.25),
    dict(budget=0.25, weights="snap"),
    dict(budget=0.3, key_weight=3.0),
    dict(budget=0.2, evict=True),
    dict(budget=0.15, evict=True),
    dict(budget=0.3, floor_share=1.0),
    dict(budget=0.3, floor_share=0.5, evict=True, weights="snap", key_weight=2.0),
]


@pytest.mark.parametrize("case", CASES, ids=[",".join(f"{k}={v}" for k, v in c.items()) for c in CASES])
def test_compress_choice_equals_plain_statement(case):
    m, mu, b, rungs, rb, eb = _setup(11)
    kw = dict(case)
    if kw.get("weights") == "snap":
        kw["weights"] = np.random.default_rng(12).uniform(0.05, 2.0, m["key"].shape[0]).astype(np.float32)
    got = kvtc_ref.compress_choice(m, mu, b, rungs, rb, eb, sinks=2, exact_recent=3, **kw)
    key, value, first, remaining = _plain(m, mu, b, rungs, rb, eb, 2, 3, **kw)
    assert got["first"] == first and got["remaining"] == remaining
    assert np.array_equal(got["key"], key) and np.array_equal(got["value"], value)
    assert _bytes(got, rb, eb) <= got["remaining"]
    assert (got["key"] >= first - (1 if kw.get("evict") else 0)).all()


def test_floor_is_the_finest_affordable_uniform_rung():
    m, mu, b, rungs, rb, eb = _setup(13)
    got = kvtc_ref.compress_choice(m, mu, b, rungs, rb, eb, sinks=2, exact_recent=3, budget=0.3, floor_share=1.0)
    middle = got["span"][1] - got["span"][0]
    sizes = [k + v for k, v in zip(rb["key"] + [eb], rb["value"] + [eb])]
    affordable = [r for r, s in enumerate(sizes) if middle * s <= got["remaining"]]
    assert got["first"] == max(affordable)
    assert (got["key"] >= got["first"]).all() and (got["value"] >= got["first"]).all()
    # with eviction available the floor still keeps every token
    ev = kvtc_ref.compress_choice(m, mu, b, rungs, rb, eb, sinks=2, exact_recent=3, budget=0.3, floor_share=1.0,
                                  evict=True)
    assert (ev["key"] >= 0).all() and ev["first"] == 1 + max(affordable)


def test_key_rescaling_leaves_choice_unchanged_only_with_energy_normalisation():
    m, mu, b, rungs, rb, eb = _setup(14)
    scaled = dict(m)
    scaled["key"] = (mu["key"] + np.float32(8.0) * (m["key"] - mu["key"])).astype(np.float32)
    base = kvtc_ref.compress_choice(m, mu, b, rungs, rb, eb, sinks=2, exact_recent=3, budget=0.25)
    again = kvtc_ref.compress_choice(scaled, mu, b, rungs, rb, eb, sinks=2, exact_recent=3, budget=0.25)
    assert np.array_equal(base["key"], again["key"]) and np.array_equal(base["value"], again["value"])
    # the same rule without the energy normalisation moves upgrades between keys and values
    k0, v0, _, _ = _plain(m, mu, b, rungs, rb, eb, 2, 3, 0.25, normalise=False)
    k1, v1, _, _ = _plain(scaled, mu, b, rungs, rb, eb, 2, 3, 0.25, normalise=False)
    assert not (np.array_equal(k0, k1) and np.array_equal(v0, v1))


def test_zero_importance_tokens_stay_at_the_floor():
    m, mu, b, rungs, rb, eb = _setup(15)
    w = np.ones(40, np.float32)
    w[[5, 6, 9]] = 0.0
    got = kvtc_ref.compress_choice(m, mu, b, rungs, rb, eb, sinks=2, exact_recent=3, budget=0.2, weights=w,
                                   floor_share=0.5)
    start = got["span"][0]
    for t in (5, 6, 9):
        assert got["key"][t - start] == got["first"] and got["value"][t - start] == got["first"]
    assert (got["key"] > got["first"]).any()  # the budget did buy upgrades for the others


def test_eviction_keys_take_values_and_cost_nothing():
    m, mu, b, rungs, rb, eb = _setup(16)
    got = kvtc_ref.compress_choice(m, mu, b, rungs, rb, eb, sinks=2, exact_recent=3, budget=0.15, evict=True)
    assert (got["key"] < 0).any(), "a tight budget should evict some keys"
    assert (got["value"][got["key"] < 0] == -1).all()
    assert _bytes(got, rb, eb) <= got["remaining"]


def test_span_and_budget_split_known_answers():
    m, mu, b, rungs, rb, eb = _setup(17, tokens=14)
    got = kvtc_ref.compress_choice(m, mu, b, rungs, rb, eb, sinks=4, exact_recent=6, budget=1.0)
    assert got["span"] == (4, 8)
    assert got["budget_bytes"] == int(1.0 * 14 * 2 * eb)
    assert got["remaining"] == got["budget_bytes"] - 10 * 2 * eb
    short = {k: v[:3] for k, v in m.items()}
    none = kvtc_ref.compress_choice(short, mu, b, rungs, rb, eb, sinks=4, exact_recent=6, budget=2.0)
    assert none["span"] == (3, 3) and none["key"].size == 0
