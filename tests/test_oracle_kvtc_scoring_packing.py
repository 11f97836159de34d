"""Pins of oracle/kvtc_ref.py, oracle/scoring_ref.py and oracle/packing_ref.py (CPU).

Allocator: an explicit Python restatement of the greedy rule (per-slot
upgrade values made monotone with a running minimum, one global order by value
with ties in slot-major index order, the longest affordable prefix) on tiny
inputs, brute force over every per-slot prefix set for the optimality it implies
on concave inputs, the budget/prefix invariants, and the shipped torch
allocator (torch's stable sort).  kvtc quantizer: the closed-form grid and the
shipped torch quantizer bit for bit.  Scoring: brute-force float64 softmax over
all keys, Python rounding of the selection count, torch.topk on distinct
scores.  Packing: pack/unpack round trip, the byte sizes of both tiers against
the reference's counts, and the GPU lane formula that rebuilds four codes with
one AND-OR per plane and a rotate.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from oracle import kvtc_ref, packing_ref, scoring_ref
from oracle import progressive_ref as pr


def greedy_reference(errors, level_bytes, middle, budget):
    """Plain-Python statement of the allocation rule (scripts/kvtc.py:277-298)."""
    slots, levels = errors.shape
    sizes = [list(map(float, level_bytes[:levels]))] * middle + [list(map(float, level_bytes[levels:]))] * middle
    base = sum(s[0] for s in sizes)
    if base > budget:
        raise ValueError
    items = []
    for i in range(slots):
        run = float("inf")
        for l in range(levels - 1):
            gain = max(float(np.float32(errors[i, l]) - np.float32(errors[i, l + 1])), 0.0)
            cost = sizes[i][l + 1] - sizes[i][l]
            run = min(run, gain / cost)
            items.append((-run, i * (levels - 1) + l, i, cost))
    items.sort(key=lambda x: (x[0], x[1]))
    counts, spent = [0] * slots, 0.0
    for _, _, i, cost in items:
        if spent + cost > budget - base:
            break
        spent += cost
        counts[i] += 1
    return np.array(counts)


def test_allocate_rungs_matches_plain_statement_and_torch():
    import kvtc

    rng = np.random.default_rng(0)
    for trial in range(40):
        middle, levels = int(rng.integers(1, 6)), int(rng.integers(2, 6))
        errors = np.sort(rng.random((2 * middle, levels)).astype(np.float32), axis=1)[:, ::-1].copy()
        if trial % 3 == 0:  # ties and non-monotone gains
            errors = np.round(errors * 4) / 4
            errors[:, 1] += 0.1
        level_bytes = np.concatenate([np.cumsum(rng.integers(1, 9, levels)), np.cumsum(rng.integers(1, 9, levels))])
        base = middle * (level_bytes[0] + level_bytes[levels])
        budget = int(base + rng.integers(0, 6 * middle * 8 + 1))
        want = greedy_reference(errors, level_bytes, middle, budget)
        got = kvtc_ref.allocate_rungs(errors, level_bytes, middle, budget)
        assert np.array_equal(got, want), trial
        shipped = kvtc.allocate_rungs(torch.from_numpy(errors), torch.from_numpy(level_bytes), middle, budget)
        assert np.array_equal(shipped.numpy(), want), trial
        # invariants: within budget, never beyond the top level
        sizes = np.repeat(level_bytes.reshape(2, levels), middle, axis=0)
        spent = sizes[np.arange(2 * middle), got].sum()
        assert spent <= budget and (got <= levels - 1).all()


def test_allocate_rungs_raises_below_coarsest():
    with pytest.raises(ValueError):
        kvtc_ref.allocate_rungs(np.ones((2, 3), np.float32), np.array([5, 6, 7, 5, 6, 7]), 1, 9)


def test_allocate_rungs_optimal_on_concave_unit_costs():
    """With unit step costs and decreasing gains the greedy prefix is the exact optimum:
    checked against brute force over every per-slot level choice."""
    rng = np.random.default_rng(2)
    for _ in range(20):
        middle, levels = 2, 4
        gains = np.sort(rng.random((2 * middle, levels - 1)), axis=1)[:, ::-1]
        errors = np.concatenate([gains.sum(1, keepdims=True), gains.sum(1, keepdims=True) - np.cumsum(gains, 1)], 1)
        errors = errors.astype(np.float32)
        level_bytes = np.array([1, 2, 3, 4, 1, 2, 3, 4])
        budget = int(4 + rng.integers(0, 13))
        got = kvtc_ref.allocate_rungs(errors, level_bytes, middle, budget)
        best = min(sum(errors[i, c[i]] for i in range(4))
                   for c in itertools.product(range(levels), repeat=4) if sum(c) + 4 <= budget)
        assert sum(errors[i, got[i]] for i in range(4)) == pytest.approx(best, rel=1e-6, abs=1e-6)


def test_quantize_groups_grid_and_shipped_torch():
    import kvtc

    rng = np.random.default_rng(1)
    x = (rng.standard_normal((16, 256)) * rng.uniform(0.01, 5, (16, 1))).astype(np.float32)
    bits = np.array([8, 4, 2, 0])
    q = kvtc_ref.quantize_groups(x, bits, 64)
    shipped = kvtc.quantize_groups(torch.from_numpy(x), torch.from_numpy(bits), 64).numpy()
    assert np.array_equal(q.view(np.uint32), shipped.view(np.uint32))
    g = x.reshape(16, 4, 64)
    qg = q.reshape(16, 4, 64)
    assert (qg[:, 3] == 0).all()
    for j, b in enumerate(bits[:3]):
        low = g[:, j].min(-1).astype(np.float16).astype(np.float32)
        scale = np.maximum((g[:, j].max(-1) - low) / np.float32(2 ** int(b) - 1), np.float32(1e-8))
        scale = scale.astype(np.float16).astype(np.float32)
        k = (qg[:, j] - low[:, None]) / scale[:, None]
        assert np.allclose(k, np.round(k), atol=1e-3) and (k > -1e-3).all() and (k < 2 ** int(b) - 1 + 1e-3).all()
        inside = (g[:, j] >= low[:, None]) & (g[:, j] <= (low + scale * (2 ** int(b) - 1))[:, None])
        err = np.abs(g[:, j] - qg[:, j])
        assert (err[inside] <= (scale[:, None] / 2 + 1e-5 * np.abs(g[:, j]) + 1e-6)[inside]).all()
    # rint rounds half to even: low 0, max 3 -> scale 1; 0.5 -> 0, 1.5 -> 2, 2.5 -> 2
    half = np.array([[0.0, 3.0, 0.5, 1.5, 2.5] + [0.0] * 59], dtype=np.float32)
    hq = kvtc_ref.quantize_groups(half, np.array([2]), 64)
    assert hq[0, :5].tolist() == [0.0, 3.0, 0.0, 2.0, 2.0]


def test_rung_bytes_closed_form():
    assert kvtc_ref.rung_bytes(np.array([8, 4, 2, 0]), 64) == 64 + 32 + 16 + 3 * 4


def test_layer_probabilities_brute_force():
    rng = np.random.default_rng(3)
    Hq, Hkv, ql, d, n, E = 6, 2, 3, 8, 11, 4
    q = rng.standard_normal((Hq, ql, d)).astype(np.float32)
    kc = rng.standard_normal((Hkv, n, d)).astype(np.float32)
    ke = rng.standard_normal((Hkv, E, d)).astype(np.float32)
    kq = rng.standard_normal((Hkv, ql, d)).astype(np.float32)
    got = scoring_ref.layer_probabilities(q, kc, ke, kq, 0.35)
    want = np.zeros((Hkv, n))
    for h in range(Hq):
        kv = h // 3
        for i in range(ql):
            keys = np.concatenate([kc[kv], ke[kv], kq[kv, : i + 1]]).astype(np.float64)
            s = keys @ q[h, i].astype(np.float64) * 0.35
            p = np.exp(s - s.max())
            p /= p.sum()
            want[kv] += p[:n]
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-7)


def test_select_count_python_rounding():
    assert scoring_ref.select_count(0.01, 16348) == 163
    assert scoring_ref.select_count(0.01, 16350) == 164  # 163.5 rounds half to even -> 164
    assert scoring_ref.select_count(0.01, 16250) == 162  # 162.5 -> 162
    assert scoring_ref.select_count(0.001, 10) == 1


def test_topk_indices_match_torch_topk_on_distinct_values():
    rng = np.random.default_rng(4)
    for n, k in ((100, 7), (5000, 50), (17, 17)):
        s = rng.permutation(n).astype(np.float32) + rng.random(n).astype(np.float32) * 0.1
        want = np.sort(torch.topk(torch.from_numpy(s), k).indices.numpy())
        assert np.array_equal(scoring_ref.topk_indices(s, k), want)
        assert scoring_ref.topk_margin(s, k) > 0
    ties = np.array([3, 1, 3, 2, 3], dtype=np.float32)
    assert scoring_ref.topk_indices(ties, 2).tolist() == [0, 2]  # ties: lower index first


def test_plane_words_round_trip_and_gpu_lane_formula():
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 256, 64).astype(np.uint8)
    for p in range(8):
        pos = packing_ref.bit_position(np.arange(64), p)
        assert sorted(pos.tolist()) == list(range(64))  # a bijection per plane
        w = int(packing_ref.plane_word(codes, p))
        assert np.array_equal(packing_ref.word_codes(w, p), (codes >> (7 - p)) & 1)
    # device rule: rotr(OR_p plane[p] & (0x01010101 << ((w + 7 - p) & 7)), w) = codes 4w..4w+3 of a half
    for m in range(9):
        words = [int(packing_ref.plane_word(codes, p)) if p < m else 0 for p in range(8)]
        trunc = codes & np.uint8((0xFF << (8 - m)) & 0xFF)
        for half in range(2):
            pl = [(w >> (32 * half)) & 0xFFFFFFFF for w in words]
            for w in range(8):
                acc = 0
                for p in range(8):
                    acc |= pl[p] & ((0x01010101 << ((w + 7 - p) & 7)) & 0xFFFFFFFF)
                rot = ((acc >> w) | (acc << (32 - w))) & 0xFFFFFFFF if w else acc
                got = [(rot >> (8 * i)) & 0xFF for i in range(4)]
                assert got == trunc[32 * half + 4 * w: 32 * half + 4 * w + 4].tolist(), (m, half, w)


def test_pack_unpack_and_tier_sizes():
    rng = np.random.default_rng(6)
    groups, tokens = 3, 40
    order = pr.order_from_sequence([0, 1, 0, 2, 1, 0, 2, 2, 1, 0, 0, 1, 2, 0, 1, 2, 0, 1, 2, 0, 1, 2, 1, 2], groups)
    codes = rng.integers(0, 256, (tokens, groups, 64)).astype(np.uint8)
    low = rng.standard_normal((tokens, groups)).astype(np.float16)
    span = np.abs(rng.standard_normal((tokens, groups))).astype(np.float16)
    pieces = rng.integers(0, order.pieces + 1, tokens)
    hot, hot_off, cold, cold_off = packing_ref.pack(codes, low, span, pieces, order)
    assert np.array_equal(np.diff(hot_off), order.prefix_bytes[pieces])
    assert np.array_equal(np.diff(cold_off), order.prefix_bytes[-1] - order.prefix_bytes[pieces])
    c, lo, sp, planes = packing_ref.unpack(hot, hot_off[:-1], pieces, order, groups)
    m = planes.astype(np.int64)
    mask = ((0xFF << (8 - m)) & 0xFF).astype(np.uint8)[..., None]
    assert np.array_equal(c, codes & mask)
    present = m > 0
    assert np.array_equal(lo[present].view(np.uint16), low[present].view(np.uint16))
    assert np.array_equal(sp[present].view(np.uint16), span[present].view(np.uint16))
    # segment offset tables agree with the packed layout
    seg = packing_ref.segment_offsets(order)
    for t in range(tokens):
        k = pieces[t]
        sizes = np.where(order.planes[k] > 0, 4 + 8 * order.planes[k].astype(int), 0)
        assert np.array_equal(seg[k], np.concatenate([[0], np.cumsum(sizes)[:-1]]))


def test_ladder_code_bytes_known_answers_and_packbits():
    """LSB-first code packing (scripts/kvtc_storage.py:21-27 bit order) on hand-computed bytes and
    against numpy.packbits(bitorder="little") of each code's bits."""
    assert packing_ref.pack_ladder_codes(np.tile([0, 1, 2, 3], 16), 2) == bytes([0xE4]) * 16
    assert packing_ref.pack_ladder_codes(np.tile([1, 2], 32), 4) == bytes([0x21]) * 32
    assert packing_ref.pack_ladder_codes(np.arange(64), 8) == bytes(range(64))
    rng = np.random.default_rng(11)
    for width in (2, 4, 8):
        codes = rng.integers(0, 2**width, 64)
        bits = ((codes[:, None] >> np.arange(width)) & 1).astype(np.uint8).reshape(-1)
        want = np.packbits(bits, bitorder="little").tobytes()
        assert packing_ref.pack_ladder_codes(codes, width) == want


def test_quantize_groups_codes_dequantize_and_shipped_torch():
    """quantize_groups == dequantize_codes(quantize_groups_codes) bit for bit, and the shipped
    torch codes (kvtc.quantize_groups_codes) equal the oracle's."""
    import kvtc

    rng = np.random.default_rng(12)
    x = (rng.standard_normal((50, 4 * 64)) * np.array([3.0, 0.5, 1e-3, 7.0]).repeat(64)).astype(np.float32)
    bits = np.array([8, 0, 2, 4])
    codes, low, scale = kvtc_ref.quantize_groups_codes(x, bits, 64)
    assert codes[:, 0].max() <= 255 and codes[:, 2].max() <= 3 and codes[:, 3].max() <= 15
    assert not codes[:, 1].any()
    deq = kvtc_ref.dequantize_codes(codes, low, scale, bits)
    assert np.array_equal(deq.view(np.uint32), kvtc_ref.quantize_groups(x, bits, 64).view(np.uint32))
    c, lo, sc = kvtc.quantize_groups_codes(torch.from_numpy(x), torch.from_numpy(bits), 64)
    assert np.array_equal(c.numpy(), codes)
    assert np.array_equal(lo.numpy().view(np.uint16), low.view(np.uint16))
    assert np.array_equal(sc.numpy().view(np.uint16), scale.view(np.uint16))


def test_pack_ladder_sizes_and_offsets():
    rng = np.random.default_rng(13)
    bits = np.array([[2, 0, 0, 0], [4, 2, 0, 2], [8, 4, 2, 0], [8, 8, 8, 8]])
    n = 30
    codes = rng.integers(0, 256, (n, 4, 64)).astype(np.uint8)
    low = rng.standard_normal((n, 4)).astype(np.float16)
    scale = np.abs(rng.standard_normal((n, 4))).astype(np.float16)
    rung = rng.integers(0, 4, n)
    masked = codes & ((1 << bits[rung]) - 1).astype(np.uint8)[..., None]
    blob, off = packing_ref.pack_ladder(masked, low, scale, rung, bits)
    assert np.array_equal(np.diff(off), [kvtc_ref.rung_bytes(bits[r], 64) for r in rung])
    seg = packing_ref.ladder_segment_offsets(bits)
    for t in range(n):
        for g in np.nonzero(bits[rung[t]])[0]:
            s = off[t] + seg[rung[t], g]
            assert blob[s:s + 2].view(np.float16)[0] == low[t, g]
            width = bits[rung[t], g]
            body = blob[s + 4:s + 4 + 8 * width].tobytes()
            assert body == packing_ref.pack_ladder_codes(masked[t, g], width)


@pytest.mark.parametrize("order_kind", ["irregular", "plane_major"])
def test_pack_fast_equals_pack(order_kind):
    """The vectorised packer (used at full size) gives the loop packer's four results byte for byte,
    including tokens with no hot piece and tokens with every piece."""
    rng = np.random.default_rng(61)
    groups, tokens = 3, 50
    if order_kind == "irregular":
        order = pr.order_from_sequence([0, 1, 0, 2, 1, 0, 2, 2, 1, 0, 0, 1, 2, 0, 1, 2, 0, 1, 2, 0], groups)
    else:
        order = pr.plane_major_order(groups)
    codes = rng.integers(0, 256, (tokens, groups, 64)).astype(np.uint8)
    low = rng.standard_normal((tokens, groups)).astype(np.float16)
    span = np.abs(rng.standard_normal((tokens, groups))).astype(np.float16)
    pieces = rng.integers(0, order.pieces + 1, tokens)
    pieces[:2] = (0, order.pieces)
    for a, b in zip(packing_ref.pack(codes, low, span, pieces, order),
                    packing_ref.pack_fast(codes, low, span, pieces, order)):
        assert a.dtype == b.dtype and np.array_equal(a, b)


def test_rung_errors_equal_decode_at_each_rung():
    """A rung's error from the table lookup (progressive.py:159-160) equals the squared error of the
    token decoded at that rung's plane map, summed over groups, over the mean energy; weights scale
    each token by w / mean(w)."""
    rng = np.random.default_rng(62)
    tokens, groups = 30, 4
    x = (rng.standard_normal((tokens, groups * 64)) * np.repeat(rng.uniform(0.01, 2, groups), 64)).astype(np.float32)
    order = pr.order_from_sequence([0, 1, 2, 3, 0, 0, 1, 2, 3, 3, 1, 2, 0, 1, 2, 3] * 2, groups,
                                   rungs=[0, 3, 7, 16, 32])
    codes, low, span = pr.quantize8(x, 64)
    table = pr.error_table(x, codes, low, span)
    got = pr.rung_errors(x, table, order)
    energy = np.float64(np.square(x.astype(np.float64)).sum(axis=1).mean())
    for j, k in enumerate(order.rungs):
        deq = pr.dequantize(codes, low, span, order.planes[k][None].repeat(tokens, 0)).astype(np.float64)
        want = np.square(x - deq).sum(axis=1) / energy
        np.testing.assert_allclose(got[:, j], want, rtol=1e-5, atol=1e-9)
    w = rng.uniform(0.1, 3.0, tokens).astype(np.float32)
    np.testing.assert_allclose(pr.rung_errors(x, table, order, w), got * (w / w.mean())[:, None], rtol=1e-5)
    assert pr.level_bytes(order) == [int(order.prefix_bytes[k]) + 1 for k in order.rungs]
