"""Pins of oracle/progressive_ref.py (CPU): quantize8 / dequantize against exact rational
arithmetic rounded once per operation, the nesting of bit-plane codes, byte accounting
against hand-written formulas, and the error table against a float64 brute force."""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import progressive_ref as pr

F32_MAX = Fraction(float(np.finfo(np.float32).max))


def f32_round(x: Fraction) -> np.float32:
    """Round an exact rational to the nearest float32 (ties to even) without double rounding."""
    guess = np.float32(float(x))
    cands = {guess, np.nextafter(guess, np.float32(-np.inf)), np.nextafter(guess, np.float32(np.inf))}
    best = None
    for c in sorted(cands, key=float):
        if not np.isfinite(c):
            continue
        d = abs(Fraction(float(c)) - x)
        even = (np.array(c, dtype=np.float32).view(np.uint32) & 1) == 0
        if best is None or d < best[0] or (d == best[0] and even):
            best = (d, c)
    return best[1]


def fp16_samples(seed: int, count: int) -> list[tuple[np.float16, np.float16]]:
    rng = np.random.default_rng(seed)
    low = rng.normal(0, 2, count).astype(np.float16)
    span = np.abs(rng.normal(0, 2, count)).astype(np.float16)
    # edge values: tiny / subnormal spans, large spans, negative and positive lows
    extra_low = np.array([0.0, -0.0, 1e-4, -65504.0, 3.0, -1e-7], dtype=np.float16)
    extra_span = np.array([6e-8, 1e-5, 65504.0, 1.0, 0.0009765625, 2.0], dtype=np.float16)
    return list(zip(np.concatenate([low, extra_low]), np.concatenate([span, extra_span])))


def test_dequantize_matches_rational_rounding_exhaustive():
    """Every index at every plane count m = 0..8 for sampled fp16 (low, span): the oracle equals
    low + ((idx + 0.5) * span) / 2^m with each operation rounded to float32 on its own."""
    pairs = fp16_samples(11, 40)
    for low, span in pairs:
        codes = np.arange(256, dtype=np.uint8).reshape(4, 1, 64)
        lo = np.full((4, 1), low, dtype=np.float16)
        sp = np.full((4, 1), span, dtype=np.float16)
        for m in range(9):
            got = pr.dequantize(codes, lo, sp, np.full((1, 1), m)).reshape(-1)
            for code in range(0, 256, 1 << (8 - m) if m else 256):
                if m == 0:
                    assert got[code] == 0.0
                    continue
                idx = code >> (8 - m)
                prod = f32_round((Fraction(idx) + Fraction(1, 2)) * Fraction(float(span)))
                quot = f32_round(Fraction(float(prod)) / (1 << m))
                want = f32_round(Fraction(float(low)) + Fraction(float(quot)))
                assert got[code] == want, (float(low), float(span), m, code)
            # all codes with the same top m bits decode identically (nesting)
            if m:
                blocks = got.reshape(1 << m, -1)
                assert (blocks == blocks[:, :1]).all()


def test_quantize8_matches_rational_rounding():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((6, 128)) * np.array([3.0, 0.01, 1e3, 1.0, 1e-3, 50.0])[:, None]).astype(np.float32)
    codes, low, span = pr.quantize8(x, 64)
    for t in range(6):
        for g in range(2):
            part = x[t, g * 64:(g + 1) * 64]
            lo = np.float16(part.min())
            assert low[t, g] == lo
            rng_f32 = f32_round(Fraction(float(part.max())) - Fraction(float(np.float32(lo))))
            sp = np.float16(max(rng_f32, np.float32(1e-8)))
            assert span[t, g] == sp
            for j in range(64):
                diff = f32_round(Fraction(float(part[j])) - Fraction(float(np.float32(lo))))
                q = f32_round(Fraction(float(diff)) / Fraction(float(np.float32(sp))))
                scaled = f32_round(Fraction(float(q)) * 256)
                want = min(255, max(0, int(np.floor(float(scaled)))))
                assert codes[t, g, j] == want


def test_quantize8_nesting_and_error_bound():
    """Top m bits of the 8-bit code are the m-bit code, and |x - dequant_m(x)| <= span / 2^(m+1)
    (plus fp16 rounding of low and span and float32 rounding)."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((32, 256)).astype(np.float32)
    codes, low, span = pr.quantize8(x, 64)
    grouped = x.reshape(32, 4, 64)
    scaled = (grouped - low.astype(np.float32)[..., None]) / span.astype(np.float32)[..., None]
    for m in range(1, 9):
        top = codes >> (8 - m)
        assert np.array_equal(top, np.clip(np.floor(scaled * np.float32(2 ** m)), 0, 2 ** m - 1).astype(np.uint8))
        deq = pr.dequantize(codes, low, span, np.full((1, 4), m)).reshape(32, 4, 64)
        # inside [low, low + span] the bin half-width bounds the error; values clamped into the
        # first or last bin (fp16 rounding of low and span) add that rounding
        slack = (np.abs(grouped.max(-1) - (low.astype(np.float32) + span.astype(np.float32)))
                 + np.abs(grouped.min(-1) - low.astype(np.float32)))[..., None]
        bound = span.astype(np.float32)[..., None] / 2 ** (m + 1) + slack + 1e-5 * np.abs(grouped) + 1e-6
        assert (np.abs(grouped - deq) <= bound).all(), m


def test_quantize8_degenerate_group_defined_as_zero():
    """A constant group whose fp16 span rounds to 0 gives 0/0 for members equal to low; the
    reference's NaN -> uint8 cast is undefined, the build defines code 0 (parity unpinned for
    this case).  Members above low give +inf -> clamped to 255, as in the reference."""
    x = np.zeros((1, 64), dtype=np.float32)
    x[0, 1] = 1e-9
    codes, low, span = pr.quantize8(x, 64)
    assert span[0, 0] == 0 and low[0, 0] == 0
    assert codes[0, 0, 0] == 0 and codes[0, 0, 1] == 255 and (codes[0, 0, 2:] == 0).all()


def test_plane_major_order_bytes_closed_form():
    for groups in (1, 3, 16, 32):
        order = pr.plane_major_order(groups)
        assert order.planes.shape == (8 * groups + 1, groups)
        for k in range(8 * groups + 1):
            m = order.planes[k]
            assert (m == k // groups + (np.arange(groups) < k % groups)).all()
            # 8 B per piece plus a 4 B header for every group that has at least one plane
            assert order.prefix_bytes[k] == 8 * k + 4 * int((m > 0).sum())
        assert order.prefix_bytes[-1] == groups * (4 + 64)
        assert order.rungs == [groups * m for m in range(1, 9)]


def test_order_from_sequence_rejects_ninth_plane():
    with pytest.raises(ValueError):
        pr.order_from_sequence([0] * 9, 1)


def test_hot_cold_fetched_bytes_closed_form():
    groups = 4
    order = pr.plane_major_order(groups)
    rng = np.random.default_rng(1)
    pieces = {kind: rng.integers(0, 8 * groups + 1, 50) for kind in ("key", "value")}
    orders = {"key": order, "value": order}
    exact_tokens, exact_bytes = 36, 1000
    full = groups * 68
    seg = lambda k: 8 * k + 4 * min(k, groups)  # noqa: E731  plane-major: first G pieces carry a header
    want_hot = exact_tokens * 2 * exact_bytes + sum(seg(int(k)) + 1 for kind in pieces for k in pieces[kind])
    assert pr.hot_bytes(orders, pieces, exact_tokens, exact_bytes) == want_hot
    want_cold = sum(full - seg(int(k)) for kind in pieces for k in pieces[kind])
    assert pr.cold_bytes(orders, pieces) == want_cold
    rows = np.array([0, 7, 49])
    want_fetch = sum(full - seg(int(pieces[kind][r])) for kind in pieces for r in rows)
    assert pr.fetched_bytes(orders, pieces, rows) == want_fetch


def test_error_table_brute_force():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 128)).astype(np.float32)
    codes, low, span = pr.quantize8(x, 64)
    table = pr.error_table(x, codes, low, span)
    assert table.shape == (8, 2, 9)
    for t in range(8):
        for g in range(2):
            part = x[t, g * 64:(g + 1) * 64].astype(np.float64)
            assert table[t, g, 0] == pytest.approx(float((part ** 2).sum()), rel=1e-5)
            for m in range(1, 9):
                idx = codes[t, g].astype(np.int64) >> (8 - m)
                dq = float(low[t, g]) + (idx + 0.5) * float(span[t, g]) / 2 ** m
                assert table[t, g, m] == pytest.approx(float(((part - dq) ** 2).sum()), rel=1e-3, abs=1e-9)
            # more planes never increase the error by more than rounding
            assert (np.diff(table[t, g, 1:]) <= 1e-6 + 1e-3 * table[t, g, 1:-1]).all()
