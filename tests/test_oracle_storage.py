"""Pins of the byte-storage oracle (oracle/storage_ref.py, scripts/kvtc_storage.py): hand-written
bytes for a small cache, hand-computed and numpy-computed code packings, the reference's own
round-trip check (the restored cache equals the in-memory compressed one) and the closed-form size.
A plausible slip (MSB-first codes, widths or rungs out of order, shifts and scales swapped,
exact rows stored after the exact tokens) changes the hand-written bytes."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import kvtc_ref
from oracle import storage_ref as st


def _bits_lsb_first(codes, width):
    return np.array([(int(c) >> i) & 1 for c in codes for i in range(width)], np.uint8)


def test_pack_codes_known_answers():
    assert st.pack_codes([1, 2, 3, 0, 3], 2) == bytes([0x39, 0x03])
    assert st.pack_codes([0xA, 0x5, 0xF], 4) == bytes([0x5A, 0x0F])
    assert st.pack_codes([7, 200, 0], 8) == bytes([7, 200, 0])
    assert st.packed_length(5, 2) == 2 and st.packed_length(3, 4) == 2 and st.packed_length(3, 8) == 3
    rng = np.random.default_rng(0)
    for width in (2, 4, 8):
        codes = rng.integers(0, 2**width, size=203)
        packed = st.pack_codes(codes, width)
        # numpy's little-endian bit packing of the LSB-first bit stream
        assert packed == np.packbits(_bits_lsb_first(codes, width), bitorder="little").tobytes()
        assert np.array_equal(st.unpack_codes(packed, width, codes.size), codes.astype(np.uint8))


def _hand_cache():
    bits = np.array([[2, 0], [4, 2]])  # two rungs over two groups of 4; rung 2 is the exact rung
    keys = {"rungs": np.array([1, 0, 2]), "bits": bits,
            "coefficients": np.array([[0, 1, 2, 15, 10, 11, 12, 13], [-1, 0, 1, 2, 5, 5, 5, 5], [0] * 8], np.float32),
            "matrix_rows": np.array([[9] * 8, [9] * 8, [0.5, -0.5, 1, -1, 2, -2, 0.25, 4]], np.float32),
            "exact_tokens": np.array([[1] * 8, [-2] * 8], np.float32), "features": 8}
    values = {"rungs": np.array([0, 0, 0]), "bits": bits,
              "coefficients": np.array([[0, 3, 3, 0, 9, 9, 9, 9], [4, 5, 6, 7, 1, 1, 1, 1],
                                        [0, 0.5, 1, 1.5, 2, 2, 2, 2]], np.float32),
              "matrix_rows": np.zeros((3, 8), np.float32),
              "exact_tokens": np.array([[0] * 8, [0.5] * 8], np.float32), "features": 8}
    return keys, values


def test_encode_hand_written_bytes():
    keys, values = _hand_cache()
    data = st.encode(5, 1, 4, [keys, values], group=4)
    one, minus_two, half = "003c", "00c0", "0038"
    want = "".join([
        "05000000" "01000000" "04000000",                     # tokens, start, end
        # keys: rung ids
        "010002",
        "e4" "00bc" "003c",                                   # rung 0: width 2 (t1 group 0): codes, shift -1, scale 1
        "e4" "0049" "003c",                                   # rung 1: width 2 (t0 group 1): shift 10, scale 1
        "10f2" "0000" "003c",                                 #         width 4 (t0 group 0): codes 0,1,2,15
        "0038" "00b8" "003c" "00bc" "0040" "00c0" "0034" "0044",  # rung 2 (exact): fp16 matrix row of t2
        one * 8 + minus_two * 8,                              # exact tokens (sink, recent)
        # values: rung ids, then rung 0 for t0, t1, t2 (codes, shifts, scales)
        "000000",
        "3c" "e4" "e4" "0000" "0044" "0000" "003c" "003c" "0038",
        "0000" * 8 + half * 8,
    ])
    assert data.hex() == want
    assert len(data) == st.stored_bytes(5, 3, [keys, values], group=4) == 129


def test_decode_inverts_encode_on_the_hand_cache():
    keys, values = _hand_cache()
    data = st.encode(5, 1, 4, [keys, values], group=4)
    metas = [{"bits": keys["bits"], "rank": 8, "features": 8}] * 2
    out = st.decode(data, metas, group=4)
    assert out["header"] == (5, 1, 4)
    k, v = out["streams"]
    assert np.array_equal(k["rungs"], [1, 0, 2]) and np.array_equal(v["rungs"], [0, 0, 0])
    assert np.array_equal(k["coefficients"][0], [0, 1, 2, 15, 10, 11, 12, 13])
    assert np.array_equal(k["coefficients"][1], [-1, 0, 1, 2, 0, 0, 0, 0])  # group 1 dropped at rung 0
    assert np.array_equal(k["coefficients"][2], np.zeros(8))                # exact rung: rows kept aside
    assert np.array_equal(k["exact_rows"][0], [2])
    assert np.array_equal(k["exact_rows"][1].astype(np.float32), keys["matrix_rows"][2:3])
    assert np.array_equal(v["exact_tokens"].astype(np.float32), values["exact_tokens"])
    with pytest.raises(ValueError, match="Decoded 129 of 130 bytes"):
        st.decode(data + b"\0", metas, group=4)


@pytest.mark.parametrize("seed", [0, 1])
def test_round_trip_equals_quantize_groups(seed):
    """The reference's check (FINDINGS.md:468-469): restoring gives back exactly what compress kept."""
    rng = np.random.default_rng(seed)
    group, groups, features, tokens, start, end = 64, 6, 96, 40, 4, 30
    rank = group * groups
    bits = rng.choice([0, 2, 4, 8], size=(4, groups))
    bits[0] = 0
    bits[0, 0] = 2
    middle = end - start
    streams, metas = [], []
    for _ in range(2):
        s = {"rungs": rng.integers(0, bits.shape[0] + 1, size=middle), "bits": bits,
             "coefficients": rng.normal(size=(middle, rank)).astype(np.float32) * 3,
             "matrix_rows": rng.normal(size=(middle, features)).astype(np.float32),
             "exact_tokens": rng.normal(size=(tokens - middle, features)).astype(np.float32), "features": features}
        streams.append(s)
        metas.append({"bits": bits, "rank": rank, "features": features})
    data = st.encode(tokens, start, end, streams, group)
    assert len(data) == st.stored_bytes(tokens, middle, streams, group)
    out = st.decode(data, metas, group)
    for s, o in zip(streams, out["streams"]):
        assert np.array_equal(o["rungs"], s["rungs"])
        for t in range(middle):
            r = s["rungs"][t]
            if r == bits.shape[0]:
                assert np.array_equal(o["coefficients"][t], np.zeros(rank))
                continue
            want = kvtc_ref.quantize_groups(s["coefficients"][t:t + 1], bits[r], group)[0]
            assert np.array_equal(o["coefficients"][t], want), (t, r)
        idx, rows = o["exact_rows"]
        assert np.array_equal(idx, np.nonzero(s["rungs"] == bits.shape[0])[0])
        assert np.array_equal(rows, s["matrix_rows"][idx].astype(np.float16))
        assert np.array_equal(o["exact_tokens"], s["exact_tokens"].astype(np.float16))


def test_evicted_tokens_raise():
    keys, values = _hand_cache()
    keys = dict(keys, rungs=np.array([1, -1, 2]))
    with pytest.raises(NotImplementedError, match="evicted tokens"):
        st.encode(5, 1, 4, [keys, values], group=4)
