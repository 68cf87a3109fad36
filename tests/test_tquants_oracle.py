"""Pin the oracle's TQ1_0 / TQ2_0 restatement (oracle/tquants_oracle.c) to the reference's
tests/fixtures/upstream-tquants.json records: packed bytes, decoded values, the generic
Q8_K dot's bits and the quantizer output (src/kernels/tquants.rs:17-324; the reference's
own test is tests/tquants.rs), plus the digit closed forms on every byte."""

import math

import numpy as np
import pytest

import fixtures_util as fx

CASES = fx.load_json("upstream-tquants.json")["Cases"]


def _ids(case):
    return f"{case['TypeId']}-{case['Name']}"


def test_fixture_holds_both_kinds():
    assert len(CASES) == 10
    assert {c["TypeId"] for c in CASES} == {34, 35}
    assert all(c["Count"] % 256 == 0 for c in CASES)


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_tq_decode_matches_reference_records(case):
    import oracle

    kind, count = case["TypeId"], case["Count"]
    packed = bytes.fromhex(case["OutputHex"])
    assert len(packed) == count // 256 * (54 if kind == 34 else 66)
    got = oracle.decode_row(kind, count, packed)
    assert got.astype("<f4").tobytes() == bytes.fromhex(case["DecodedHex"])


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_tq_generic_dot_matches_reference_bits(case):
    import oracle

    kind, count = case["TypeId"], case["Count"]
    packed = bytes.fromhex(case["OutputHex"])
    act = bytes.fromhex(case["ActivationsHex"])
    got = oracle.packed_dot(kind, count, packed, act)
    assert np.float32(got).tobytes() == bytes.fromhex(case["GenericDotHex"])
    # The per-row entry over prepared Q8_K blocks gives the same bits.
    q = np.frombuffer(act, oracle.Q8K_DTYPE)
    assert np.float32(oracle.dot_tq(kind, packed, q)).tobytes() == bytes.fromhex(case["GenericDotHex"])


@pytest.mark.parametrize("case", [c for c in CASES if isinstance(c.get("InputHex"), str)], ids=_ids)
def test_tq_quantizer_matches_reference_bytes(case):
    import oracle

    x = np.frombuffer(bytes.fromhex(case["InputHex"]), "<f4")
    assert oracle.quantize_row(case["TypeId"], x) == bytes.fromhex(case["OutputHex"])


def test_tq1_digits_invert_the_canonical_encoding():
    """Every 5-digit base-3 code q (digit 0 most significant) packed as ceil(q*256/243)
    decodes to its own digits, minus one, at elements col + 32k."""
    import oracle

    for q in range(243):
        blk = np.zeros(54, np.uint8)
        blk[0] = math.ceil(q * 256 / 243)
        codes = oracle.tq_codes(34, blk)
        digits = [(q // 3 ** (4 - k)) % 3 for k in range(5)]
        assert [int(codes[32 * k]) for k in range(5)] == [d - 1 for d in digits], q


def test_tq2_fields_decode_every_byte():
    import oracle

    for b in range(256):
        blk = np.zeros(66, np.uint8)
        blk[32 + 5] = b  # second half, column 5
        codes = oracle.tq_codes(35, blk)
        assert [int(codes[128 + 5 + 32 * k]) for k in range(4)] == [((b >> (2 * k)) & 3) - 1 for k in range(4)]
        assert np.count_nonzero(codes + 1) == np.count_nonzero(np.array([((b >> (2 * k)) & 3) for k in range(4)]))
