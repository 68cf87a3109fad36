"""Pin the oracle's activation and row quantizers to the reference's native captures.

Mirrors tests/row_quantizers.rs, src/kernels.rs:5157-5291 and
src/kernels/pinned_q8_tests.rs.
"""

import numpy as np
import pytest

import fixtures_util as fx


def _q8_wire(block) -> bytes:
    """Q8_0 34-byte wire form of a prepared block: f16(scale) + codes."""
    from oracle import float_to_half

    return float_to_half(float(block["scale"])).to_bytes(2, "little") + block["values"].tobytes()


def _q8_1_wire(block) -> bytes:
    from oracle import float_to_half

    return (float_to_half(float(block["scale"])).to_bytes(2, "little")
            + float_to_half(float(block["sum"])).to_bytes(2, "little") + block["values"].tobytes())


def test_row_quantizers_match_native_production_bytes(oracle):
    data = fx.load_json("row-quantizers-path.json")
    seen = set()
    for case in data["Cases"]:
        kind = case["TypeId"]
        x = np.frombuffer(fx.hexbytes(case["InputHex"]), dtype="<f4")
        expected = fx.hexbytes(case["OutputHex"])
        if kind == 1:  # F16: binary16 RNE of every value (pins float_to_half)
            got = b"".join(oracle.float_to_half(float(v)).to_bytes(2, "little") for v in x)
        else:
            got = oracle.quantize_row(kind, x)
        assert got == expected, (kind, case["Name"])
        seen.add(kind)
    assert seen == {1, 8, 15, 142, 143}
    assert len(data["Cases"]) == 20


def test_pinned_q8_preparation_matches_native_rounding_capture(oracle):
    # src/kernels.rs:5157-5231: six captured 70-byte records (Q8_0 then Q8_1).
    blob = fx.read("swift-q8-parity.bin")
    meta = fx.load_json("swift-q8-parity.json")
    assert fx.sha256(blob) == meta["fixture_sha256"]
    assert len(meta["cases"]) == 6
    for idx, case in enumerate(meta["cases"]):
        x = fx.f32_from_hex_words(case["input_bits"])
        assert x.size == 32
        for columns in (128, 32):
        # PTQ1 pinned uses the native-scale contract; Q4_1 pinned uses the generic pinned
        # contract; both reproduce these captures.
            xs = np.tile(x, columns // 32)
            for contract in (oracle.Q8_PINNED_NATIVE, oracle.Q8_PINNED):
                for blk in oracle.quantize_q8_0(xs, contract):
                    assert _q8_wire(blk) == blob[idx * 70: idx * 70 + 34]
                    assert _q8_1_wire(blk) == blob[idx * 70 + 34: (idx + 1) * 70]
        if idx == 1:
            # Source contract keeps roundf's ties away from zero.
            src = oracle.quantize_q8_0(np.tile(x, 4), oracle.Q8_SOURCE)
            assert list(src[0]["values"][2:8]) == [1, -1, 2, -2, 3, -3]
        bad = np.tile(x, 4).copy()
        bad[17] = np.nan
        with pytest.raises(oracle.OracleError):
            oracle.quantize_q8_0(bad, oracle.Q8_PINNED_NATIVE)


def test_pinned_q8k_preparation_matches_native_half_boundary_capture(oracle):
    # src/kernels.rs:5233-5291
    blob = fx.read("swift-q8k-parity.bin")
    meta = fx.load_json("swift-q8k-parity.json")
    assert fx.sha256(blob) == meta["fixture_sha256"]
    for case, (word, native_code, source_code) in enumerate([(0xBE010F7E, 71, 72), (0x3E010F7E, -71, -72)]):
        x = np.zeros(256, np.float32)
        x[0] = np.uint32(0x3E653D88).view(np.float32)
        x[1] = np.uint32(word).view(np.float32)
        pinned = oracle.quantize_q8k(x, pinned=True)
        assert pinned[0]["values"][1] == native_code
        assert pinned.tobytes() == blob[case * 292: (case + 1) * 292]
        source = oracle.quantize_q8k(x, pinned=False)
        assert source[0]["values"][1] == source_code
        x[17] = np.nan
        with pytest.raises(oracle.OracleError):
            oracle.quantize_q8k(x, pinned=True)


def test_pinned_ptq1_scale_and_inverse_match_native_halfway_controls(oracle):
    # src/kernels/pinned_q8_tests.rs:45-80 and :90-132
    blob = fx.read("swift-ptq1-q8-scale-parity.bin")
    meta = fx.load_json("swift-ptq1-q8-scale-parity.json")
    assert fx.sha256(blob) == "cda434b51d60bbdcd417492a4af77f3ef6cb5eef6390826abb6609b8a3578dee"
    assert len(meta["cases"]) == 4
    for i, case in enumerate(meta["cases"]):
        x = np.array(case["input_bits"], dtype=np.uint32).view(np.float32)
        blk = oracle.quantize_q8_0(x, oracle.Q8_PINNED_NATIVE)
        assert _q8_wire(blk[0]) == blob[34 * i: 34 * (i + 1)], case["name"]
    codes = np.frombuffer(blob, dtype=np.int8)
    assert codes[3] == -52 and codes[34 + 3] == -77
    x0 = np.tile(np.array(meta["cases"][0]["input_bits"], dtype=np.uint32).view(np.float32), 4)
    assert oracle.quantize_q8_0(x0, oracle.Q8_PINNED_NATIVE)[0]["values"][1] == -52
    assert oracle.quantize_q8_0(x0, oracle.Q8_PINNED)[0]["values"][1] == -51
    assert oracle.quantize_q8_0(x0, oracle.Q8_SOURCE)[0]["values"][1] == -51


def test_q8k_first_strict_maximum_keeps_sign_and_bsums(oracle):
    # src/kernels.rs:484-492 (first element with strictly greatest |x| wins).
    x = np.zeros(256, np.float32)
    x[5] = -3.0
    x[9] = 3.0
    q = oracle.quantize_q8k(x, pinned=False)[0]
    # iscale = -127/max with max = -3 (the first strict maximum): x[5] -> -127, x[9] -> +127.
    assert q["values"][5] == -127 and q["values"][9] == 127
    assert q["scale"] == np.float32(1.0) / (np.float32(-127.0) / np.float32(-3.0))
    rng = np.random.default_rng(3)
    y = rng.standard_normal(1024).astype(np.float32)
    for pinned in (False, True):
        qq = oracle.quantize_q8k(y, pinned)
        sums = qq["values"].reshape(-1, 16, 16).astype(np.int32).sum(-1)
        assert np.array_equal(sums, qq["sums"])
    assert oracle.quantize_q8k(np.zeros(256, np.float32), False)[0]["scale"] == 0.0


def test_quantizers_reject_partial_nonfinite_and_overflow(oracle):
    with pytest.raises(oracle.OracleError):
        oracle.quantize_q8k(np.ones(255, np.float32), False)
    for kind in (8, 15, 142, 143):
        with pytest.raises(oracle.OracleError):
            oracle.quantize_row(kind, np.full(256, np.nan, np.float32))
        with pytest.raises(oracle.OracleError):
            oracle.quantize_row(kind, np.ones(127, np.float32))
    for kind in (8, 142, 143):
        with pytest.raises(oracle.OracleError):
            oracle.quantize_row(kind, np.full(256, np.finfo(np.float32).max, np.float32))
    # Q8_K inverse-scale overflow on a tiny subnormal maximum.
    tiny = np.zeros(256, np.float32)
    tiny[0] = np.uint32(1).view(np.float32)
    with pytest.raises(oracle.OracleError):
        oracle.quantize_q8k(tiny, False)


def test_q8_source_rounds_half_away_and_pinned_ties_even(oracle):
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:7] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5]
    src = oracle.quantize_q8_0(x, oracle.Q8_SOURCE)[0]["values"]
    pin = oracle.quantize_q8_0(x, oracle.Q8_PINNED)[0]["values"]
    assert list(src[1:7]) == [1, -1, 2, -2, 3, -3]
    assert list(pin[1:7]) == [0, 0, 2, -2, 2, -2]
