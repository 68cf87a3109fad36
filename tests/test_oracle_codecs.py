"""Pin the oracle's codecs (binary16, PTQ1 trits, PQ2<->PTQ1) to the reference's golden data.

Mirrors tools/ternary/tests/cpp_reference.rs, tests/upstream_prism/ptq1.rs and
tests/packed_codec.rs.
"""

import numpy as np
import pytest

import fixtures_util as fx


def test_cpp_reference_half_to_float_cases(oracle):
    halves, _ = fx.ptq_reference()
    assert len(halves) == 26
    for h, bits in halves:
        assert oracle.half_to_float_bits(h) == bits, hex(h)


def test_half_to_float_exhaustive_roundtrip_and_numpy(oracle):
    # Every finite half converts exactly (numpy's float16->float32 is exact) and rounds back to itself.
    hs = np.arange(65536, dtype=np.uint16)
    ref = hs.view(np.float16).astype(np.float32)
    got = np.array([oracle.half_to_float(int(h)) for h in hs], dtype=np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    back = np.array([oracle.float_to_half(float(v)) for v in got[finite]], dtype=np.uint16)
    assert np.array_equal(back, hs[finite])


def test_float_to_half_matches_ieee_rne(oracle):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[np.isfinite(vals)]
    # Concentrate on the binary16 range too (normals, subnormals, overflow boundary).
    extra = (rng.standard_normal(200_000) * np.exp2(rng.uniform(-26, 17, 200_000))).astype(np.float32)
    edges = np.array([65504, 65519.99, 65520, -65520, 2**-24, 2**-25, 3 * 2**-26, 2**-14, 0.0, -0.0], np.float32)
    vals = np.concatenate([vals, extra, edges])
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.float_to_half(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)
    # NaN -> canonical quiet NaN with the sign kept (tools/ternary/src/lib.rs:104-110).
    assert oracle.float_to_half(float("nan")) & 0x7FFF == 0x7E00


def test_cpp_reference_ptq_parity(oracle):
    _, cases = fx.ptq_reference()
    assert len(cases) == 161
    assert sum(c[0] for c in cases) == 169
    for idx, (rows, blocks, pq2, ptq) in enumerate(cases):
        assert blocks in (2, 40, 48, 136)
        for a, b in zip(pq2, ptq):
            assert oracle.pack_ptq(a) == b, idx
            assert oracle.unpack_ptq(b) == a, idx


def _lcg_blocks(trials=20_000):
    # tests/upstream_prism/ptq1.rs:10-26
    seed = 12345
    out = np.zeros((trials, 28), np.uint8)
    for t in range(trials):
        for i in range(26):
            seed = (seed * 1103515245 + 12345) & 0xFFFFFFFF
            out[t, i] = (seed >> 16) & 0xFF
        out[t, 26:] = (0x00, 0x3C)
    return out


def _cpu_stage_reference(block):
    # Upstream cpu_ref stage traversal (tests/upstream_prism/ptq1.rs:30-50), written independently.
    powers = [1, 3, 9, 27, 81]
    out = []
    j = 0
    for width in (32, 16, 8):
        while j + width <= 24:
            for p in powers:
                for m in range(width):
                    q = (int(block[j + m]) * p) & 0xFF
                    out.append(((q * 3) >> 8) - 1)
            j += width
    for p in powers[:4]:
        for h in range(2):
            q = (int(block[24 + h]) * p) & 0xFF
            out.append(((q * 3) >> 8) - 1)
    return out


def test_upstream_ptq1_element_map_20000_lcg_blocks(oracle):
    blocks = _lcg_blocks()
    assert list(blocks[0, :8]) == [220, 4, 101, 170, 31, 173, 29, 90]
    # Vectorised closed form of both upstream traversals, then the oracle decoder on every block.
    for t in range(blocks.shape[0]):
        trits = oracle.decode_ptq_trits(blocks[t])
        if t < 400:
            assert list(trits) == _cpu_stage_reference(blocks[t])
        vals = oracle.decode_row(oracle.KIND_PTQ1, 128, blocks[t])
        assert np.array_equal(vals, trits.astype(np.float32))


def test_every_ptq_byte_decodes_to_fractional_trits(oracle):
    # tests/packed_codec.rs: every byte is a valid runtime trit source; digits follow frac*3.
    for x in range(256):
        blk = np.full(28, x, np.uint8)
        blk[26:] = (0, 0x3C)
        t = oracle.decode_ptq_trits(blk)
        frac = x
        digits = []
        for _ in range(5):
            frac *= 3
            digits.append((frac >> 8) - 1)
            frac &= 255
        assert list(t[:80:16]) == digits  # byte 0 carries elements 0,16,32,48,64
        assert list(t[120:128:2]) == digits[:4]  # byte 24 carries 120,122,124,126


def test_pack_rejects_reserved_symbol_and_bad_scales(oracle):
    good = fx.pq2_block(0x3C00, [(3, 2)])
    oracle.pack_ptq(good)
    bad = bytearray(good)
    bad[2] = 0xFF
    with pytest.raises(oracle.OracleError):
        oracle.pack_ptq(bytes(bad))
    for s in (0x0000, 0x8000, 0x7C00, 0xFC01):
        b = bytearray(good)
        b[0:2] = s.to_bytes(2, "little")
        with pytest.raises(oracle.OracleError):
            oracle.pack_ptq(bytes(b))
