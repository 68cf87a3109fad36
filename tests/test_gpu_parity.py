"""GPU parity: every HIP path through the C ABI against the oracle, bit-exact.

The reference's native captures (PQ2 fused/unfused KAT, PTQ1 pinned/source dot
bits, Q2_K generic dots, the closed-form matvec KATs) are replayed through the
GPU; random shapes and the benchmark configurations are compared with the CPU
oracle on identical seeded inputs.  Tolerance: 0 ULP for every integer-dot /
binary32-chain output; the source-order SwiGLU (device libm exp) is compared
with max |diff| <= 1e-3 * max |ref|.
"""

import os

import numpy as np
import pytest

import fixtures_util as fx
import prism_hip as ph
import synth
from hiprt import DeviceBuffer

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)


@pytest.fixture(scope="module")
def ctx():
    c = ph.Context(0)
    yield c
    c.close()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bits_equal(got, ref, what=""):
    g, r = bits(got), bits(ref)
    if not np.array_equal(g, r):
        idx = np.nonzero(g != r)[0]
        i = idx[0]
        raise AssertionError(f"{what}: {idx.size} mismatches, first at {i}: gpu={np.float32(got.flat[i])!r} "
                             f"oracle={np.float32(ref.flat[i])!r}")


# ---- native captures through the GPU -------------------------------------------------

def test_gpu_pinned_pq2_accumulation_matches_native_capture(ctx):
    w = bytearray([0xAA] * 68)
    w[0:2] = (0x3C01).to_bytes(2, "little")
    w[34:36] = (0x3787).to_bytes(2, "little")
    act = np.zeros(1, ph.Q8K_DTYPE)
    act["scale"] = np.uint32(0x3DA00001).view(np.float32)
    act["values"][0, :128] = 3
    act["values"][0, 128:] = -13
    act["sums"][0, :8] = 48
    act["sums"][0, 8:] = -208
    wid = ctx.weight(ph.KIND_PQ2, 256, 1, bytes(w))
    assert int(bits(ctx.project_q8k(wid, 1, act, fused=True))[0]) == 0xC1F90B01
    assert int(bits(ctx.project_q8k(wid, 1, act, fused=False))[0]) == 0xC1F90B02
    ctx.release(wid)


def test_gpu_ptq1_dot_matches_native_pinned_and_source_bits(ctx):
    blob = fx.read("swift-ptq1-dot-parity.bin")
    meta = fx.load_json("swift-ptq1-dot-parity.json")
    cur = 0
    for case in range(2):
        width = int.from_bytes(blob[cur:cur + 4], "little")
        expected = int.from_bytes(blob[cur + 4:cur + 8], "little")
        wb = width // 128 * 28
        weights = blob[cur + 8:cur + 8 + wb]
        acts = blob[cur + 8 + wb:cur + 8 + wb + width // 32 * 34]
        cur += 8 + wb + width // 32 * 34
        q8 = np.zeros(width // 32, ph.Q8_DTYPE)
        for i in range(width // 32):
            q8[i]["scale"] = np.uint16(int.from_bytes(acts[34 * i:34 * i + 2], "little")).view(np.float16)
            q8[i]["values"] = np.frombuffer(acts[34 * i + 2:34 * i + 34], np.int8)
        wid = ctx.weight(ph.KIND_PTQ1, width, 1, weights)
        assert int(bits(ctx.project_q8(wid, 1, q8, pinned=True))[0]) == expected
        assert int(bits(ctx.project_q8(wid, 1, q8, pinned=False))[0]) == meta["fixtures"][case]["source_bits"]
        ctx.release(wid)


def test_gpu_q2k_generic_dot_matches_native_records(ctx):
    for case in fx.load_json("upstream-kquants-q2k.json")["Cases"]:
        count = case["Count"]
        w = fx.hexbytes(case["OutputHex"])
        act = np.frombuffer(fx.hexbytes(case["ActivationsHex"]), ph.Q8K_DTYPE).copy()
        wid = ctx.weight(ph.KIND_Q2_K, count, 1, w)
        got = ctx.project_q8k(wid, 1, act)
        assert got.tobytes() == fx.hexbytes(case["GenericDotHex"]), case["Name"]
        ctx.release(wid)


def test_gpu_closed_form_matvec_kats(ctx):
    import oracle

    cases = []
    first = fx.pq2_block(0x3C00, [(1, 2), (2, 2), (3, 2)])
    second = fx.pq2_block(0x3800, [(0, 0)])
    x = np.zeros(256, np.float32)
    x[[0, 1, 2, 3, 128, 255]] = [127.0, 0.5, 1.5, 2.5, -1.5, -127.0]
    cases.append((ph.KIND_PQ2, 256, first + second, x, 5.0))
    w = fx.pq2_block(0x3C00, [(0, 3)]) + fx.pq2_block(0, [(0, 3)])
    x = np.zeros(256, np.float32)
    x[0] = -127.0
    cases.append((ph.KIND_PQ2, 256, w, x, -254.0))
    cases.append((ph.KIND_PQ2, 256, w, np.zeros(256, np.float32), 0.0))
    blk = oracle.pack_ptq(fx.pq2_block(0x4000, [(1, 2), (2, 2), (33, 2)]))
    x = np.zeros(128, np.float32)
    x[[0, 1, 2, 32, 33]] = [127.0, 0.5, 1.5, 63.5, 0.25]
    cases.append((ph.KIND_PTQ1, 128, blk, x, 7.0))
    blk = oracle.pack_ptq(fx.pq2_block(0x3C00, [(0, 2)]))
    x = np.zeros(128, np.float32)
    x[0] = 1.0
    cases.append((ph.KIND_PTQ1, 128, blk, x, np.float32(0.99993896)))
    f1 = fx.pq2_block(0x4000, [(1, 2), (2, 3), (33, 2)])
    x = np.zeros(128, np.float32)
    x[[0, 1, 2, 32, 33]] = [127.0, 0.5, 1.5, 63.5, 0.25]
    cases.append((ph.KIND_PQ2, 128, f1, x, 11.0))
    f2 = fx.pq2_block(0x3800, [(1, 2), (2, 3), (33, 2)])
    f3 = fx.pq2_block(0x3C00, [(1, 2), (2, 3), (33, 2)])
    cases.append((ph.KIND_PQ2, 384, f1 + f2 + f3, np.concatenate([x, x, x]), 19.25))
    for kind, cols, w, x, expected in cases:
        wid = ctx.weight(kind, cols, 1, w)
        got = ctx.project_f32(wid, 1, x)
        assert got[0] == np.float32(expected), (kind, cols, got[0], expected)
        ctx.release(wid)


# ---- quantizers ------------------------------------------------------------------------

def _quant_inputs():
    rng = np.random.default_rng(21)
    xs = [rng.standard_normal(4096).astype(np.float32),
          (rng.standard_normal(2048) * np.exp2(rng.integers(-30, 30, 2048))).astype(np.float32),
          np.zeros(512, np.float32)]
    ties = np.zeros(256, np.float32)
    ties[5], ties[9], ties[100] = -3.0, 3.0, 1.5
    xs.append(ties)
    for case in fx.load_json("swift-q8-parity.json")["cases"]:
        xs.append(np.tile(fx.f32_from_hex_words(case["input_bits"]), 8))
    for word in (0xBE010F7E, 0x3E010F7E):
        x = np.zeros(256, np.float32)
        x[0] = np.uint32(0x3E653D88).view(np.float32)
        x[1] = np.uint32(word).view(np.float32)
        xs.append(x)
    for case in fx.load_json("swift-ptq1-q8-scale-parity.json")["cases"]:
        xs.append(np.tile(np.array(case["input_bits"], np.uint32).view(np.float32), 8))
    for case in fx.load_json("row-quantizers-path.json")["Cases"]:
        if case["TypeId"] in (8, 15):
            xs.append(np.frombuffer(fx.hexbytes(case["InputHex"]), "<f4").copy())
    return xs


def test_gpu_quantizers_match_oracle_bytes(ctx):
    import oracle

    def expect(quant, args, dev_out, what):
        # Same bytes when the reference quantizer succeeds, an error when it rejects the
        # input (e.g. a binary16 scale overflow for |x| > 65504*127).
        try:
            ref = quant(*args)
        except oracle.OracleError:
            assert ctx.sync() == ph.ERR_NONFINITE, what
            return
        assert ctx.sync() == 0, what
        assert dev_out.to_numpy(np.uint8).tobytes() == ref.tobytes(), what

    for i, x in enumerate(_quant_inputs()):
        n = x.size - x.size % 256
        if n:
            xd = DeviceBuffer.from_numpy(x[:n])
            for pinned in (False, True):
                out = DeviceBuffer(n // 256 * 292)
                ctx.quantize_q8k_device(xd, n, 1, pinned, out)
                expect(oracle.quantize_q8k, (x[:n], pinned), out, ("q8k", i, pinned))
        n = x.size - x.size % 32
        xd = DeviceBuffer.from_numpy(x[:n])
        for contract in (0, 1, 2):
            out = DeviceBuffer(n // 32 * 40)
            ctx.quantize_q8_device(xd, n, 1, contract, out)
            expect(oracle.quantize_q8_0, (x[:n], contract), out, ("q8_0", i, contract))


def test_gpu_quantizer_rejects_nonfinite_and_overflow(ctx):
    x = np.ones(256, np.float32)
    x[17] = np.nan
    out = DeviceBuffer(292)
    ctx.quantize_q8k_device(DeviceBuffer.from_numpy(x), 256, 1, False, out)
    assert ctx.sync() == ph.ERR_NONFINITE
    tiny = np.zeros(256, np.float32)
    tiny[0] = np.uint32(1).view(np.float32)
    ctx.quantize_q8k_device(DeviceBuffer.from_numpy(tiny), 256, 1, False, out)
    assert ctx.sync() == ph.ERR_NONFINITE
    assert ctx.sync() == 0  # flag cleared


# ---- random shapes, every kind and contract -------------------------------------------

SHAPES = [
    (ph.KIND_PTQ1, 37, 256), (ph.KIND_PTQ1, 64, 2048), (ph.KIND_PTQ1, 50, 384), (ph.KIND_PTQ1, 33, 6144),
    (ph.KIND_PTQ1, 9, 8192), (ph.KIND_PTQ1, 21, 16384),
    (ph.KIND_PQ2, 37, 256), (ph.KIND_PQ2, 64, 2048), (ph.KIND_PQ2, 40, 384), (ph.KIND_PQ2, 33, 6144),
    (ph.KIND_PQ2, 19, 12288), (ph.KIND_PQ2, 17, 128),
    (ph.KIND_Q2_K, 37, 256), (ph.KIND_Q2_K, 64, 2048), (ph.KIND_Q2_K, 33, 6144), (ph.KIND_Q2_K, 21, 16384),
    (ph.KIND_Q8_0, 37, 128), (ph.KIND_Q8_0, 64, 2048), (ph.KIND_Q8_0, 50, 2080), (ph.KIND_Q8_0, 33, 4096),
    (ph.KIND_Q8_0, 9, 8192),
    (ph.KIND_TQ1_0, 37, 256), (ph.KIND_TQ1_0, 64, 2048), (ph.KIND_TQ1_0, 33, 6144), (ph.KIND_TQ1_0, 21, 16384),
    (ph.KIND_TQ2_0, 37, 256), (ph.KIND_TQ2_0, 64, 2048), (ph.KIND_TQ2_0, 33, 6144), (ph.KIND_TQ2_0, 19, 12288),
]


@pytest.mark.parametrize("kind,rows,cols", SHAPES)
def test_gpu_project_f32_matches_oracle_matvec(ctx, kind, rows, cols):
    import oracle

    w = synth.weights(kind, rows, cols, seed=rows * 7 + cols) if kind != ph.KIND_PQ2 else \
        synth.pq2_weights(rows, cols, seed=rows + cols, levels=4)
    x = synth.activations(cols, seed=cols + 1)
    wid = ctx.weight(kind, cols, rows, w)
    for pinned in (False, True):
        ref = oracle.matvec(kind, cols, rows, w, x, pinned, threads=THREADS)
        got = ctx.project_f32(wid, rows, x, pinned=pinned)
        assert_bits_equal(got, ref, f"kind={kind} {rows}x{cols} pinned={pinned}")
    ctx.release(wid)


@pytest.mark.parametrize("kind,rows,cols", [s for s in SHAPES if s[0] != ph.KIND_Q8_0 and s[2] % 256 == 0])
def test_gpu_project_q8k_prepared_codes(ctx, kind, rows, cols):
    import oracle

    w = synth.weights(kind, rows, cols, seed=11 + rows)
    x = synth.activations(cols, seed=cols + 2)
    wid = ctx.weight(kind, cols, rows, w)
    for pinned in (False, True):
        act = oracle.quantize_q8k(x, pinned)
        if kind == ph.KIND_PTQ1:
            ref = np.array([oracle.dot_ptq1_q8k(w[r * (cols // 128) * 28:(r + 1) * (cols // 128) * 28], act)
                            for r in range(rows)], np.float32)
        else:
            ref = oracle.project_q8k(kind, cols, rows, w, act, pinned, threads=THREADS)
        got = ctx.project_q8k(wid, rows, act.view(ph.Q8K_DTYPE), fused=pinned)
        assert_bits_equal(got, ref, f"q8k kind={kind} pinned={pinned}")
    ctx.release(wid)


@pytest.mark.parametrize("kind,rows,cols", [(ph.KIND_PTQ1, 37, 2048), (ph.KIND_PQ2, 40, 384),
                                            (ph.KIND_PQ2, 40, 2048), (ph.KIND_Q8_0, 37, 2048)])
def test_gpu_project_q8_prepared_codes(ctx, kind, rows, cols):
    import oracle

    w = synth.weights(kind, rows, cols, seed=5 + rows)
    x = synth.activations(cols, seed=cols + 3)
    wid = ctx.weight(kind, cols, rows, w)
    for contract in (0, 1, 2):
        act = oracle.quantize_q8_0(x, contract)
        for pinned in (False, True):
            ref = oracle.project_q8(kind, cols, rows, w, act, pinned, threads=THREADS)
            got = ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), pinned=pinned)
            assert_bits_equal(got, ref, f"q8 kind={kind} contract={contract} pinned={pinned}")
    ctx.release(wid)


# ---- large matrices: one wavefront per 64-row tile (>= one tile per CU) ----------------

@pytest.mark.parametrize("kind,cols", [(ph.KIND_PTQ1, 256), (ph.KIND_PTQ1, 8448), (ph.KIND_PQ2, 256), (ph.KIND_PQ2, 384),
                                       (ph.KIND_Q2_K, 256), (ph.KIND_Q8_0, 256), (ph.KIND_TQ1_0, 512),
                                       (ph.KIND_TQ2_0, 512), (ph.KIND_Q2_K, 1280), (ph.KIND_Q8_0, 640),
                                       (ph.KIND_PQ2, 1152), (ph.KIND_TQ1_0, 1280), (ph.KIND_TQ2_0, 1280)])
def test_gpu_row_tile_path_matches_oracle(ctx, kind, cols):
    """rows spans more 64-row tiles than the device has CUs (the one-wavefront-per-tile
    kernel with scalar activation loads), with a partial last tile.  From four units per
    row the tile's units are split over two wavefronts (odd unit counts here: the second
    half's terms come back through LDS and must continue the chain in unit order)."""
    import oracle

    import hiprt

    rows = 64 * hiprt.cu_count(0) + 37
    w = synth.weights(kind, rows, cols, seed=17) if kind != ph.KIND_PQ2 else synth.pq2_weights(rows, cols, 17, 4)
    x = synth.activations(cols, seed=18)
    wid = ctx.weight(kind, cols, rows, w)
    for pinned in (False, True):
        ref = oracle.matvec(kind, cols, rows, w, x, pinned, threads=THREADS)
        assert_bits_equal(ctx.project_f32(wid, rows, x, pinned=pinned), ref, f"rows kind={kind} pinned={pinned}")
    if kind in (ph.KIND_PTQ1, ph.KIND_Q8_0) or (kind == ph.KIND_PQ2 and cols % 256):
        act = oracle.quantize_q8_0(x, 1)
        ref = oracle.project_q8(kind, cols, rows, w, act, True, threads=THREADS)
        assert_bits_equal(ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), pinned=True), ref, "rows q8")
    ctx.release(wid)


@pytest.mark.parametrize("per_cu", [5, 9, 16])
@pytest.mark.parametrize("cols", [128, 384, 1024])
def test_gpu_ptq1_table_decode_matches_oracle(ctx, cols, per_cu):
    """PTQ1 on the row-tile path decodes trits through the LDS table, one workgroup per
    CU working through its tiles: 5-6 tiles per workgroup (each tile's units split over
    two wavefronts), 9-10 (eight whole tiles per workgroup, the rest as split pairs;
    single-term orders) or 16-17 (whole tiles, some wavefronts taking two); one unit (an
    empty second half), an odd and an even unit count, a partial last tile, and all
    three activation contracts."""
    import oracle

    import hiprt

    kind = ph.KIND_PTQ1
    cus = hiprt.cu_count(0)
    rows = 64 * (per_cu * cus + 3) + 37
    w = synth.weights(kind, rows, cols, seed=29 + cols)
    x = synth.activations(cols, seed=30)
    wid = ctx.weight(kind, cols, rows, w)
    for pinned in (False, True):
        ref = oracle.matvec(kind, cols, rows, w, x, pinned, threads=THREADS)
        assert_bits_equal(ctx.project_f32(wid, rows, x, pinned=pinned), ref, f"table f32 pinned={pinned}")
    for contract in (0, 2):
        act = oracle.quantize_q8_0(x, contract)
        for pinned in (False, True):
            ref = oracle.project_q8(kind, cols, rows, w, act, pinned, threads=THREADS)
            got = ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), pinned=pinned)
            assert_bits_equal(got, ref, f"table q8 contract={contract} pinned={pinned}")
    if cols % 256 == 0:
        act = oracle.quantize_q8k(x, False)
        nb = cols // 128 * 28
        ref = np.array([oracle.dot_ptq1_q8k(w[r * nb:(r + 1) * nb], act) for r in range(0, rows, 997)], np.float32)
        got = ctx.project_q8k(wid, rows, act.view(ph.Q8K_DTYPE))
        assert_bits_equal(got[::997], ref, "table q8k")
    ctx.release(wid)


@pytest.mark.parametrize("per_cu4", [3, 6, 14])
@pytest.mark.parametrize("cols", [384, 4096, 5120, 8064])
def test_gpu_ptq1_table_spread_matches_oracle(ctx, cols, per_cu4):
    """From half a tile to eight tiles per CU, prepared-activation PTQ1 rows of up to 64
    units run table workgroups of one, two or four tiles (per_cu4 / 4 tiles per CU here),
    each tile's units spread over 16, 8 or 4 wavefronts and their terms folded in unit order
    from LDS (pinned PTQ1 only where its nine terms per unit fit; beyond, its earlier
    forms): bit-exact in every contract (source, pinned, native-scale pinned Q8_0, and
    Q8_K), with odd unit counts (3, 63) and a partial last tile."""
    import oracle

    import hiprt

    kind = ph.KIND_PTQ1
    cus = hiprt.cu_count(0)
    rows = 64 * (per_cu4 * cus // 4) + 37
    w = synth.weights(kind, rows, cols, seed=71 + cols + per_cu4)
    x = synth.activations(cols, seed=72)
    wid = ctx.weight(kind, cols, rows, w)
    for contract, pinned in ((0, False), (1, True), (2, True), (1, False)):
        act = oracle.quantize_q8_0(x, contract)
        ref = oracle.project_q8(kind, cols, rows, w, act, pinned, threads=THREADS)
        got = ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), pinned=pinned)
        assert_bits_equal(got, ref, f"spread q8 contract={contract} pinned={pinned}")
    if cols % 256 == 0:
        act = oracle.quantize_q8k(x, False)
        nb = cols // 128 * 28
        sample = list(range(0, rows, 97)) + list(range(rows - 20, rows))
        ref = np.array([oracle.dot_ptq1_q8k(w[r * nb:(r + 1) * nb], act) for r in sample], np.float32)
        got = ctx.project_q8k(wid, rows, act.view(ph.Q8K_DTYPE))
        assert_bits_equal(got[sample], ref, "spread q8k")
    ctx.release(wid)


@pytest.mark.parametrize("per_cu4", [3, 6, 15])
@pytest.mark.parametrize("kind,cols", [(ph.KIND_Q8_0, 2048), (ph.KIND_Q8_0, 4224), (ph.KIND_PQ2, 2048),
                                       (ph.KIND_PQ2, 4224), (ph.KIND_Q2_K, 2048), (ph.KIND_Q2_K, 4352),
                                       (ph.KIND_TQ1_0, 2304), (ph.KIND_TQ1_0, 4096), (ph.KIND_TQ2_0, 2048),
                                       (ph.KIND_TQ2_0, 4352)])
def test_gpu_rows_n_wavefronts_matches_oracle(ctx, kind, cols, per_cu4):
    """Between half a tile and four tiles per CU (per_cu4 / 4 here), prepared activations
    of the non-PTQ1 formats run 16 wavefronts per tile below one tile per CU and 8 from one
    (8 with 8 to 15 units per row), each walking a contiguous unit range whose terms
    wavefront 0 folds from LDS in unit order: bit-exact in every contract, with even and
    odd unit counts and a partial last tile."""
    import oracle

    import hiprt

    cus = hiprt.cu_count(0)
    rows = 64 * (per_cu4 * cus // 4) + 37
    w = synth.weights(kind, rows, cols, seed=81 + cols) if kind != ph.KIND_PQ2 else \
        synth.pq2_weights(rows, cols, 81 + cols, 4)
    x = synth.activations(cols, seed=82)
    wid = ctx.weight(kind, cols, rows, w)
    if kind in (ph.KIND_Q8_0, ph.KIND_PQ2):
        for contract, pinned in ((1, False), (0, True)):
            act = oracle.quantize_q8_0(x, contract)
            ref = oracle.project_q8(kind, cols, rows, w, act, pinned, threads=THREADS)
            got = ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), pinned=pinned)
            assert_bits_equal(got, ref, f"rows-n q8 kind={kind} contract={contract} pinned={pinned}")
    if cols % 256 == 0 and kind != ph.KIND_Q8_0:
        for fused in (False, True):
            act = oracle.quantize_q8k(x, fused)
            ref = oracle.project_q8k(kind, cols, rows, w, act, fused, threads=THREADS)
            got = ctx.project_q8k(wid, rows, act.view(ph.Q8K_DTYPE), fused=fused)
            assert_bits_equal(got, ref, f"rows-n q8k kind={kind} fused={fused}")
    ctx.release(wid)


@pytest.mark.parametrize("per_cu", [9, 10])
def test_gpu_ptq1_pinned_table_tail_4096(ctx, per_cu):
    """Pinned PTQ1 at 4096 columns on the table kernel: nine terms per unit leave room in
    LDS for two split pairs beside the table, so 9-10 tiles per CU run the last round as
    split pairs and 10-11 fall back to whole tiles; both must equal the oracle bit for bit
    (f32 input and both pinned Q8_0 contracts)."""
    import oracle

    import hiprt

    kind, cols = ph.KIND_PTQ1, 4096
    cus = hiprt.cu_count(0)
    rows = 64 * (per_cu * cus + 1) + 21
    # Every 128-weight unit drawn from a pool of 65536 canonically packed units: rows stay
    # distinct, and the matrix takes a fraction of the packer's time at this size.
    pool = synth.weights(kind, 512, 16384, seed=61 + per_cu).reshape(-1, 28)
    pick = np.random.default_rng(63 + per_cu).integers(0, pool.shape[0], rows * cols // 128)
    w = pool[pick].reshape(-1)
    x = synth.activations(cols, seed=62)
    wid = ctx.weight(kind, cols, rows, w)
    ref = oracle.matvec(kind, cols, rows, w, x, True, threads=THREADS)
    assert_bits_equal(ctx.project_f32(wid, rows, x, pinned=True), ref, f"pinned f32 per_cu={per_cu}")
    for contract in (1, 2):
        act = oracle.quantize_q8_0(x, contract)
        ref = oracle.project_q8(kind, cols, rows, w, act, True, threads=THREADS)
        got = ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), pinned=True)
        assert_bits_equal(got, ref, f"pinned q8 contract={contract} per_cu={per_cu}")
    ctx.release(wid)


@pytest.mark.parametrize("cols", [384, 512])
@pytest.mark.parametrize("tokens", [2, 3])
def test_gpu_ptq1_table_batch_matches_per_token_oracle(ctx, cols, tokens):
    """Two or three PTQ1 tokens on a matrix of eight tiles per CU run the table kernel
    with the unit decoded once and one chain per token: each token's row must equal its
    own matvec in every contract (source, pinned, native-scale Q8_0, Q8_K), with an odd
    unit count and a partial last tile."""
    import oracle

    import hiprt

    kind = ph.KIND_PTQ1
    rows = 64 * 8 * hiprt.cu_count(0) + 37
    w = synth.weights(kind, rows, cols, seed=43)
    wid = ctx.weight(kind, cols, rows, w)
    X = synth.activations(cols, seed=44 + tokens, tokens=tokens)
    for pinned in (False, True):
        ref = oracle.prefill(kind, cols, rows, w, X, pinned, threads=THREADS)
        got = ctx.project_f32(wid, rows, X, tokens=tokens, pinned=pinned)
        assert_bits_equal(got, ref, f"table batch f32 tokens={tokens} pinned={pinned}")
    nq8, nq8k = cols // 32, cols // 256
    for contract, pinned in ((0, False), (2, True), (2, False)):
        act = np.concatenate([oracle.quantize_q8_0(X[t], contract) for t in range(tokens)])
        ref = np.stack([oracle.project_q8(kind, cols, rows, w, act[t * nq8:(t + 1) * nq8], pinned, threads=THREADS)
                        for t in range(tokens)])
        got = ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), tokens=tokens, pinned=pinned)
        assert_bits_equal(got, ref, f"table batch q8 tokens={tokens} contract={contract} pinned={pinned}")
    if cols % 256 == 0:
        act = np.concatenate([oracle.quantize_q8k(X[t], False) for t in range(tokens)])
        got = ctx.project_q8k(wid, rows, act.view(ph.Q8K_DTYPE), tokens=tokens)
        nb = cols // 128 * 28
        sample = list(range(0, rows, 97)) + list(range(rows - 20, rows))
        ref = np.array([[oracle.dot_ptq1_q8k(w[r * nb:(r + 1) * nb], act[t * nq8k:(t + 1) * nq8k]) for r in sample]
                        for t in range(tokens)], np.float32)
        assert_bits_equal(got[:, sample], ref, f"table batch q8k tokens={tokens}")
    ctx.release(wid)


@pytest.mark.parametrize("rows", [1024 + 53, 20480 + 37, 40960 + 37, 65536 + 37, 131072 + 37])
@pytest.mark.parametrize("kind,cols", [(ph.KIND_PTQ1, 128), (ph.KIND_PTQ1, 384), (ph.KIND_PTQ1, 512), (ph.KIND_PQ2, 512),
                                       (ph.KIND_PQ2, 384), (ph.KIND_Q2_K, 512), (ph.KIND_Q8_0, 256),
                                       (ph.KIND_TQ1_0, 512), (ph.KIND_TQ2_0, 256), (ph.KIND_TQ1_0, 1280),
                                       (ph.KIND_TQ2_0, 768)])
def test_gpu_skinny_batch_matches_per_token_oracle(ctx, kind, cols, rows):
    """2..17 tokens run weights-once on the int8 matrix cores, 16 rows per block: the
    row counts cover 8, 4, 2 and 1 wavefronts per block (K split over the workgroup,
    terms folded through LDS), and rows x tokens cover both activation sources (prepared
    blocks gathered directly, or a lane-ordered copy); pinned PTQ1 takes four masked
    MFMAs per group (one per native lane subset), at most two wavefronts per block;
    TQ1_0 / TQ2_0 take each unit's integer from four MFMAs on signed digits or fields (TQ1_0's
    last byte of each lane group gathered at stride 4).  Each token's row must equal its own
    matvec, in every contract, with partial chunks of the 16-token batch, a partial last tile
    and 16-row block."""
    import oracle

    w = synth.weights(kind, rows, cols, seed=41) if kind != ph.KIND_PQ2 else synth.pq2_weights(rows, cols, 41, 4)
    wid = ctx.weight(kind, cols, rows, w)
    for tokens in (2, 5, 17):
        X = synth.activations(cols, seed=42 + tokens, tokens=tokens)
        for pinned in (False, True):
            ref = oracle.prefill(kind, cols, rows, w, X, pinned, threads=THREADS)
            got = ctx.project_f32(wid, rows, X, tokens=tokens, pinned=pinned)
            assert_bits_equal(got, ref, f"batch f32 kind={kind} tokens={tokens} pinned={pinned}")
        nq8, nq8k = cols // 32, cols // 256
        if kind not in (ph.KIND_Q2_K, ph.KIND_TQ1_0, ph.KIND_TQ2_0):
            for contract, pinned in ((0, False), (2, True)) if kind == ph.KIND_PTQ1 else ((1, False), (0, True)):
                act = np.concatenate([oracle.quantize_q8_0(X[t], contract) for t in range(tokens)])
                ref = np.stack([oracle.project_q8(kind, cols, rows, w, act[t * nq8:(t + 1) * nq8], pinned,
                                                  threads=THREADS) for t in range(tokens)])
                got = ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), tokens=tokens, pinned=pinned)
                assert_bits_equal(got, ref, f"batch q8 kind={kind} tokens={tokens} pinned={pinned}")
        if cols % 256 == 0 and kind != ph.KIND_Q8_0:
            for fused in (False, True):
                act = np.concatenate([oracle.quantize_q8k(X[t], fused) for t in range(tokens)])
                got = ctx.project_q8k(wid, rows, act.view(ph.Q8K_DTYPE), tokens=tokens, fused=fused)
                if kind == ph.KIND_PTQ1:
                    nb = cols // 128 * 28
                    sample = list(range(0, rows, 97)) + list(range(rows - 20, rows))
                    ref = np.array([[oracle.dot_ptq1_q8k(w[r * nb:(r + 1) * nb], act[t * nq8k:(t + 1) * nq8k])
                                     for r in sample] for t in range(tokens)], np.float32)
                    got = got[:, sample]
                else:
                    ref = np.stack([oracle.project_q8k(kind, cols, rows, w, act[t * nq8k:(t + 1) * nq8k], fused,
                                                       threads=THREADS) for t in range(tokens)])
                assert_bits_equal(got, ref, f"batch q8k kind={kind} tokens={tokens} fused={fused}")
    ctx.release(wid)


@pytest.mark.parametrize("rows,cols,tokens", [(5120 + 37, 17408, 2), (2048 + 5, 8192, 3), (2048 + 5, 8192, 4),
                                              (4096 - 3, 8192, 8), (1000, 16384, 6), (17408 + 37, 5120, 2),
                                              (17408 + 37, 5120, 4), (5120 + 3, 6144, 4), (6144 + 5, 5120, 3),
                                              (5120 + 37, 17408, 8)])
def test_gpu_splitk_long_rows_match_oracle(ctx, rows, cols, tokens):
    """Long PTQ1 rows on few tiles at two to eight tokens (source order) take the two-pass
    split-K: one wavefront per (tile, four units) stores each unit's term per (token, row) in
    global memory, and a fold kernel adds them in unit order.  Prepared source blocks and f32
    input (quantized first) equal the oracle's per-token matvec bit for bit (a partial last
    tile, 40 to 136 units per row, fewer and more tiles than CUs)."""
    import oracle

    w = synth.ptq1_weights(rows, cols, seed=rows + tokens)
    wid = ctx.weight(ph.KIND_PTQ1, cols, rows, w)
    X = synth.activations(cols, seed=tokens, tokens=tokens).reshape(tokens, cols)
    nq8 = cols // 32
    act = np.concatenate([oracle.quantize_q8_0(X[t], 0) for t in range(tokens)])
    ref = np.stack([oracle.project_q8(ph.KIND_PTQ1, cols, rows, w, act[t * nq8:(t + 1) * nq8], False, threads=THREADS)
                    for t in range(tokens)])
    assert_bits_equal(ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), tokens=tokens), ref,
                      f"split-K prepared {rows}x{cols} tokens={tokens}")
    ref = oracle.prefill(ph.KIND_PTQ1, cols, rows, w, X, False, threads=THREADS)
    assert_bits_equal(ctx.project_f32(wid, rows, X, tokens=tokens), ref, f"split-K f32 {rows}x{cols} tokens={tokens}")
    assert not ctx.faulted
    ctx.release(wid)


@pytest.mark.parametrize("rows,cols,tokens", [(5120 + 37, 17408, 2), (6144 + 5, 16384, 2), (4096 - 3, 14336, 3)])
def test_gpu_splitk_pq2_matches_oracle(ctx, rows, cols, tokens):
    """Long PQ2 rows on few tiles with Q8_K activations in the unfused order take the two-pass
    split-K at two tokens from 5120 rows; the fused order and three tokens keep their kernels.  Prepared blocks in both orders and f32 input equal the oracle's
    per-token matvec bit for bit."""
    import oracle

    w = synth.pq2_weights(rows, cols, rows + tokens, 4)
    wid = ctx.weight(ph.KIND_PQ2, cols, rows, w)
    X = synth.activations(cols, seed=tokens + 3, tokens=tokens).reshape(tokens, cols)
    nq8k = cols // 256
    for fused in (False, True):
        act = np.concatenate([oracle.quantize_q8k(X[t], fused) for t in range(tokens)])
        ref = np.stack([oracle.project_q8k(ph.KIND_PQ2, cols, rows, w, act[t * nq8k:(t + 1) * nq8k], fused,
                                           threads=THREADS) for t in range(tokens)])
        got = ctx.project_q8k(wid, rows, act.view(ph.Q8K_DTYPE), tokens=tokens, fused=fused)
        assert_bits_equal(got, ref, f"split-K PQ2 prepared {rows}x{cols} tokens={tokens} fused={fused}")
    ref = oracle.prefill(ph.KIND_PQ2, cols, rows, w, X, False, threads=THREADS)
    assert_bits_equal(ctx.project_f32(wid, rows, X, tokens=tokens), ref, f"split-K PQ2 f32 {rows}x{cols} tokens={tokens}")
    assert not ctx.faulted
    ctx.release(wid)


@pytest.mark.parametrize("kind,rows,cols,tokens", [(ph.KIND_PTQ1, 200, 1024, 40), (ph.KIND_PTQ1, 6144 + 37, 512, 100),
                                                   (ph.KIND_Q8_0, 300, 512, 70), (ph.KIND_Q2_K, 300, 512, 70),
                                                   (ph.KIND_PQ2, 300, 512, 70), (ph.KIND_TQ1_0, 300, 512, 70),
                                                   (ph.KIND_TQ2_0, 300, 512, 70), (ph.KIND_Q2_K, 65536 + 37, 256, 16)])
def test_gpu_prepared_activations_gemm_matches_oracle(ctx, kind, rows, cols, tokens):
    """Prepared multi-token activations take the prefill GEMMs from their token thresholds, with
    a prep that copies the blocks instead of quantizing: PTQ1 with Q8_0 blocks of each contract
    in both chain orders (f16 GEMM), Q8_0 with Q8_0 blocks, Q2_K, PQ2 (both chains), TQ1_0 and
    TQ2_0 with Q8_K blocks (int8 GEMM).  Every token row equals the oracle's matvec on that
    token's blocks, bit for bit."""
    import oracle

    w = synth.weights(kind, rows, cols, seed=rows + tokens) if kind != ph.KIND_PQ2 else \
        synth.pq2_weights(rows, cols, rows, 4)
    wid = ctx.weight(kind, cols, rows, w)
    X = synth.activations(cols, seed=tokens + kind, tokens=tokens).reshape(tokens, cols)
    nq8, nq8k = cols // 32, cols // 256
    if kind in (ph.KIND_PTQ1, ph.KIND_Q8_0):
        for contract, pinned in ((0, False), (2, True), (1, False)) if kind == ph.KIND_PTQ1 else ((1, False), (0, True)):
            act = np.concatenate([oracle.quantize_q8_0(X[t], contract) for t in range(tokens)])
            ref = np.stack([oracle.project_q8(kind, cols, rows, w, act[t * nq8:(t + 1) * nq8], pinned, threads=THREADS)
                            for t in range(tokens)])
            got = ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), tokens=tokens, pinned=pinned)
            assert_bits_equal(got, ref, f"prepared q8 kind={kind} tokens={tokens} contract={contract} pinned={pinned}")
    else:
        for fused in (False, True):
            act = np.concatenate([oracle.quantize_q8k(X[t], fused) for t in range(tokens)])
            ref = np.stack([oracle.project_q8k(kind, cols, rows, w, act[t * nq8k:(t + 1) * nq8k], fused,
                                               threads=THREADS) for t in range(tokens)])
            got = ctx.project_q8k(wid, rows, act.view(ph.Q8K_DTYPE), tokens=tokens, fused=fused)
            assert_bits_equal(got, ref, f"prepared q8k kind={kind} tokens={tokens} fused={fused}")
    assert not ctx.faulted
    ctx.release(wid)


@pytest.mark.parametrize("kind,cols,rows", [(ph.KIND_PTQ1, 128, 65536 + 37), (ph.KIND_PTQ1, 640, 65536 + 37),
                                            (ph.KIND_PTQ1, 384, 131072 + 5), (ph.KIND_Q8_0, 128, 65536 + 37),
                                            (ph.KIND_Q8_0, 640, 65536 + 1), (ph.KIND_Q8_0, 384, 131072 + 63),
                                            (ph.KIND_PTQ1, 128, 6144 + 37), (ph.KIND_PTQ1, 640, 8192 + 1),
                                            (ph.KIND_PTQ1, 4096, 6144 + 11), (ph.KIND_PTQ1, 7168, 6144),
                                            (ph.KIND_PTQ1, 384, 32768 + 77), (ph.KIND_Q8_0, 640, 6144 + 53)])
def test_gpu_quad_batch_matches_per_token_oracle(ctx, kind, cols, rows):
    """Two to four tokens of a large PTQ1 or Q8_0 matrix run on the 4x4x4 int8 matrix
    cores, one row per lane (tokens on the A side, the lane's row on the B side); with
    fewer than four tokens the last one is repeated and not stored.  Source PTQ1 takes that
    kernel from two tiles per CU (513 tiles here) and, from 3/8 of a tile per CU, splits
    each tile's units over a workgroup's wavefronts and folds the per-unit terms from LDS
    (up to 56 units per row; pinned PTQ1 and Q8_0 take the skinny kernel below 65536 rows).
    Every token's row must equal its own matvec in both contracts, through
    the f32 entry and through prepared blocks of each Q8_0 contract, with a partial last
    tile and an odd unit count."""
    import oracle

    w = synth.weights(kind, rows, cols, seed=43)
    wid = ctx.weight(kind, cols, rows, w)
    nq8 = cols // 32
    for tokens in (2, 3, 4):
        X = synth.activations(cols, seed=44 + tokens, tokens=tokens)
        for pinned in (False, True):
            ref = oracle.prefill(kind, cols, rows, w, X, pinned, threads=THREADS)
            got = ctx.project_f32(wid, rows, X, tokens=tokens, pinned=pinned)
            assert_bits_equal(got, ref, f"quad f32 kind={kind} tokens={tokens} pinned={pinned}")
        for contract, pinned in ((0, False), (2, True), (1, False)) if kind == ph.KIND_PTQ1 else ((1, False), (0, True)):
            act = np.concatenate([oracle.quantize_q8_0(X[t], contract) for t in range(tokens)])
            ref = np.stack([oracle.project_q8(kind, cols, rows, w, act[t * nq8:(t + 1) * nq8], pinned,
                                              threads=THREADS) for t in range(tokens)])
            got = ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), tokens=tokens, pinned=pinned)
            assert_bits_equal(got, ref, f"quad q8 kind={kind} tokens={tokens} contract={contract} pinned={pinned}")
    ctx.release(wid)


@pytest.mark.parametrize("cols,rows", [(256, 65536 + 37), (768, 65536 + 1), (1024, 131072 + 63)])
def test_gpu_q2k_quad_batch_matches_per_token_oracle(ctx, cols, rows):
    """Two to four tokens of a Q2_K matrix of 65536 rows or more run on the 4x4x4 int8
    matrix cores, one row per lane: the weight operand carries scale * code and a second
    product with the sub-block's min gives min * bsum, so both integer sums of
    dot_q2_k_block are exact.  Every token's row must equal its own matvec, through the f32
    entry (both Q8_K contracts) and through prepared Q8_K blocks, with a partial last tile
    and one to four units per row."""
    import oracle

    kind = ph.KIND_Q2_K
    w = synth.weights(kind, rows, cols, seed=47)
    wid = ctx.weight(kind, cols, rows, w)
    nq8k = cols // 256
    for tokens in (2, 3, 4):
        X = synth.activations(cols, seed=48 + tokens, tokens=tokens)
        for pinned in (False, True):
            ref = oracle.prefill(kind, cols, rows, w, X, pinned, threads=THREADS)
            got = ctx.project_f32(wid, rows, X, tokens=tokens, pinned=pinned)
            assert_bits_equal(got, ref, f"q2k quad f32 tokens={tokens} pinned={pinned}")
            act = np.concatenate([oracle.quantize_q8k(X[t], pinned) for t in range(tokens)])
            ref = np.stack([oracle.project_q8k(kind, cols, rows, w, act[t * nq8k:(t + 1) * nq8k], False,
                                               threads=THREADS) for t in range(tokens)])
            got = ctx.project_q8k(wid, rows, act.view(ph.Q8K_DTYPE), tokens=tokens)
            assert_bits_equal(got, ref, f"q2k quad q8k tokens={tokens} pinned={pinned}")
    ctx.release(wid)


# ---- multi-token, groups, backend op -------------------------------------------------

def test_gpu_prefill_and_mul_mat_equal_per_token_matvec(ctx):
    import oracle

    rows, cols, M = 96, 2048, 9
    for kind in (ph.KIND_PTQ1, ph.KIND_Q2_K, ph.KIND_PQ2, ph.KIND_Q8_0):
        w = synth.weights(kind, rows, cols, seed=kind)
        X = synth.activations(cols, seed=4, tokens=M)
        wid = ctx.weight(kind, cols, rows, w)
        for pinned in (False, True):
            ref = oracle.prefill(kind, cols, rows, w, X, pinned, threads=THREADS)
            assert_bits_equal(ctx.prefill(wid, rows, X, pinned=pinned), ref, f"prefill kind={kind}")
        assert_bits_equal(ctx.mul_mat(wid, rows, X), oracle.prefill(kind, cols, rows, w, X, False, THREADS), "mul_mat")
        ctx.release(wid)


@pytest.mark.parametrize("rows,cols,M", [(200, 2048, 33), (64, 384, 37), (130, 1024, 300), (6144, 2048, 128),
                                         (192, 512, 1030), (96, 256, 4100), (100, 256, 200), (320, 512, 512),
                                         (96, 256, 4096), (130, 1152, 1100), (6144, 2048, 1024),
                                         (6044, 2048, 2048), (32768 + 37, 256, 64), (32768 + 37, 256, 100),
                                         (32768 + 37, 256, 130), (8192 + 37, 256, 32), (17408 + 37, 256, 48)])
def test_gpu_prefill_gemm_equals_per_token_matvec(ctx, rows, cols, M):
    """PTQ1 prefill runs as one f16-MFMA GEMM from 32 tokens on (33 below 8192 rows), in both
    contracts; every token row must equal the reference's per-token matvec bit for bit
    (partial row tiles, idle wavefronts of a partial 128-row block, an odd block count, 32,
    64 and 128 tokens per workgroup, padding tokens, and the XCD-major grid, taken when the
    token groups are a multiple of eight: M = 200, 512, 4096; nine blocks per row at 1152
    columns, the benchmark's matrix at 1024 tokens, a partial last tile at 6044 rows and
    2048 tokens; at 32805 rows the large-matrix choice of 32, 64 and 128 tokens per
    workgroup; at 17445 rows and 48 tokens more block-split workgroups than CUs, so the
    plain kernel).  The pinned contract's
    kernel takes each native lane's integer sum from its own masked MFMA and runs the
    four FMA lanes of dot_q8_groups_pinned."""
    import oracle

    w = synth.ptq1_weights(rows, cols, seed=rows + M)
    X = synth.activations(cols, seed=M, tokens=M)
    X[3] *= 1e-3  # a token with small scales
    wid = ctx.weight(ph.KIND_PTQ1, cols, rows, w)
    ref = oracle.prefill(ph.KIND_PTQ1, cols, rows, w, X, False, threads=THREADS)
    assert_bits_equal(ctx.prefill(wid, rows, X, pinned=False), ref, f"prefill gemm {rows}x{cols} M={M}")
    assert_bits_equal(ctx.mul_mat(wid, rows, X), ref, "mul_mat gemm")
    ref = oracle.prefill(ph.KIND_PTQ1, cols, rows, w, X, True, threads=THREADS)
    assert_bits_equal(ctx.prefill(wid, rows, X, pinned=True), ref, f"pinned prefill gemm {rows}x{cols} M={M}")
    ctx.release(wid)


@pytest.mark.parametrize("kind", [ph.KIND_Q2_K, ph.KIND_PQ2, ph.KIND_Q8_0, ph.KIND_TQ1_0, ph.KIND_TQ2_0])
@pytest.mark.parametrize("rows,cols,M", [(200, 2048, 48), (64, 256, 49), (130, 1024, 300), (37, 512, 129),
                                         (6144, 2048, 128), (192, 512, 1030), (100, 768, 513), (6044, 4096, 64),
                                         (300, 1280, 16), (65536 + 37, 256, 16), (32768 + 37, 256, 128),
                                         (16384 + 37, 512, 20)])
def test_gpu_k_prefill_gemm_equals_per_token_matvec(ctx, kind, rows, cols, M):
    """Q2_K, PQ2, TQ1_0 and TQ2_0 (Q8_K activations) and Q8_0 prefill runs as one int8-MFMA
    GEMM, 32 or 64 tokens per workgroup: from 48 tokens (17 on matrices of at least 16384
    rows, 16 from 65536 rows; 16 tokens of 300 rows take the skinny kernel).  Q2_K: isum from the matrix cores on scale-weighted
    codes, msum from a binary16 product of the sub-block mins and sums, the two outer products
    of the token and row scales; PQ2: each 128-element block's integer dot on signed codes and
    its outer product of scales, folded unfused or fused by contract; Q8_0: each 32-element
    block's dot and scale product, folded block by block; TQ1_0 / TQ2_0: the unit's integer
    dot on the signed base-3 digits or 2-bit fields and one outer product of scales.  Every
    token row equals the reference's per-token matvec bit for bit, in both contracts (partial
    row tiles, a single-unit row, padding tokens, an all-zero token, the XCD-major grid)."""
    import oracle

    w = synth.weights(kind, rows, cols, seed=rows + M)
    X = synth.activations(cols, seed=M, tokens=M)
    X[3] *= 1e-3  # a token with small scales
    X[5] = 0.0    # an all-zero token
    wid = ctx.weight(kind, cols, rows, w)
    for pinned in (False, True):
        ref = oracle.prefill(kind, cols, rows, w, X, pinned, threads=THREADS)
        assert_bits_equal(ctx.prefill(wid, rows, X, pinned=pinned), ref,
                          f"gemm kind={kind} {rows}x{cols} M={M} pinned={pinned}")
    assert_bits_equal(ctx.mul_mat(wid, rows, X), oracle.prefill(kind, cols, rows, w, X, False, THREADS), "mul_mat")
    ctx.release(wid)


@pytest.mark.parametrize("kind,rows,cols", [(ph.KIND_Q2_K, 151936, 4096), (ph.KIND_Q8_0, 32768, 4096),
                                         (ph.KIND_PQ2, 32768, 4096), (ph.KIND_TQ2_0, 65536, 4096)])
def test_gpu_large_matvec_sampled_rows_match_oracle(ctx, kind, rows, cols):
    """Benchmark-sized matrices on the row-tile kernels (two wavefronts per tile here):
    every 997th row and the last row equal the oracle's matvec of those rows, in both
    contracts."""
    import oracle

    w = synth.weights(kind, rows, cols, seed=rows + kind) if kind != ph.KIND_PQ2 else \
        synth.pq2_weights(rows, cols, seed=rows, levels=4)
    x = synth.activations(cols, seed=cols + kind)
    sample = np.r_[np.arange(0, rows, 997), rows - 1]
    wsub = np.ascontiguousarray(w.reshape(rows, -1)[sample]).ravel()
    wid = ctx.weight(kind, cols, rows, w)
    for pinned in (False, True):
        ref = oracle.matvec(kind, cols, len(sample), wsub, x, pinned, threads=THREADS)
        got = ctx.project_f32(wid, rows, x, pinned=pinned)
        assert_bits_equal(got[sample], ref, f"kind={kind} {rows}x{cols} pinned={pinned}")
    ctx.release(wid)


def test_gpu_prefill_bench_shape_matches_oracle(ctx):
    """PTQ1 6144x2048 at 2048 tokens (64 tokens per workgroup, XCD-major grid): sampled
    token rows equal the oracle's per-token matvec bit for bit, and every token row equals
    the GPU's skinny-batch kernel (15 tokens per launch), itself bit-exact against the
    oracle."""
    import oracle

    rows, cols, M = 6144, 2048, 2048
    w = synth.ptq1_weights(rows, cols, seed=11)
    X = synth.activations(cols, seed=12, tokens=M)
    wid = ctx.weight(ph.KIND_PTQ1, cols, rows, w)
    Y = ctx.prefill(wid, rows, X, pinned=False)
    for t in (0, 1, 63, 64, 777, 1024, M - 1):
        ref = oracle.matvec(ph.KIND_PTQ1, cols, rows, w, X[t], False, threads=THREADS)
        assert_bits_equal(Y[t], ref, f"prefill token {t}")
    for t0 in range(0, M, 15):
        n = min(15, M - t0)
        got = ctx.project_f32(wid, rows, X[t0:t0 + n], tokens=n, pinned=False).reshape(n, rows)
        assert_bits_equal(Y[t0:t0 + n], got, f"prefill tokens {t0}..{t0 + n - 1} against the skinny kernel")
    ctx.release(wid)


def test_gpu_project_f32_group_siblings(ctx):
    import oracle

    cols = 2048
    ws = [synth.ptq1_weights(r, cols, seed=r) for r in (64, 48, 80)]
    ids = [ctx.weight(ph.KIND_PTQ1, cols, r, w) for r, w in zip((64, 48, 80), ws)]
    x = synth.activations(cols, seed=9)
    for pinned in (False, True):
        outs = ctx.project_f32_group(ids, [64, 48, 80], x, pinned=pinned)
        for r, w, o in zip((64, 48, 80), ws, outs):
            assert_bits_equal(o, oracle.matvec(ph.KIND_PTQ1, cols, r, w, x, pinned), "group")
    for i in ids:
        ctx.release(i)


# ---- FFN ------------------------------------------------------------------------------

@pytest.mark.parametrize("kind", [ph.KIND_Q2_K, ph.KIND_PQ2, ph.KIND_PTQ1, ph.KIND_Q8_0, ph.KIND_TQ1_0,
                                  ph.KIND_TQ2_0])
def test_gpu_ffn_chain(ctx, kind):
    import oracle

    hidden, ffn = 2048, 6144
    wg = synth.weights(kind, ffn, hidden, seed=1)
    wu = synth.weights(kind, ffn, hidden, seed=2)
    wd = synth.weights(kind, hidden, ffn, seed=3)
    x = synth.activations(hidden, seed=4)
    res = synth.activations(hidden, seed=5)
    g, u, d = (ctx.weight(kind, hidden, ffn, wg), ctx.weight(kind, hidden, ffn, wu), ctx.weight(kind, ffn, hidden, wd))
    # pinned: ggml vector exp + correctly rounded division -> bit-exact end to end
    ref, h = oracle.ffn(kind, hidden, ffn, wg, wu, wd, x, res, pinned=True, threads=THREADS)
    assert_bits_equal(ctx.ffn_swiglu(g, u, ffn, x, pinned=True), h, "swiglu pinned")
    assert_bits_equal(ctx.ffn_chain(g, u, d, hidden, x, res, pinned=True), ref, "ffn pinned")
    # source: libm exp on each side; compare with the tolerance stated in the module docstring
    ref, h = oracle.ffn(kind, hidden, ffn, wg, wu, wd, x, None, pinned=False, threads=THREADS)
    got_h = ctx.ffn_swiglu(g, u, ffn, x, pinned=False)
    assert np.max(np.abs(got_h - h)) <= 1e-6 * np.max(np.abs(h))
    got = ctx.ffn_chain(g, u, d, hidden, x, None, pinned=False)
    assert np.max(np.abs(got - ref)) <= 1e-3 * np.max(np.abs(ref))
    for i in (g, u, d):
        ctx.release(i)


# ---- errors ---------------------------------------------------------------------------

def test_gpu_errors_clear_output_and_do_not_latch(ctx):
    rows, cols = 8, 256
    w = bytearray(synth.ptq1_weights(rows, cols, seed=1).tobytes())
    w[28 * 5 + 26:28 * 5 + 28] = (0x7C00).to_bytes(2, "little")  # +inf scale in row 2
    wid = ctx.weight(ph.KIND_PTQ1, cols, rows, bytes(w))
    rc, out = ctx.project_f32(wid, rows, synth.activations(cols, 1), check=False)
    assert rc == ph.ERR_NONFINITE and not out.any()
    x = synth.activations(cols, 2)
    x[3] = np.inf
    good = ctx.weight(ph.KIND_PTQ1, cols, rows, synth.ptq1_weights(rows, cols, seed=2))
    rc, out = ctx.project_f32(good, rows, x, check=False)
    assert rc == ph.ERR_NONFINITE and not out.any()
    rc, out = ctx.project_q8(good, rows, np.zeros(3, ph.Q8_DTYPE), check=False)
    assert rc == ph.ERR_INVALID_INPUT and not out.any()
    assert not ctx.supports(ph.KIND_Q2_K, 256, 4, ph.PATH_Q8)
    assert not ctx.supports(ph.KIND_PQ2, 384, 4, ph.PATH_Q8K)
    assert ctx.supports(ph.KIND_PQ2, 384, 4, ph.PATH_Q8)
    assert not ctx.faulted and ctx.operation_capacity() > 0
    assert ctx.operation_count(ph.KIND_PTQ1, 2048, 16) == 2048 * 16
    ok = ctx.project_f32(good, rows, synth.activations(cols, 3))
    assert np.isfinite(ok).all()
    ctx.release(wid)
    ctx.release(good)


@pytest.mark.parametrize("kind,size", [(ph.KIND_TQ1_0, 54), (ph.KIND_TQ2_0, 66)])
@pytest.mark.parametrize("tokens", [1, 4, 64])
def test_gpu_tq_nonfinite_scale_fails_every_path(ctx, kind, size, tokens):
    """A TQ block whose binary16 scale is infinite makes the reference's dot fail (scale(),
    src/kernels.rs:152-154; src/kernels/tquants.rs:282): the one-token matvec, the skinny
    batch (4 tokens) and the int8 prefill GEMM (64 tokens) report NONFINITE, leave the output
    cleared and do not latch."""
    rows, cols = 2048, 512
    w = bytearray(synth.weights(kind, rows, cols, seed=7).tobytes())
    at = (1000 * (cols // 256) + 1) * size + size - 2  # row 1000, second block's scale
    w[at:at + 2] = (0x7C00).to_bytes(2, "little")
    wid = ctx.weight(kind, cols, rows, bytes(w))
    X = synth.activations(cols, seed=8, tokens=tokens).reshape(tokens, cols)
    rc, out = ctx.project_f32(wid, rows, X[0] if tokens == 1 else X, tokens=tokens, check=False)
    assert rc == ph.ERR_NONFINITE and not np.asarray(out).any()
    assert not ctx.faulted
    good = ctx.weight(kind, cols, rows, synth.weights(kind, rows, cols, seed=7))
    assert np.isfinite(ctx.project_f32(good, rows, X[0] if tokens == 1 else X, tokens=tokens)).all()
    ctx.release(wid)
    ctx.release(good)


def test_gpu_failed_calls_clear_outputs(ctx):
    """Every failing projection zero-fills the outputs whose length it knows, whatever the
    failure: an ineligible path (Q8_K activations for a Q8_0 weight), a bad extent, an
    unknown weight in a group, a null input."""
    rows, cols = 40, 256
    q8 = ctx.weight(ph.KIND_Q8_0, cols, rows, synth.q8_0_weights(rows, cols, seed=3))
    rc, out = ctx.project_q8k(q8, rows, np.zeros(1, ph.Q8K_DTYPE), check=False)
    assert rc == ph.ERR_UNSUPPORTED and out.shape == (rows,) and not out.any()
    rc, out = ctx.project_q8(q8, rows, np.zeros(2, ph.Q8_DTYPE), check=False)
    assert rc == ph.ERR_INVALID_INPUT and not out.any()
    good = ctx.weight(ph.KIND_PTQ1, cols, rows, synth.ptq1_weights(rows, cols, seed=4))
    rc, outs = ctx.project_f32_group([good, 987654321], [rows, rows], synth.activations(cols, 5), check=False)
    assert rc == ph.ERR_INVALID_INPUT and not outs[0].any()
    assert not ctx.faulted
    ctx.release(q8)
    ctx.release(good)


def test_gpu_device_calls_reject_a_foreign_stream(ctx):
    """Device-pointer calls share the context's scratch and error flag, so they run on the
    context stream only; another stream is an argument error that does not latch."""
    rows, cols = 64, 256
    wid = ctx.weight(ph.KIND_PTQ1, cols, rows, synth.ptq1_weights(rows, cols, seed=6))
    x = DeviceBuffer.from_numpy(synth.activations(cols, 6))
    out = DeviceBuffer(rows * 4)
    with ph.Context(0) as other:
        foreign = other.stream()
        with pytest.raises(ph.PrismError) as e:
            ctx.project_device(wid, ph.PATH_F32, x, 1, False, out, foreign)
        assert e.value.code == ph.ERR_INVALID_INPUT
    assert not ctx.faulted
    ctx.project_device(wid, ph.PATH_F32, x, 1, False, out, ctx.stream())
    assert ctx.sync() == 0
    ctx.release(wid)


@pytest.mark.parametrize("kind", [ph.KIND_PTQ1, ph.KIND_PQ2, ph.KIND_Q8_0])
def test_gpu_wide_small_matrix_keeps_a_layout_every_order_can_run(ctx, kind):
    """One 64-row tile of 32768 inputs: the small-matrix kernel's LDS cannot hold the
    activation or the pinned PTQ1 terms of such rows, so the input is quantized first and a
    row-tile kernel (no width limit) takes the tile; every contract must run and match the
    oracle, without a latch."""
    import oracle

    rows, cols = 64, 32768
    w = synth.weights(kind, rows, cols, seed=kind + 9)
    x = synth.activations(cols, seed=kind + 10)
    wid = ctx.weight(kind, cols, rows, w)
    for pinned in (False, True):
        ref = oracle.matvec(kind, cols, rows, w, x, pinned, threads=THREADS)
        assert_bits_equal(ctx.project_f32(wid, rows, x, pinned=pinned), ref, f"wide pinned={pinned}")
    if kind != ph.KIND_PQ2:
        act = oracle.quantize_q8_0(x, 2)
        ref = oracle.project_q8(kind, cols, rows, w, act, True, threads=THREADS)
        assert_bits_equal(ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), pinned=True), ref, "wide q8 pinned")
    assert not ctx.faulted
    ctx.release(wid)


@pytest.mark.parametrize("kind,rows,cols", [(ph.KIND_PTQ1, 320 + 5, 17408), (ph.KIND_PQ2, 100, 14336),
                                            (ph.KIND_Q2_K, 130, 14336), (ph.KIND_Q8_0, 200, 14336),
                                            (ph.KIND_TQ1_0, 90, 14336), (ph.KIND_TQ2_0, 70, 14336)])
def test_gpu_wide_rows_few_tiles_every_token_count(ctx, kind, rows, cols):
    """FFN-down-like widths (14336, 17408 inputs) on a few 64-row tiles, stored tiled: one
    token takes the split kernel with wider lane groups, or the row-tile fallback where its
    LDS cannot hold the rows; two or three tokens run token by token (PTQ1, PQ2) or on the
    batch kernels, and PTQ1 from 33 tokens the prefill GEMM; every output equals the
    oracle's per-token matvec."""
    import oracle

    w = synth.weights(kind, rows, cols, seed=kind + rows)
    wid = ctx.weight(kind, cols, rows, w)
    for M in (1, 2, 3, 33):
        X = synth.activations(cols, seed=M + kind, tokens=M).reshape(M, cols)
        for pinned in (False, True):
            ref = oracle.prefill(kind, cols, rows, w, X, pinned, threads=THREADS)
            got = ctx.project_f32(wid, rows, X[0], pinned=pinned) if M == 1 else ctx.prefill(wid, rows, X, pinned=pinned)
            assert_bits_equal(got.reshape(-1), ref.reshape(-1), f"wide kind={kind} {rows}x{cols} M={M} pinned={pinned}")
    if kind in (ph.KIND_PTQ1, ph.KIND_Q8_0):
        act = oracle.quantize_q8_0(synth.activations(cols, seed=7), 1)
        ref = oracle.project_q8(kind, cols, rows, w, act, True, threads=THREADS)
        assert_bits_equal(ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), pinned=True), ref, "wide q8")
    assert not ctx.faulted
    ctx.release(wid)


def test_gpu_weight_cache_by_key_and_budget():
    with ph.Context(0, max_resident_bytes=4096) as c:
        w = synth.ptq1_weights(16, 256, seed=1)
        a = c.weight(ph.KIND_PTQ1, 256, 16, w, key=42)
        b = c.weight(ph.KIND_PTQ1, 256, 16, w, key=42)
        assert a == b and c.resident_bytes() == w.size
        with pytest.raises(ph.PrismError) as e:
            c.weight(ph.KIND_PTQ1, 256, 256, synth.ptq1_weights(256, 256, seed=2), key=43)
        assert e.value.code == ph.ERR_RESOURCE


# ---- device-pointer path and determinism ----------------------------------------------

def test_gpu_device_pointer_path_matches_oracle(ctx):
    """prism_hip_project_device on a context-owned (tiled) copy of device bytes, with
    device input and output, equals the oracle; so does a repeated host call."""
    import oracle

    rows, cols = 300, 4096
    for kind in (ph.KIND_PTQ1, ph.KIND_Q2_K, ph.KIND_Q8_0, ph.KIND_PQ2):
        w = synth.weights(kind, rows, cols, seed=kind + 1)
        x = synth.activations(cols, seed=12)
        wid = ctx.weight_from_device(kind, cols, rows, DeviceBuffer.from_numpy(w))
        ref = oracle.matvec(kind, cols, rows, w, x, False, threads=THREADS)
        out = DeviceBuffer(rows * 4)
        ctx.project_device(wid, ph.PATH_F32, DeviceBuffer.from_numpy(x), 1, False, out)
        assert ctx.sync() == 0
        assert_bits_equal(out.to_numpy(np.float32), ref, f"device path kind={kind}")
        assert_bits_equal(ctx.project_f32(wid, rows, x), ref, f"host path kind={kind}")
        ctx.release(wid)


# Native row-major weights registered with prism_hip_weight_wrap_device run the
# native-layout kernels (matvec.hip): k_matvec in its unit-count buckets (16, 32, 48,
# 64 units with 16 lanes per row; 128 and 256 units with 64 lanes), four or one
# wavefronts per workgroup by the LDS the terms need, and k_matvec_generic for odd-group
# PQ2 and rows beyond 256 units or the LDS limit.  rows = 37: two full 16-row tiles and
# a partial one.
NATIVE = [(k, c) for c in (2048, 4096, 6144, 8192, 16384, 32768)
          for k in (ph.KIND_PTQ1, ph.KIND_PQ2, ph.KIND_Q2_K, ph.KIND_Q8_0)] + \
         [(ph.KIND_PQ2, 384), (ph.KIND_PQ2, 1152), (ph.KIND_PTQ1, 33024), (ph.KIND_Q8_0, 33024)]


@pytest.mark.parametrize("kind,cols", NATIVE)
def test_gpu_wrapped_native_rows_match_oracle(ctx, kind, cols):
    import oracle

    rows = 37
    w = synth.weights(kind, rows, cols, seed=cols + kind) if kind != ph.KIND_PQ2 else \
        synth.pq2_weights(rows, cols, seed=cols, levels=4)
    x = synth.activations(cols, seed=cols + 7)
    wd = DeviceBuffer.from_numpy(w)
    wid = ctx.weight_device(kind, cols, rows, wd)
    for pinned in (False, True):
        ref = oracle.matvec(kind, cols, rows, w, x, pinned, threads=THREADS)
        assert_bits_equal(ctx.project_f32(wid, rows, x, pinned=pinned), ref, f"native f32 pinned={pinned}")
    if kind in (ph.KIND_PTQ1, ph.KIND_Q8_0) or (kind == ph.KIND_PQ2 and cols % 256):
        for contract in (0, 1, 2):
            act = oracle.quantize_q8_0(x, contract)
            for pinned in (False, True):
                ref = oracle.project_q8(kind, cols, rows, w, act, pinned, threads=THREADS)
                got = ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), pinned=pinned)
                assert_bits_equal(got, ref, f"native q8 contract={contract} pinned={pinned}")
    if kind != ph.KIND_Q8_0 and cols % 256 == 0:
        for fused in (False, True):
            act = oracle.quantize_q8k(x, fused)
            if kind == ph.KIND_PTQ1:
                nb = cols // 128 * 28
                ref = np.array([oracle.dot_ptq1_q8k(w[r * nb:(r + 1) * nb], act) for r in range(rows)], np.float32)
            else:
                ref = oracle.project_q8k(kind, cols, rows, w, act, fused, threads=THREADS)
            got = ctx.project_q8k(wid, rows, act.view(ph.Q8K_DTYPE), fused=fused)
            assert_bits_equal(got, ref, f"native q8k fused={fused}")
    ctx.release(wid)


def test_gpu_wrapped_native_multi_token_matches_oracle(ctx):
    """Several tokens through the native-layout kernels (one launch per token)."""
    import oracle

    rows, cols, M = 70, 2048, 3
    for kind in (ph.KIND_PTQ1, ph.KIND_Q2_K, ph.KIND_Q8_0, ph.KIND_PQ2):
        w = synth.weights(kind, rows, cols, seed=kind + 3)
        X = synth.activations(cols, seed=kind, tokens=M)
        wd = DeviceBuffer.from_numpy(w)
        wid = ctx.weight_device(kind, cols, rows, wd)
        for pinned in (False, True):
            ref = oracle.prefill(kind, cols, rows, w, X, pinned, threads=THREADS)
            assert_bits_equal(ctx.project_f32(wid, rows, X, tokens=M, pinned=pinned), ref, f"native tokens {kind}")
        ctx.release(wid)


def test_gpu_q8_0_rounding_order_known_answers(ctx):
    """The hand-derived Q8_0 x Q8_0 answers (fixtures_util.q8_0_order_kats) on the tiled
    and the native-layout kernels."""
    for name, w, act, want, _ in fx.q8_0_order_kats():
        cols = len(w) // 34 * 32
        act = act.view(ph.Q8_DTYPE)
        tiled = ctx.weight(ph.KIND_Q8_0, cols, 1, w)
        assert int(bits(ctx.project_q8(tiled, 1, act))[0]) == want, name
        ctx.release(tiled)
        wd = DeviceBuffer.from_numpy(np.frombuffer(w, np.uint8).copy())
        native = ctx.weight_device(ph.KIND_Q8_0, cols, 1, wd)
        assert int(bits(ctx.project_q8(native, 1, act))[0]) == want, name
        ctx.release(native)


@pytest.mark.parametrize("kind", [ph.KIND_TQ1_0, ph.KIND_TQ2_0])
def test_gpu_wrapped_native_tq_rows_match_oracle(ctx, kind):
    """A caller-owned device buffer in the native row-major layout (no tiled copy) runs
    the reference-order row kernel; it must match the oracle like the tiled path."""
    import oracle

    rows, cols = 70, 1024
    w = synth.weights(kind, rows, cols, seed=kind)
    x = synth.activations(cols, seed=13)
    wd = DeviceBuffer.from_numpy(w)
    wid = ctx.weight_device(kind, cols, rows, wd)
    for pinned in (False, True):
        ref = oracle.matvec(kind, cols, rows, w, x, pinned, threads=THREADS)
        assert_bits_equal(ctx.project_f32(wid, rows, x, pinned=pinned), ref, f"native kind={kind} pinned={pinned}")
    ctx.release(wid)
