"""GPU tests of the executor surface beyond single projections: the trait's eligibility
queries, the multi-token sibling and FFN entry points, and weights whose tiled layout
lives in caller-owned device memory.

Every projection output is compared with the oracle per token (0 ULP); the pinned FFN
chain is bit-exact end to end, the source chain (device libm exp in SiLU) is compared
with max |diff| <= 1e-3 * max |ref|, as the single-token chain tests do.
"""

import os

import numpy as np
import pytest

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
        idx = np.nonzero(g.ravel() != r.ravel())[0]
        i = idx[0]
        raise AssertionError(f"{what}: {idx.size} mismatches, first at {i}: gpu={np.float32(got.flat[i])!r} "
                             f"oracle={np.float32(ref.flat[i])!r}")


# ---- eligibility (projection.rs:112-114, 212-214, 261-269) ----------------------------

def test_gpu_eligibility_queries(ctx):
    P, Q2, PQ, Q8 = ph.KIND_PTQ1, ph.KIND_Q2_K, ph.KIND_PQ2, ph.KIND_Q8_0
    assert ctx.supports_tile_tokens()
    # groups: one width, one contract whatever `pinned` is
    assert ctx.supports_f32_group([(P, 2048, 2048), (P, 2048, 512), (P, 2048, 512)])
    assert ctx.supports_f32_group([(Q2, 2048, 6144), (Q2, 2048, 6144)])
    assert ctx.supports_f32_group([(PQ, 2048, 64), (Q2, 2048, 64)])  # both Q8_K
    assert not ctx.supports_f32_group([(P, 2048, 64), (Q2, 2048, 64)])  # Q8_0 vs Q8_K
    assert not ctx.supports_f32_group([(P, 2048, 64), (P, 1024, 64)])  # widths differ
    # odd-group PQ2 and PTQ1 share Q8_0 in the source contract but not when pinned
    assert not ctx.supports_f32_group([(PQ, 384, 64), (P, 384, 64)])
    assert not ctx.supports_f32_group([(P, 2048, 64)] * 9)
    assert not ctx.supports_f32_group([])
    assert not ctx.supports_f32_group([(P, 2000, 64)])  # incomplete block
    # FFN
    assert ctx.supports_f32_ffn_swiglu((Q2, 2048, 6144), (Q2, 2048, 6144))
    assert ctx.supports_f32_ffn_swiglu((P, 2048, 6144), (P, 2048, 6144))
    assert not ctx.supports_f32_ffn_swiglu((Q2, 2048, 6144), (P, 2048, 6144))
    assert not ctx.supports_f32_ffn_swiglu((Q2, 2048, 6144), (Q2, 2048, 4096))
    assert ctx.supports_f32_ffn_chain((Q2, 2048, 6144), (Q2, 2048, 6144), (Q2, 6144, 2048))
    assert ctx.supports_f32_ffn_chain((Q8, 2048, 6144), (Q8, 2048, 6144), (Q8, 6144, 2048))
    assert not ctx.supports_f32_ffn_chain((Q2, 2048, 6144), (Q2, 2048, 6144), (Q2, 2048, 6144))
    assert not ctx.supports_f32_ffn_chain((Q2, 2048, 6144), (Q2, 2048, 6144), (P, 6144, 2048))
    assert not ctx.faulted


# ---- multi-token siblings (projection.rs:158-210) -------------------------------------

@pytest.mark.parametrize("kind,tokens", [(ph.KIND_PTQ1, 1), (ph.KIND_PTQ1, 3), (ph.KIND_PTQ1, 16),
                                         (ph.KIND_PTQ1, 21), (ph.KIND_Q2_K, 5), (ph.KIND_Q8_0, 4),
                                         (ph.KIND_PQ2, 7)])
def test_gpu_group_tokens_match_oracle(ctx, kind, tokens):
    import oracle

    cols = 2048
    rows = (2048, 512, 512)  # a q/k/v-shaped triple; the pair is its first two
    ws = [synth.weights(kind, r, cols, seed=100 + i) for i, r in enumerate(rows)]
    ids = [ctx.weight(kind, cols, r, w) for r, w in zip(rows, ws)]
    X = synth.activations(cols, seed=7, tokens=tokens).reshape(tokens, cols)
    for n in (2, 3):
        for pinned in (False, True):
            outs = ctx.project_f32_group_tokens(ids[:n], rows[:n], X, pinned=pinned)
            for i in range(n):
                for t in sorted({0, tokens // 2, tokens - 1}):
                    ref = oracle.matvec(kind, cols, rows[i], ws[i], X[t], pinned, threads=THREADS)
                    assert_bits_equal(outs[i][t], ref, f"member {i} token {t} pinned={pinned}")
    for i in ids:
        ctx.release(i)


def test_gpu_group_tokens_errors_clear_outputs(ctx):
    cols = 512
    a = ctx.weight(ph.KIND_PTQ1, cols, 64, synth.ptq1_weights(64, cols, seed=1))
    b = ctx.weight(ph.KIND_Q2_K, cols, 64, synth.q2k_weights(64, cols, seed=2))
    X = synth.activations(cols, seed=3, tokens=4).reshape(4, cols)
    rc, outs = ctx.project_f32_group_tokens([a, b], [64, 64], X, check=False)
    assert rc == ph.ERR_UNSUPPORTED and not any(o.any() for o in outs)
    assert not ctx.faulted
    ctx.release(a)
    ctx.release(b)


# ---- multi-token FFN (projection.rs:239-259, 328-355) ---------------------------------

@pytest.mark.parametrize("kind", [ph.KIND_Q2_K, ph.KIND_PTQ1, ph.KIND_PQ2, ph.KIND_Q8_0])
def test_gpu_ffn_tokens(ctx, kind):
    import oracle

    hidden, ffn, tokens = 2048, 6144, 5
    wg = synth.weights(kind, ffn, hidden, seed=1)
    wu = synth.weights(kind, ffn, hidden, seed=2)
    wd = synth.weights(kind, hidden, ffn, seed=3)
    X = synth.activations(hidden, seed=4, tokens=tokens).reshape(tokens, hidden)
    R = synth.activations(hidden, seed=5, tokens=tokens).reshape(tokens, hidden)
    g, u, d = (ctx.weight(kind, hidden, ffn, wg), ctx.weight(kind, hidden, ffn, wu), ctx.weight(kind, ffn, hidden, wd))
    # pinned: bit-exact against the oracle for two tokens, and every token equals the
    # single-token chain (itself bit-exact against the oracle in the FFN chain tests)
    H = ctx.ffn_swiglu_tokens(g, u, ffn, X, pinned=True)
    Y = ctx.ffn_chain_tokens(g, u, d, hidden, X, R, pinned=True)
    for t in (0, tokens - 1):
        ref, h = oracle.ffn(kind, hidden, ffn, wg, wu, wd, X[t], R[t], pinned=True, threads=THREADS)
        assert_bits_equal(H[t], h, f"swiglu pinned token {t}")
        assert_bits_equal(Y[t], ref, f"chain pinned token {t}")
    for t in range(tokens):
        assert_bits_equal(Y[t], ctx.ffn_chain(g, u, d, hidden, X[t], R[t], pinned=True), f"chain vs single {t}")
    # source: device libm exp in SiLU
    Y = ctx.ffn_chain_tokens(g, u, d, hidden, X, None, pinned=False)
    for t in (0, tokens - 1):
        ref, _ = oracle.ffn(kind, hidden, ffn, wg, wu, wd, X[t], None, pinned=False, threads=THREADS)
        assert np.max(np.abs(Y[t] - ref)) <= 1e-3 * np.max(np.abs(ref))
    for i in (g, u, d):
        ctx.release(i)


def test_gpu_ffn_tokens_prefill_sized(ctx):
    """32 tokens of PTQ1 in the source contract: gate and up take the tiled-prefill GEMM,
    the down projection too, with the residual added after it."""
    import oracle

    kind, hidden, ffn, tokens = ph.KIND_PTQ1, 2048, 6144, 32
    wg = synth.weights(kind, ffn, hidden, seed=11)
    wu = synth.weights(kind, ffn, hidden, seed=12)
    wd = synth.weights(kind, hidden, ffn, seed=13)
    X = synth.activations(hidden, seed=14, tokens=tokens).reshape(tokens, hidden)
    R = synth.activations(hidden, seed=15, tokens=tokens).reshape(tokens, hidden)
    g, u, d = (ctx.weight(kind, hidden, ffn, wg), ctx.weight(kind, hidden, ffn, wu), ctx.weight(kind, ffn, hidden, wd))
    Y = ctx.ffn_chain_tokens(g, u, d, hidden, X, R, pinned=True)
    for t in (0, 17, 31):
        ref, _ = oracle.ffn(kind, hidden, ffn, wg, wu, wd, X[t], R[t], pinned=True, threads=THREADS)
        assert_bits_equal(Y[t], ref, f"pinned token {t}")
    Y = ctx.ffn_chain_tokens(g, u, d, hidden, X, R, pinned=False)
    for t in (0, 31):
        assert np.max(np.abs(Y[t] - ctx.ffn_chain(g, u, d, hidden, X[t], R[t], pinned=False))) == 0.0
    for i in (g, u, d):
        ctx.release(i)


# ---- tiled layout in caller-owned memory (src/backend/allocator.rs:10-50) ------------

@pytest.mark.parametrize("kind,rows,cols", [(ph.KIND_PTQ1, 2048, 2048), (ph.KIND_PTQ1, 1000, 4096),
                                            (ph.KIND_Q2_K, 6144, 2048), (ph.KIND_Q8_0, 20000, 1024),
                                            (ph.KIND_PQ2, 300, 2048)])
def test_gpu_caller_owned_tiled_weights(ctx, kind, rows, cols):
    import oracle

    w = synth.weights(kind, rows, cols, seed=rows + kind)
    native = DeviceBuffer.from_numpy(w)
    nbytes = ctx.tiled_bytes(kind, cols, rows)
    assert nbytes >= w.size and nbytes - w.size < 8 * w.size // rows
    tiled = DeviceBuffer(nbytes)
    tiled.upload(np.full(nbytes, 0xA5, np.uint8))  # padding must be cleared by the repack
    ctx.repack_tiled(kind, cols, rows, native, tiled)
    native.free()  # the wrapped buffer alone must serve the projections
    before = ctx.resident_bytes()
    wid = ctx.weight_tiled_device(kind, cols, rows, tiled)
    assert ctx.resident_bytes() == before  # the caller owns the memory
    X = synth.activations(cols, seed=3, tokens=3).reshape(3, cols)
    for pinned in (False, True):
        ref = oracle.matvec(kind, cols, rows, w, X[0], pinned, threads=THREADS)
        assert_bits_equal(ctx.project_f32(wid, rows, X[0], pinned=pinned), ref, f"pinned={pinned}")
        Y = ctx.project_f32(wid, rows, X, tokens=3, pinned=pinned)
        assert_bits_equal(Y[2], oracle.matvec(kind, cols, rows, w, X[2], pinned, threads=THREADS), "token 2")
    ctx.release(wid)
    tiled.free()


def test_gpu_caller_owned_tiled_rejects_bad_sizes(ctx):
    rows, cols = 256, 2048
    w = synth.ptq1_weights(rows, cols, seed=1)
    native = DeviceBuffer.from_numpy(w)
    nbytes = ctx.tiled_bytes(ph.KIND_PTQ1, cols, rows)
    small = DeviceBuffer(nbytes - 64)
    with pytest.raises(ph.PrismError) as e:
        ctx.repack_tiled(ph.KIND_PTQ1, cols, rows, native, small)
    assert e.value.code == ph.ERR_INVALID_INPUT
    with pytest.raises(ph.PrismError) as e:
        ctx.weight_tiled_device(ph.KIND_PTQ1, cols, rows, small)
    assert e.value.code == ph.ERR_INVALID_INPUT
    # Every width has a tiled layout (one 64-row tile of 32768 Q8_0 inputs: the native bytes,
    # no padding rows), and the repack refuses a destination of another size; only a tensor
    # whose 64-row tile passes 2 GiB (32-bit in-tile offsets) has none.
    assert ctx.tiled_bytes(ph.KIND_Q8_0, 32768, 64) == 64 * (32768 // 32) * 34
    q8 = DeviceBuffer.from_numpy(synth.q8_0_weights(64, 32768, seed=2))
    with pytest.raises(ph.PrismError) as e:
        ctx.repack_tiled(ph.KIND_Q8_0, 32768, 64, q8, small)
    assert e.value.code == ph.ERR_INVALID_INPUT
    assert ctx.tiled_bytes(ph.KIND_Q8_0, 32 << 20, 64) == 0
    assert not ctx.faulted


# ---- LoRA FFN chain (projection.rs:290-326, 653-697) ---------------------------------

@pytest.mark.parametrize("kind", [ph.KIND_PTQ1, ph.KIND_Q2_K])
def test_gpu_ffn_chain_lora_matches_chain_and_oracle_dot(ctx, kind):
    """The chain's output equals prism_hip_ffn_chain's bit for bit, and the LoRA A dot
    equals the oracle's lora_a_dot of the same SwiGLU vector (prism_hip_ffn_swiglu, the
    same kernels) bit for bit, in both contracts: a sparse factor (every partial sum exact:
    the workgroup's tree sum), a dense N(0, 1) factor and one spanning 1e-30..1e20 (the
    index-ordered fallback when the exactness bound fails)."""
    import oracle

    hidden, ffn = 2048, 6144
    wg = synth.weights(kind, ffn, hidden, seed=21)
    wu = synth.weights(kind, ffn, hidden, seed=22)
    wd = synth.weights(kind, hidden, ffn, seed=23)
    g, u, d = (ctx.weight(kind, hidden, ffn, wg), ctx.weight(kind, hidden, ffn, wu), ctx.weight(kind, ffn, hidden, wd))
    assert ctx.supports_f32_ffn_chain_lora((kind, hidden, ffn), (kind, hidden, ffn), (kind, ffn, hidden))
    x = synth.activations(hidden, seed=24)
    r = synth.activations(hidden, seed=25)
    rng = np.random.default_rng(26)
    sparse = np.zeros(ffn, np.float32)
    sparse[rng.choice(ffn, 12, replace=False)] = rng.integers(-64, 65, 12) / 64.0
    dense = rng.standard_normal(ffn).astype(np.float32)
    wide = (rng.standard_normal(ffn) * 10.0 ** rng.uniform(-30, 20, ffn)).astype(np.float32)
    for pinned in (False, True):
        h = ctx.ffn_swiglu(g, u, ffn, x, pinned=pinned)
        chain = ctx.ffn_chain(g, u, d, hidden, x, r, pinned=pinned)
        for name, la in (("sparse", sparse), ("dense", dense), ("wide", wide)):
            out, dot = ctx.ffn_chain_lora(g, u, d, hidden, x, la, r, pinned=pinned)
            assert_bits_equal(out, chain, f"{name} pinned={pinned} output")
            want = oracle.lora_a_dot(la, h, pinned)
            assert_bits_equal(np.float32(dot), np.float32(want), f"{name} pinned={pinned} dot")
    # 6144 % 16 == 0: the pinned contract takes the lanes; a planted NaN in the factor is
    # refused before any launch and clears the output.
    bad = dense.copy()
    bad[17] = np.nan
    (rc, out), dot = ctx.ffn_chain_lora(g, u, d, hidden, x, bad, r, pinned=True, check=False)
    assert rc == ph.ERR_INVALID_INPUT and not out.any() and dot == 0.0
    assert not ctx.faulted
    for i in (g, u, d):
        ctx.release(i)


# ---- rotated FFN chain: hadamard_block_size (projection.rs:271-355) -------------------

@pytest.mark.parametrize("kind", [ph.KIND_PTQ1, ph.KIND_Q2_K, ph.KIND_Q8_0, ph.KIND_PQ2, ph.KIND_TQ1_0,
                                  ph.KIND_TQ2_0])
def test_gpu_ffn_chain_hadamard(ctx, kind):
    """The SwiGLU vector rotated blockwise ahead of down: pinned bit-exact against the
    oracle's rotated chain for blocks of 32, 256 and 2048 (the SwiGLU width is 6144), on a
    single token, three tokens and the LoRA chain (whose dot takes the unrotated vector);
    block 1 is no rotation; a block that is not a power of two, does not divide 6144 or
    exceeds 8192 is refused with a zeroed output."""
    import oracle

    hidden, ffn = 2048, 6144
    wg = synth.weights(kind, ffn, hidden, seed=31)
    wu = synth.weights(kind, ffn, hidden, seed=32)
    wd = synth.weights(kind, hidden, ffn, seed=33)
    g, u, d = (ctx.weight(kind, hidden, ffn, wg), ctx.weight(kind, hidden, ffn, wu), ctx.weight(kind, ffn, hidden, wd))
    X = synth.activations(hidden, seed=34, tokens=3).reshape(3, hidden)
    R = synth.activations(hidden, seed=35, tokens=3).reshape(3, hidden)
    la = np.random.default_rng(36).standard_normal(ffn).astype(np.float32)
    plain = ctx.ffn_chain(g, u, d, hidden, X[0], R[0], pinned=True)
    assert_bits_equal(ctx.ffn_chain(g, u, d, hidden, X[0], R[0], pinned=True, hadamard_block=1), plain, "block 1")
    _, plain_dot = ctx.ffn_chain_lora(g, u, d, hidden, X[0], la, R[0], pinned=True)
    for block in (32, 256, 2048):
        ref, _ = oracle.ffn(kind, hidden, ffn, wg, wu, wd, X[0], R[0], pinned=True, threads=THREADS,
                            hadamard_block=block)
        got = ctx.ffn_chain(g, u, d, hidden, X[0], R[0], pinned=True, hadamard_block=block)
        assert_bits_equal(got, ref, f"block {block}")
        assert not np.array_equal(got, plain)
        out, dot = ctx.ffn_chain_lora(g, u, d, hidden, X[0], la, R[0], pinned=True, hadamard_block=block)
        assert_bits_equal(out, ref, f"lora block {block}")
        assert_bits_equal(np.float32(dot), np.float32(plain_dot), f"lora dot block {block}")
        Y = ctx.ffn_chain_tokens(g, u, d, hidden, X, R, pinned=True, hadamard_block=block)
        assert_bits_equal(Y[0], ref, f"tokens block {block}")
        for t in (1, 2):
            assert_bits_equal(Y[t], ctx.ffn_chain(g, u, d, hidden, X[t], R[t], pinned=True, hadamard_block=block),
                              f"token {t} block {block}")
    ref, _ = oracle.ffn(kind, hidden, ffn, wg, wu, wd, X[1], None, pinned=False, threads=THREADS, hadamard_block=256)
    got = ctx.ffn_chain(g, u, d, hidden, X[1], None, pinned=False, hadamard_block=256)
    assert np.max(np.abs(got - ref)) <= 1e-3 * np.max(np.abs(ref))
    # Device pointers: the same bits, and h receives the unrotated SwiGLU vector.
    xd, rd = DeviceBuffer.from_numpy(X[0]), DeviceBuffer.from_numpy(R[0])
    od, hd = DeviceBuffer(hidden * 4), DeviceBuffer(ffn * 4)
    ctx.ffn_chain_device(g, u, d, xd, rd, True, od, hd, hadamard_block=256)
    assert ctx.sync() == 0
    assert_bits_equal(od.to_numpy(np.float32), ctx.ffn_chain(g, u, d, hidden, X[0], R[0], pinned=True,
                                                            hadamard_block=256), "device block 256")
    assert_bits_equal(hd.to_numpy(np.float32), ctx.ffn_swiglu(g, u, ffn, X[0], pinned=True), "device h")
    for bad in (96, 4096, 16384):
        rc, out = ctx.ffn_chain(g, u, d, hidden, X[0], R[0], pinned=True, check=False, hadamard_block=bad)
        assert rc == ph.ERR_INVALID_INPUT and not out.any(), bad
        rc, out = ctx.ffn_chain_tokens(g, u, d, hidden, X, R, pinned=True, check=False, hadamard_block=bad)
        assert rc == ph.ERR_INVALID_INPUT and not out.any(), bad
    assert not ctx.faulted
    for i in (g, u, d):
        ctx.release(i)


# ---- latched device fault (tools/adreno-vulkan/src/executor.rs:1507-1530) -------------

def test_gpu_latched_fault_refuses_everything():
    """A latched fault (forced from the host: no GPU is faulted) makes every eligibility
    query false and the capacity 0, and every call fails with PRISM_ERR_DEVICE_FAULT and a
    cleared output, weight uploads and decoders included; another context is unaffected."""
    P, Q2 = ph.KIND_PTQ1, ph.KIND_Q2_K
    cols, rows = 2048, 128
    w = synth.ptq1_weights(rows, cols, seed=41)
    x = synth.activations(cols, seed=42)
    c = ph.Context(0)
    other = ph.Context(0)
    try:
        wid = c.weight(P, cols, rows, w)
        good = c.project_f32(wid, rows, x)
        assert c.supports(P, cols, rows, ph.PATH_F32) and c.supports_tile_tokens()
        assert c.operation_capacity() > 0 and c.operation_count(P, cols, rows) == cols * rows
        c.inject_fault()
        assert c.faulted and "latched" in c.last_error
        assert not any(c.supports(P, cols, rows, path) for path in (ph.PATH_Q8K, ph.PATH_Q8, ph.PATH_F32))
        assert not c.supports_f32_group([(P, cols, rows), (P, cols, rows)])
        assert not c.supports_f32_ffn_swiglu((Q2, 2048, 6144), (Q2, 2048, 6144))
        assert not c.supports_f32_ffn_chain((Q2, 2048, 6144), (Q2, 2048, 6144), (Q2, 6144, 2048))
        assert not c.supports_f32_ffn_chain_lora((Q2, 2048, 6144), (Q2, 2048, 6144), (Q2, 6144, 2048))
        assert not c.supports_tile_tokens()
        assert c.operation_capacity() == 0 and c.operation_count(P, cols, rows) == -1
        for tokens in (1, 4, 32):
            X = synth.activations(cols, seed=43, tokens=tokens).reshape(tokens, cols)
            rc, out = c.project_f32(wid, rows, X, tokens=tokens, check=False)
            assert rc == ph.ERR_DEVICE_FAULT and not out.any(), tokens
        with pytest.raises(ph.PrismError) as e:
            c.weight(P, cols, rows, w, key=7)
        assert e.value.code == ph.ERR_DEVICE_FAULT
        with pytest.raises(ph.PrismError) as e:
            ph.Decoder(c, synth.decoder_model(44, kv_prefill=4, hidden=512, ffn=1024, heads=4, kv_heads=2,
                                              vocab=2048, layers=1, max_tokens=16))
        assert e.value.code == ph.ERR_DEVICE_FAULT
        assert not other.faulted
        oid = other.weight(P, cols, rows, w)
        assert_bits_equal(other.project_f32(oid, rows, x), good, "other context")
    finally:
        c.close()
        other.close()


# ---- statistics (MatvecStatistics / MatvecDiagnostics, src/kernels.rs:1725-1830) ------

def test_gpu_statistics_and_diagnostics():
    """A fresh context counts per matrix: a successful F32 projection (one preparation,
    one attempt, one success, one device operation), an unknown weight id (rejected
    before dispatch), a null input (a preparation failure, no matrix attempt), a
    three-member group (three attempts, one grouped dispatch, one shared preparation) and
    a prepared Q8_0 call (no preparation).  The diagnostics follow the last call."""
    c = ph.Context(0)
    try:
        zero = {k: 0 for k in ("preparations", "preparation_failures", "matrix_attempts", "matrix_successes",
                               "rejected_before_dispatch", "device_operations", "grouped_dispatches")}
        assert c.statistics() == zero
        assert c.diagnostics() == {"dispatched": False, "succeeded": False}
        cols, rows = 2048, 256
        w = synth.ptq1_weights(rows, cols, seed=5)
        wid = c.weight(ph.KIND_PTQ1, cols, rows, w)
        x = synth.activations(cols, seed=6)
        c.project_f32(wid, rows, x)
        want = dict(zero, preparations=1, matrix_attempts=1, matrix_successes=1, device_operations=1)
        assert c.statistics() == want
        assert c.diagnostics() == {"dispatched": True, "succeeded": True}
        rc, _ = c.project_f32(wid + 1000, rows, x, check=False)
        assert rc == ph.ERR_INVALID_INPUT
        want.update(preparations=2, matrix_attempts=2, rejected_before_dispatch=1)
        assert c.statistics() == want
        assert c.diagnostics() == {"dispatched": False, "succeeded": False}
        rc = ph.lib().prism_hip_project_f32(c._h, wid, None, 1, 0, None)
        assert rc == ph.ERR_INVALID_INPUT
        want.update(preparations=3, preparation_failures=1)
        assert c.statistics() == want
        ids = [c.weight(ph.KIND_PTQ1, cols, r, synth.ptq1_weights(r, cols, seed=r)) for r in (64, 128, 64)]
        c.project_f32_group(ids, [64, 128, 64], x)
        want.update(preparations=4, matrix_attempts=5, matrix_successes=4, device_operations=4, grouped_dispatches=1)
        assert c.statistics() == want
        import oracle

        act = oracle.quantize_q8_0(x, ph.Q8_SOURCE)
        c.project_q8(wid, rows, act)
        want.update(matrix_attempts=6, matrix_successes=5, device_operations=5)
        assert c.statistics() == want
        assert c.diagnostics() == {"dispatched": True, "succeeded": True}
    finally:
        c.close()
