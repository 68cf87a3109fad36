"""The benchmark workloads at their stated sizes, through the C ABI, against the oracle.

- c0: PTQ1 2048x2048 matvec, every row.
- c2: PTQ1 6144x2048 prefill, M = 128, 512 and 2048, source and pinned, sampled tokens.
- c4: W 12288x4096 in PTQ1, Q2_K and Q8_0, every row, batch 1, 4 and 16 (the 192-tile
  split plan of the small-matrix kernel at batch 1, the matrix-core skinny kernel at 4
  and 16); the 151936x4096 LM-head shape in the same formats, sampled rows, batch 1, 4
  and 16.
- c3: the 28-layer synthetic decoder, four teacher-forced greedy steps from a
  1024-token cache (graph replay).

Tolerance: 0 ULP for every matvec output; the decoder's logits within
1e-3 * max |logit| with equal greedy tokens (test_gpu_decoder.check_against_oracle).
"""

import os

import numpy as np
import pytest

import prism_hip as ph
import synth

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)
FORMATS = (ph.KIND_PTQ1, ph.KIND_Q2_K, ph.KIND_Q8_0)


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
        idx = np.argwhere(g != r)
        raise AssertionError(f"{what}: {len(idx)} mismatches, first at {tuple(idx[0])}")


def test_gpu_c0_ptq1_2048_every_row(ctx):
    import oracle

    rows = cols = 2048
    w = synth.ptq1_weights(rows, cols, seed=0)
    x = synth.activations(cols, seed=0)
    wid = ctx.weight(ph.KIND_PTQ1, cols, rows, w)
    for pinned in (False, True):
        ref = oracle.matvec(ph.KIND_PTQ1, cols, rows, w, x, pinned, threads=THREADS)
        assert_bits_equal(ctx.project_f32(wid, rows, x, pinned=pinned), ref, f"c0 pinned={pinned}")
    for contract in (0, 2):
        act = oracle.quantize_q8_0(x, contract)
        ref = oracle.project_q8(ph.KIND_PTQ1, cols, rows, w, act, contract == 2, threads=THREADS)
        assert_bits_equal(ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), pinned=contract == 2), ref, "c0 q8")
    ctx.release(wid)


@pytest.mark.parametrize("kind", FORMATS)
def test_gpu_c4_12288x4096_every_row(ctx, kind):
    """Batch 1 (f32 and prepared activations, both contracts) and batches 4 and 16, every
    row of every token against the oracle's per-token matvec."""
    import oracle

    rows, cols = 12288, 4096
    w = synth.weights(kind, rows, cols, seed=kind + 100)
    wid = ctx.weight(kind, cols, rows, w)
    x = synth.activations(cols, seed=kind)
    for pinned in (False, True):
        ref = oracle.matvec(kind, cols, rows, w, x, pinned, threads=THREADS)
        assert_bits_equal(ctx.project_f32(wid, rows, x, pinned=pinned), ref, f"B=1 pinned={pinned}")
    if kind == ph.KIND_Q2_K:
        for fused in (False, True):
            act = oracle.quantize_q8k(x, fused)
            ref = oracle.project_q8k(kind, cols, rows, w, act, fused, threads=THREADS)
            assert_bits_equal(ctx.project_q8k(wid, rows, act.view(ph.Q8K_DTYPE), fused=fused), ref, "B=1 q8k")
    else:
        for contract, pinned in ((0, False), (1, True), (2, True)):
            act = oracle.quantize_q8_0(x, contract)
            ref = oracle.project_q8(kind, cols, rows, w, act, pinned, threads=THREADS)
            assert_bits_equal(ctx.project_q8(wid, rows, act.view(ph.Q8_DTYPE), pinned=pinned), ref, "B=1 q8")
    for tokens in (4, 16):
        X = synth.activations(cols, seed=kind + tokens, tokens=tokens)
        for pinned in (False, True):
            ref = oracle.prefill(kind, cols, rows, w, X, pinned, threads=THREADS)
            got = ctx.project_f32(wid, rows, X, tokens=tokens, pinned=pinned)
            assert_bits_equal(got, ref, f"B={tokens} pinned={pinned}")
    ctx.release(wid)


@pytest.mark.parametrize("M", [128, 512, 2048])
def test_gpu_c2_prefill_both_contracts_every_token(ctx, M):
    """The prefill workload (PTQ1 6144x2048, M tokens) in both contracts: the source
    contract on the f16-MFMA GEMM, the pinned one (the contract the reference's graph
    hands the executor) on its own GEMM.  Every token and every row against the oracle's
    per-token matvec (about 1.3 ms of host work per token at 16 threads)."""
    import oracle

    rows, cols = 6144, 2048
    w = synth.ptq1_weights(rows, cols, seed=9)
    X = synth.activations(cols, seed=10 + M, tokens=M)
    wid = ctx.weight(ph.KIND_PTQ1, cols, rows, w)
    for pinned in (False, True):
        Y = ctx.prefill(wid, rows, X, pinned=pinned)
        ref = oracle.prefill(ph.KIND_PTQ1, cols, rows, w, X, pinned, threads=THREADS)
        assert_bits_equal(Y, ref, f"M={M} pinned={pinned}")
    ctx.release(wid)


@pytest.fixture(scope="module")
def lm_head_weights():
    cache = {}

    def get(kind):
        if kind not in cache:
            cache.clear()  # one 151936 x 4096 matrix in host memory at a time
            cache[kind] = synth.weights(kind, 151936, 4096, seed=kind + 200)
        return cache[kind]

    return get


@pytest.mark.parametrize("kind", FORMATS)
def test_gpu_c4_151936x4096_every_row(ctx, lm_head_weights, kind):
    """The LM-head shape: every row, batch 1, 4 and 16, both contracts, equal to the
    oracle's matvec (20 to 60 ms of host work per token at 16 threads)."""
    import oracle

    rows, cols = 151936, 4096
    w = lm_head_weights(kind)
    wid = ctx.weight(kind, cols, rows, w)
    for tokens in (1, 4, 16):
        X = synth.activations(cols, seed=kind + 7 * tokens, tokens=tokens)
        for pinned in (False, True):
            ref = oracle.prefill(kind, cols, rows, w, X.reshape(tokens, cols), pinned, threads=THREADS)
            got = ctx.project_f32(wid, rows, X, tokens=tokens, pinned=pinned).reshape(tokens, rows)
            assert_bits_equal(got, ref, f"B={tokens} pinned={pinned}")
    ctx.release(wid)


def test_gpu_c3_28_layers_teacher_forced(ctx):
    """The full synthetic decode workload: 28 layers, hidden 2048, 16/4 heads of 128,
    FFN 6144, tied 151936-token Q8_0 LM head, 1024 cached tokens; 32 greedy steps
    (positions 1024..1055) replayed from the captured graph, each step's logits and token
    against the oracle's decode step fed the GPU's previous token (about 0.5 s of host
    work per step at 16 threads)."""
    from test_gpu_decoder import check_against_oracle

    steps = 32
    model = synth.decoder_model(0, kv_prefill=1024)
    assert model["geometry"]["layers"] == 28
    dec = ph.Decoder(ctx, model, max_steps=steps)
    try:
        toks, logits, _ = dec.generate(1, 1024, steps, graph=True, logits=True)
    finally:
        dec.close()
    identical = check_against_oracle(model, 1024, 1, toks, logits)
    print(f"c3: {identical} of {steps} steps bit-identical to the oracle")
