"""GPU parity over the dispatch space: seeded random (kind, rows, columns, tokens, contract)
cases through prism_hip_project_f32, each token row against the oracle's per-token matvec
bit for bit.

The library picks among a dozen kernels by kind, contract, matrix size (tiles per CU), row
width and token count: row-tile, two- and N-wavefront, table (whole, split, tail, spread),
split-K, token-by-token, 4x4x4 batch, skinny, weights-once batch, and the f16 / int8 prefill
GEMMs with their token-group choices.  The cases below are drawn so that every one of those
regions is visited (sizes from one partial tile to a few tiles per CU, widths up to 8192
inputs, odd unit counts, PQ2 in both of its activation contracts, 1 to 300 tokens), with the
oracle's work per case bounded.  The seed is fixed, so a failure names a reproducible case.
"""

import os

import numpy as np
import pytest

import prism_hip as ph
import synth

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)

KINDS = [ph.KIND_PTQ1, ph.KIND_PQ2, ph.KIND_Q2_K, ph.KIND_Q8_0, ph.KIND_TQ1_0, ph.KIND_TQ2_0]
ROWS = [37, 200, 1000, 4100, 9000, 16411, 33000, 70000]
COLS = [256, 384, 512, 1152, 1280, 2048, 4096, 8192]
TOKENS = [1, 2, 3, 4, 5, 8, 15, 16, 17, 31, 32, 33, 48, 64, 100, 130, 300]
MAX_WORK = 3e8  # rows * cols * tokens per case


# Wide rows (the reference's MUL_MAT widths among them): the split-K, token-by-token and
# quad-split regions, with more token counts between the batch kernels' thresholds.
COLS_WIDE = [5120, 6144, 12288, 14336, 17408]
TOKENS_WIDE = TOKENS + [6, 7, 9, 12, 20, 40, 65, 96]


def _cases(n: int = 160, seed: int = 20261202, cols_list=COLS, tokens_list=TOKENS):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        kind = KINDS[int(rng.integers(len(KINDS)))]
        rows = ROWS[int(rng.integers(len(ROWS)))]
        cols = cols_list[int(rng.integers(len(cols_list)))]
        tokens = tokens_list[int(rng.integers(len(tokens_list)))]
        if cols % synth.LAYOUT[kind][0] or rows * cols * tokens > MAX_WORK:
            continue
        out.append((kind, rows, cols, tokens, bool(rng.integers(2))))
    return out


@pytest.fixture(scope="module")
def ctx():
    c = ph.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("kind,rows,cols,tokens,pinned",
                         _cases() + _cases(100, 20261203, COLS_WIDE, TOKENS_WIDE))
def test_gpu_dispatch_sweep_matches_oracle(ctx, kind, rows, cols, tokens, pinned):
    import oracle

    w = synth.weights(kind, rows, cols, seed=rows + cols + tokens)
    X = synth.activations(cols, seed=tokens + kind, tokens=tokens).reshape(tokens, cols)
    wid = ctx.weight(kind, cols, rows, w)
    try:
        ref = oracle.prefill(kind, cols, rows, w, X, pinned, threads=THREADS)
        got = ctx.project_f32(wid, rows, X[0] if tokens == 1 else X, tokens=tokens, pinned=pinned)
        g = np.ascontiguousarray(got, np.float32).reshape(-1).view(np.uint32)
        r = np.ascontiguousarray(ref, np.float32).reshape(-1).view(np.uint32)
        if not np.array_equal(g, r):
            bad = np.nonzero(g != r)[0]
            raise AssertionError(f"kind={kind} {rows}x{cols} tokens={tokens} pinned={pinned}: {bad.size} "
                                 f"mismatches, first at token {bad[0] // rows} row {bad[0] % rows}")
        assert not ctx.faulted
    finally:
        ctx.release(wid)
