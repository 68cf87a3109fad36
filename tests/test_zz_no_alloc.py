"""prism_hip_project_device_noalloc against prism_hip_project_device, bit for bit.

The no-allocation entry point carves every scratch buffer from the fixed per-GPU array
instead of the context's grow-only buffers.  Each case runs two calls in a row, the
second with a smaller input (fewer tokens), covering each scratch user: the quantized
activation of a row-tile matvec, the skinny batch's lane-ordered activation copy, and
the prefill GEMM's token codes; plus prepared-block inputs and the oversize rejection.
"""

import numpy as np
import pytest

import prism_hip as ph
import synth
from hiprt import DeviceBuffer

pytestmark = pytest.mark.gpu

# (kind, rows, cols, tokens of the first call, tokens of the second): f32 inputs.
CASES = [
    (ph.KIND_PTQ1, 6144, 2048, 64, 20),     # prefill GEMM: token codes in scratch
    (ph.KIND_Q8_0, 20480, 512, 9, 5),       # skinny batch, lane-ordered copy in scratch
    (ph.KIND_Q2_K, 40960, 512, 17, 3),      # the same for Q2_K (from 32768 rows), two 16-token chunks
    (ph.KIND_Q8_0, 16384 + 37, 1024, 1, 1),  # row-tile matvec: quantized activation in scratch
    (ph.KIND_PTQ1, 16384 + 37, 512, 3, 2),  # PTQ1 table batch (prepared in scratch)
    (ph.KIND_PQ2, 200, 2048, 2, 1),         # small matrix, quantizing prologue (no scratch)
]


def _run(ctx, fn, wid, path, x, tokens, rows, pinned):
    out = DeviceBuffer(rows * tokens * 4)
    fn(wid, path, x, tokens, pinned, out, ctx.stream())
    assert ctx.sync() == 0
    return out.to_numpy(np.float32)


@pytest.mark.parametrize("kind,rows,cols,t1,t2", CASES)
def test_gpu_noalloc_equals_project_device(kind, rows, cols, t1, t2):
    with ph.Context(0) as ctx:
        w = synth.weights(kind, rows, cols, seed=rows + cols)
        wid = ctx.weight(kind, cols, rows, w)
        for pinned in (False, True):
            for tokens in (t1, t2):
                X = synth.activations(cols, seed=tokens + 31 * pinned, tokens=tokens)
                x = DeviceBuffer.from_numpy(np.ascontiguousarray(X, np.float32))
                ref = _run(ctx, ctx.project_device, wid, ph.PATH_F32, x, tokens, rows, pinned)
                got = _run(ctx, ctx.project_device_noalloc, wid, ph.PATH_F32, x, tokens, rows, pinned)
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (kind, rows, tokens, pinned)
        ctx.release(wid)


def test_gpu_noalloc_prepared_blocks_and_second_smaller_call():
    import oracle

    rows, cols = 20480, 1024
    with ph.Context(0) as ctx:
        w = synth.ptq1_weights(rows, cols, seed=5)
        wid = ctx.weight(ph.KIND_PTQ1, cols, rows, w)
        for tokens in (16, 6):
            X = synth.activations(cols, seed=tokens, tokens=tokens)
            act = np.concatenate([oracle.quantize_q8_0(X[t], 0) for t in range(tokens)])
            a = DeviceBuffer.from_numpy(act.view(np.uint8))
            ref = _run(ctx, ctx.project_device, wid, ph.PATH_Q8, a, tokens, rows, False)
            got = _run(ctx, ctx.project_device_noalloc, wid, ph.PATH_Q8, a, tokens, rows, False)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), tokens
        ctx.release(wid)


def test_gpu_noalloc_rejects_calls_beyond_the_static_scratch():
    """A 4096-token prefill of 4096 inputs needs 32 MiB of token codes, twice the static
    scratch: the call fails before launching anything, and the context stays usable."""
    rows, cols, tokens = 256, 4096, 4096
    with ph.Context(0) as ctx:
        wid = ctx.weight(ph.KIND_PTQ1, cols, rows, synth.ptq1_weights(rows, cols, seed=1))
        x = DeviceBuffer(tokens * cols * 4)
        out = DeviceBuffer(tokens * rows * 4)
        rc = ctx.project_device_noalloc(wid, ph.PATH_F32, x, tokens, False, out, check=False)
        assert rc == ph.ERR_UNSUPPORTED
        assert "static scratch" in ctx.last_error
        assert not ctx.faulted
        small = DeviceBuffer.from_numpy(synth.activations(cols, seed=2))
        ctx.project_device_noalloc(wid, ph.PATH_F32, small, 1, False, out)
        assert ctx.sync() == 0
        ctx.release(wid)
