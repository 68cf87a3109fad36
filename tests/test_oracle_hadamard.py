"""Pin the oracle's blockwise Hadamard rotation (src/kernels.rs:3952-3987) and the FFN
chain that rotates the SwiGLU vector ahead of down (src/kernels/projection.rs:271-290).

Checks: the reference's own fixture (tests/kernels.rs:405-413); Sylvester's matrix
(scipy.linalg.hadamard) on small integers, where every butterfly sum is exact and only
the final binary32 product with fl(1/fl(sqrt(block))) rounds; a hand-derived case whose
rounding depends on the butterfly order; block independence, involution and the error
cases.
"""

import numpy as np
import pytest
import scipy.linalg

import synth

F32 = np.float32


def _norm(block: int) -> np.float32:
    # normalization = 1.0 / integer_float(count).sqrt() in binary32
    return F32(1.0) / np.sqrt(F32(block))


def test_hadamard_reference_fixture(oracle):
    # tests/kernels.rs:405-413
    v = oracle.hadamard([1.0, 2.0, 3.0, 4.0], 4)
    assert v.tolist() == [5.0, -1.0, -2.0, 0.0]
    assert oracle.hadamard(v, 4).tolist() == [1.0, 2.0, 3.0, 4.0]
    with pytest.raises(RuntimeError):
        oracle.hadamard(np.zeros(0, F32), 0)
    with pytest.raises(RuntimeError):
        oracle.hadamard(np.ones(3, F32), 3)


@pytest.mark.parametrize("block", [2, 4, 8, 32, 64, 128, 512, 1024])
def test_hadamard_matches_sylvester_matrix_on_integers(oracle, block):
    rng = np.random.default_rng(block)
    x = rng.integers(-64, 65, size=block).astype(F32)
    exact = scipy.linalg.hadamard(block).astype(np.float64) @ x.astype(np.float64)
    assert np.all(np.abs(exact) < 2**24)  # every butterfly sum is an exact binary32 integer
    want = exact.astype(F32) * _norm(block)
    got = oracle.hadamard(x, block)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_hadamard_butterfly_order_known_answer(oracle):
    # x = [1, e, e, e] with e = 2^-24.  Half 1 first: (1 + e -> 1 by ties-to-even, 1 - e,
    # 2e, 0); half 2: (1 + 2e, 1 - e, 1 - 2e, 1 - e).  The exact transform is
    # (1 + 3e, 1 - e, 1 - e, 1 - e); half 2 first would round into position 1 instead.
    e = 2.0**-24
    got = oracle.hadamard(np.array([1.0, e, e, e], F32), 4)
    want = np.array([(1 + 2 * e) / 2, (1 - e) / 2, (1 - 2 * e) / 2, (1 - e) / 2], F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_hadamard_blocks_are_independent_and_involutive(oracle):
    rng = np.random.default_rng(3)
    x = rng.integers(-100, 101, size=8 * 64).astype(F32)
    whole = oracle.hadamard(x, 64)
    parts = np.concatenate([oracle.hadamard(x[i:i + 64], 64) for i in range(0, x.size, 64)])
    assert np.array_equal(whole.view(np.uint32), parts.view(np.uint32))
    # Block 64 has the exact normalization 1/8: the rotation is its own inverse on integers.
    assert np.array_equal(oracle.hadamard(whole, 64), x)
    y = rng.standard_normal(4096).astype(F32)
    back = oracle.hadamard(oracle.hadamard(y, 256), 256)
    assert np.max(np.abs(back - y)) <= 1e-5 * np.max(np.abs(y))


def test_hadamard_rejects_bad_blocks_and_nonfinite_values(oracle):
    with pytest.raises(RuntimeError):
        oracle.hadamard(np.ones(96, F32), 64)  # block does not divide the vector
    with pytest.raises(RuntimeError):
        oracle.hadamard(np.ones(96, F32), 48)
    with pytest.raises(RuntimeError):
        oracle.hadamard(np.array([1.0, np.nan], F32), 2)
    with pytest.raises(RuntimeError):
        oracle.hadamard(np.array([3e38, 3e38, 0.0, 0.0], F32), 4)  # the sum overflows


@pytest.mark.parametrize("kind", [synth.KIND_PTQ1, synth.KIND_Q2_K])
def test_rotated_ffn_chain_composes_swiglu_rotation_and_down(oracle, kind):
    hidden, ffn = 256, 512
    wg = synth.weights(kind, ffn, hidden, seed=1)
    wu = synth.weights(kind, ffn, hidden, seed=2)
    wd = synth.weights(kind, hidden, ffn, seed=3)
    x = synth.activations(hidden, seed=4)
    r = synth.activations(hidden, seed=5)
    base, h = oracle.ffn(kind, hidden, ffn, wg, wu, wd, x, r, pinned=True)
    for none in (0, 1):
        out, h1 = oracle.ffn(kind, hidden, ffn, wg, wu, wd, x, r, pinned=True, hadamard_block=none)
        assert np.array_equal(out.view(np.uint32), base.view(np.uint32))
    for block in (32, 128, 512):
        out, h2 = oracle.ffn(kind, hidden, ffn, wg, wu, wd, x, r, pinned=True, hadamard_block=block)
        assert np.array_equal(h2.view(np.uint32), h.view(np.uint32))  # h stays unrotated
        down = oracle.matvec(kind, ffn, hidden, wd, oracle.hadamard(h, block), pinned=True)
        want = down + r
        assert np.array_equal(out.view(np.uint32), want.view(np.uint32))
        assert not np.array_equal(out, base)
    with pytest.raises(RuntimeError):
        oracle.ffn(kind, hidden, ffn, wg, wu, wd, x, r, pinned=True, hadamard_block=96)
