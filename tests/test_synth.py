"""The synthetic generators produce canonical reference byte layouts (checked with the oracle)."""

import numpy as np

import synth


def test_ptq1_packer_matches_canonical_pack_ptq(oracle):
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 3, (200, 128), dtype=np.int8)
    scales = (np.abs(rng.normal(0, 0.02, 200)) + 1e-3).astype(np.float16).view(np.uint8).reshape(-1, 2)
    got = synth.pack_ptq1(codes, scales)
    pq2 = synth.pack_pq2(codes, scales)
    for b in range(200):
        assert oracle.pack_ptq(pq2[b].tobytes()) == got[b].tobytes()
        assert list(oracle.decode_ptq_trits(got[b])) == list(codes[b].astype(int) - 1)


def test_generators_have_reference_extents_and_finite_scales(oracle):
    for kind, (g, bb) in synth.LAYOUT.items():
        w = synth.weights(kind, 8, 512, seed=3)
        assert w.size == 8 * 512 // g * bb
        dec = oracle.decode_row(kind, 8 * 512, w)  # all scales finite
        assert np.isfinite(dec).all()


def test_ternary_codes_are_uniform():
    w = synth.ptq1_weights(64, 2048, seed=0).reshape(-1, 28)
    import oracle as o

    t = np.concatenate([o.decode_ptq_trits(w[i]) for i in range(0, w.shape[0], 7)])
    frac = [(t == v).mean() for v in (-1, 0, 1)]
    assert max(abs(f - 1 / 3) for f in frac) < 0.01
