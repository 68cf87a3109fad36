"""test-backend-ops' MUL_MAT geometries (the reference's conformance set,
tests/upstream_prism/backend-ops-geometries.json) through prism_hip_mul_mat.

The reference runs MUL_MAT for a packed A as one public matvec per column of B
(src/backend/call.rs:808-823, src/backend/ops.rs:444-466) and checks it against a CPU
product with a normalized-error bound; here every output is compared with the oracle's
per-column matvec bit for bit.  The plain 2-D cases of the path's formats are kept (A in
Q8_0, Q2_K, PQ2 or PTQ1, B in F32, no batching, broadcast or permutation): 260 distinct
geometries from 1 to 4096 rows, 1 to 4096 columns of B and widths from 32 to 393216.
"""

import json
import os

import numpy as np
import pytest

import fixtures_util as fx
import synth

THREADS = min(16, os.cpu_count() or 1)


def test_mulmat_fixture_is_the_filtered_reference_file():
    meta = fx.load_json("PROVENANCE.json")["backend-ops-mulmat.json"]
    assert fx.sha256(fx.read("backend-ops-mulmat.json")) == meta["local_sha256"]
    data = fx.load_json("backend-ops-mulmat.json")
    assert len(data["Eval"]) == meta["cases"] == 331
    for e in data["Eval"]:
        a = e["Arguments"]
        assert e["Class"] == "test_mul_mat" and a[0] in (8, 10, 142, 143) and a[1] == 0
        assert a[5] == [1, 1] and a[6] == [1, 1] and a[7] == [0, 1, 2, 3]
    assert len(data["Perf"]) == 125
    for e in data["Perf"]:
        a = e["Arguments"]
        assert e["Class"] == "test_mul_mat" and a[0] in (8, 10, 142, 143) and a[1] == 0
        assert a[5] == [1, 1] and a[6] == [1, 1] and a[7] == [0, 1, 2, 3]
    geoms = fx.mulmat_geometries()
    assert len(geoms) == 260
    block = {8: 32, 10: 256, 142: 128, 143: 128}
    assert all(k % block[t] == 0 for t, m, n, k in geoms)


@pytest.mark.gpu
def test_gpu_mul_mat_backend_ops_geometries():
    import oracle
    import prism_hip as ph

    with ph.Context(0) as ctx:
        for i, (kind, m, n, k) in enumerate(fx.mulmat_geometries()):
            w = synth.weights(kind, m, k, seed=1000 + i)
            B = synth.activations(k, seed=2000 + i, tokens=n).reshape(n, k)
            wid = ctx.weight(kind, k, m, w)
            got = ctx.mul_mat(wid, m, B)
            ref = oracle.prefill(kind, k, m, w, B, False, threads=THREADS).reshape(n, m)
            if not np.array_equal(got.view(np.uint32), ref.view(np.uint32)):
                bad = np.argwhere(got.view(np.uint32) != ref.view(np.uint32))
                j, r = bad[0]
                raise AssertionError(json.dumps({"kind": kind, "m": m, "n": n, "k": k, "mismatches": len(bad),
                                                 "first": [int(j), int(r), float(got[j, r]), float(ref[j, r])]}))
            ctx.release(wid)
        assert not ctx.faulted
