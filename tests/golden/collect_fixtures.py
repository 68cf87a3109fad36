#!/usr/bin/env python3
"""Copy the reference's own fixture DATA for the packed-matvec path into tests/golden/.

Run in a container where the reference checkout is mounted at /root/reference.
Only data is taken (binary captures, JSON records of inputs/expected outputs);
no reference source is copied.  Each output keeps the SHA-256 of the original
file so the provenance chain (native capture -> reference fixture -> here) is
checkable.  JSON fixtures are reduced to the formats on this path.

Sources (paths relative to the reference checkout):
  tools/ternary/tests/fixtures/ptq-reference.bin      native C++ PQ2<->PTQ1 + f16 cases
  tests/fixtures/swift-q8-parity.{bin,json}           pinned Q8_0 rounding captures
  tests/fixtures/swift-q8k-parity.{bin,json}          pinned Q8_K fused-rounding captures
  tests/fixtures/swift-ptq1-q8-scale-parity.{bin,json} PTQ1 native-scale Q8_0 captures
  tests/fixtures/swift-ptq1-dot-parity.{bin,json}     pinned PTQ1 dot bits (+ source bits)
  tests/fixtures/row-quantizers.json                  production row-quantizer records
  tests/fixtures/upstream-kquants.json                K-quant encode/decode/dot records
  tests/upstream_prism/pq2-inputs.bin                 15 upstream PQ2 row-shape inputs
  tests/fixtures/upstream-tquants.json                TQ1_0/TQ2_0 encode/decode/dot records
  tests/fixtures/swift-activation-parity.json         pinned SiLU / SwiGLU native captures
  tests/upstream_prism/backend-ops-geometries.json    MUL_MAT geometries of test-backend-ops
                                                      (plain 2-D cases of the path's formats)
"""

import hashlib
import json
import os
import shutil
import sys

REF = os.environ.get("PRISM_REFERENCE", "/root/reference")
OUT = os.path.dirname(os.path.abspath(__file__))

COPY = [
    "tools/ternary/tests/fixtures/ptq-reference.bin",
    "tests/fixtures/swift-q8-parity.bin",
    "tests/fixtures/swift-q8-parity.json",
    "tests/fixtures/swift-q8k-parity.bin",
    "tests/fixtures/swift-q8k-parity.json",
    "tests/fixtures/swift-ptq1-q8-scale-parity.bin",
    "tests/fixtures/swift-ptq1-q8-scale-parity.json",
    "tests/fixtures/swift-ptq1-dot-parity.bin",
    "tests/fixtures/swift-ptq1-dot-parity.json",
    "tests/upstream_prism/pq2-inputs.bin",
    "tests/fixtures/upstream-tquants.json",
    "tests/fixtures/swift-activation-parity.json",
]


def sha(path: str) -> str:
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def main() -> int:
    if not os.path.isdir(REF):
        print(f"reference checkout not found at {REF}", file=sys.stderr)
        return 1
    provenance = {}
    for rel in COPY:
        src = os.path.join(REF, rel)
        dst = os.path.join(OUT, os.path.basename(rel))
        shutil.copyfile(src, dst)
        provenance[os.path.basename(rel)] = {"source": rel, "sha256": sha(src)}

    # Row quantizers: keep F16 (1), Q8_0 (8), Q8_K (15), PQ2 (142), PTQ1 (143).
    rel = "tests/fixtures/row-quantizers.json"
    src = os.path.join(REF, rel)
    with open(src) as f:
        data = json.load(f)
    keep = [c for c in data["Cases"] if c["TypeId"] in (1, 8, 15, 142, 143)]
    reduced = {k: v for k, v in data.items() if k != "Cases"}
    reduced["Cases"] = keep
    with open(os.path.join(OUT, "row-quantizers-path.json"), "w") as f:
        json.dump(reduced, f, indent=1, sort_keys=True)
    provenance["row-quantizers-path.json"] = {"source": rel, "sha256": sha(src), "type_ids": [1, 8, 15, 142, 143],
                                              "cases": len(keep)}

    # K quants: keep Q2_K (TypeId 10).
    rel = "tests/fixtures/upstream-kquants.json"
    src = os.path.join(REF, rel)
    with open(src) as f:
        data = json.load(f)
    keep = [c for c in data["Cases"] if c["TypeId"] == 10]
    reduced = {k: v for k, v in data.items() if k != "Cases"}
    reduced["Cases"] = keep
    with open(os.path.join(OUT, "upstream-kquants-q2k.json"), "w") as f:
        json.dump(reduced, f, indent=1, sort_keys=True)
    provenance["upstream-kquants-q2k.json"] = {"source": rel, "sha256": sha(src), "type_ids": [10], "cases": len(keep)}

    # MUL_MAT geometries (test_mul_mat arguments: type_a, type_b, m, n, k, bs, nr, per, ...):
    # keep A in Q8_0 (8), Q2_K (10), PQ2 (142) or PTQ1 (143) with an F32 B (type 0) and no
    # batching, broadcast or permutation -- the 2-D product prism_hip_mul_mat serves.
    rel = "tests/upstream_prism/backend-ops-geometries.json"
    src = os.path.join(REF, rel)
    with open(src) as f:
        data = json.load(f)
    def plain(e):
        a = e["Arguments"]
        return (e["Class"] == "test_mul_mat" and a[0] in (8, 10, 142, 143) and a[1] == 0 and a[5] == [1, 1]
                and a[6] == [1, 1] and a[7] == [0, 1, 2, 3])

    keep = [e for e in data["Eval"] if plain(e)]
    reduced = {k: data[k] for k in ("SchemaVersion", "Source", "SourceSha256", "EvalSha256", "PerfSha256")}
    reduced["Eval"] = keep
    reduced["Perf"] = [e for e in data["Perf"] if plain(e)]
    with open(os.path.join(OUT, "backend-ops-mulmat.json"), "w") as f:
        json.dump(reduced, f, indent=1, sort_keys=True)
    provenance["backend-ops-mulmat.json"] = {"source": rel, "sha256": sha(src), "type_ids": [8, 10, 142, 143],
                                             "cases": len(keep)}

    for name in provenance:
        provenance[name]["local_sha256"] = sha(os.path.join(OUT, name))
    with open(os.path.join(OUT, "PROVENANCE.json"), "w") as f:
        json.dump(provenance, f, indent=1, sort_keys=True)
    print(json.dumps({k: v["local_sha256"][:12] for k, v in provenance.items()}, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
