"""Parsers for the golden fixtures in tests/golden (data copied from the reference's tests)."""

import hashlib
import json
import os
import struct

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def path(name: str) -> str:
    return os.path.join(GOLDEN, name)


def read(name: str) -> bytes:
    with open(path(name), "rb") as f:
        return f.read()


def load_json(name: str):
    with open(path(name)) as f:
        return json.load(f)


def sha256(data: bytes) -> str:
    return hashlib.sha256(data).hexdigest()


def ptq_reference():
    """tools/ternary/tests/fixtures/ptq-reference.bin (layout in its README.md:17-24)."""
    data = read("ptq-reference.bin")
    assert data[:8] == b"PTPAR001"
    cur = 8
    (nh,) = struct.unpack_from("<I", data, cur)
    cur += 4
    halves = []
    for _ in range(nh):
        h, f = struct.unpack_from("<HI", data, cur)
        cur += 6
        halves.append((h, f))
    (nc,) = struct.unpack_from("<I", data, cur)
    cur += 4
    cases = []
    for _ in range(nc):
        rows, blocks = struct.unpack_from("<II", data, cur)
        cur += 8
        n = rows * blocks
        pq2 = [data[cur + 34 * i: cur + 34 * (i + 1)] for i in range(n)]
        cur += 34 * n
        ptq = [data[cur + 28 * i: cur + 28 * (i + 1)] for i in range(n)]
        cur += 28 * n
        cases.append((rows, blocks, pq2, ptq))
    assert cur == len(data)
    return halves, cases


def pq2_inputs():
    """tests/upstream_prism/pq2-inputs.bin (format in tests/upstream_prism/INPUTS.md)."""
    data = read("pq2-inputs.bin")
    assert data[:8] == b"BSPQ2I1\n"
    cur = 8
    (count,) = struct.unpack_from("<I", data, cur)
    cur += 4
    shapes = []
    for _ in range(count):
        k, m, n, nbytes = struct.unpack_from("<IIII", data, cur)
        cur += 16
        packed = data[cur: cur + nbytes]
        cur += nbytes
        act = np.frombuffer(data, dtype="<f4", count=k * n, offset=cur).copy()
        cur += 4 * k * n
        shapes.append((k, m, n, packed, act))
    assert cur == len(data)
    return shapes


def f32_from_hex_words(words):
    return np.array([int(w, 16) if isinstance(w, str) else int(w) for w in words], dtype=np.uint32).view(np.float32)


def hexbytes(s: str) -> bytes:
    return bytes.fromhex(s)


def pq2_block(scale: int, symbols) -> bytes:
    """tests/kernels.rs:27-36: all symbols 1 (weight 0) except the listed (index, symbol)."""
    b = bytearray([0x55] * 34)
    b[0:2] = struct.pack("<H", scale)
    for idx, sym in symbols:
        shift = 2 * (idx % 4)
        b[2 + idx // 4] &= ~(3 << shift) & 0xFF
        b[2 + idx // 4] |= sym << shift
    return bytes(b)


Q8_DTYPE = np.dtype([("scale", "<f4"), ("sum", "<f4"), ("values", "i1", (32,))])


def q8_0_order_kats():
    """Known answers for the Q8_0 x Q8_0 row chain out = fl(out + fl(fl(d_w*d_a)*s))
    (src/kernels.rs:1204-1248), derived by hand from binary32 round-to-nearest-even:

    A  two blocks, terms 2^-10 and fl((1+2^-10)*16385) = 16401 (16401 + 2^-10 is a tie,
       kept even); 2^-10 + 16401 ties again -> 16401.  A fused last step would give
       fl(2^-10 + 16401.0009765625) = 16401.001953125.
    B  terms 2^24, 1, 1 in block order: (2^24 + 1) ties to 2^24, then 2^24 again.  The
       reverse order (or a tree) gives 2^24 + 2.
    C  one block, d_w = 1 - 2^-11, d_a = 2 - 2^-10, s = 8197: d_w*d_a is exact
       (2 - 2^-9 + 2^-21), times 8197 = 16377.99414300918... -> 16377.994140625.
       Scaling s by d_a first gives 16385.99609375 (a tie), then 16377.9951171875.

    Returns (name, weight row bytes, activation blocks, expected bits, wrong bits)."""
    def wblock(d_bits, codes):
        c = np.zeros(32, np.int8)
        c[:len(codes)] = codes
        return int(d_bits).to_bytes(2, "little") + c.tobytes()

    def act(scale, codes):
        a = np.zeros(1, Q8_DTYPE)
        a["scale"] = np.float32(scale)
        a["values"][0, :len(codes)] = codes
        return a

    cases = []
    w = wblock(0x1400, [1]) + wblock(0x3C01, [127, 16])
    a = np.concatenate([act(1.0, [1]), act(1.0, [127, 16])])
    cases.append(("A unfused step", w, a, 0x46802200, 0x46802201))
    w = wblock(0x6400, [64, 64, 64, 64]) + wblock(0x3C00, [1]) + wblock(0x3C00, [1])
    a = np.concatenate([act(1.0, [64, 64, 64, 64]), act(1.0, [1]), act(1.0, [1])])
    cases.append(("B block order", w, a, 0x4B800000, 0x4B800001))
    w = wblock(0x3BFF, [127, 23])
    a = act(np.float16(2 - 2 ** -10), [64, 3])
    cases.append(("C scale product first", w, a, 0x467FE7FA, 0x467FE7FB))
    return cases


def mulmat_geometries():
    """The plain 2-D test_mul_mat cases of test-backend-ops for the path's formats
    (tests/upstream_prism/backend-ops-geometries.json, filtered by collect_fixtures.py):
    distinct (type, m, n, k), m rows of A, n columns of B, k the shared width."""
    data = load_json("backend-ops-mulmat.json")
    return sorted({(a[0], a[2], a[3], a[4]) for a in (e["Arguments"] for e in data["Eval"])})


def mulmat_perf_geometries():
    """test-backend-ops' MUL_MAT performance cases for the path's formats (the same filter),
    distinct (type, m, n, k) in file order."""
    out = []
    for e in load_json("backend-ops-mulmat.json")["Perf"]:
        a = e["Arguments"]
        g = (a[0], a[2], a[3], a[4])
        if g not in out:
            out.append(g)
    return out
