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
