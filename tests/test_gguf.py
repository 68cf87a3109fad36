"""GGUF v3 tensor index and the PQ2 -> PTQ1 export (include/prism_hip.h, csrc/gguf.cpp).

The index cases restate the reference's tools/gguf/tests/stream_index.rs expectations on
the same synthetic streams (a valid two-tensor file, the seven rejected layouts, the
version-2 / 1 MiB-alignment policy, bad booleans and alignments, zero tensors, interior
NUL and invalid UTF-8 in skipped string arrays).  The export is checked against the
oracle's pack_ptq on every block, verbatim copies of other tensors, the rewritten
descriptors and the receipt's SHA-256.  Host code only: no GPU."""

import hashlib
import struct

import numpy as np
import pytest

import prism_hip as ph
import synth


def _str(b: bytes) -> bytes:
    return struct.pack("<Q", len(b)) + b


def kv_u32(v):
    return struct.pack("<II", 4, v)


def kv_i32(v):
    return struct.pack("<Ii", 5, v)


def kv_bool(v):
    return struct.pack("<IB", 7, v)


def kv_string(s: bytes):
    return struct.pack("<I", 8) + _str(s)


def kv_str_array(items):
    return struct.pack("<IIQ", 9, 8, len(items)) + b"".join(_str(i) for i in items)


def kv_i32_array(items):
    return struct.pack("<IIQ", 9, 5, len(items)) + b"".join(struct.pack("<i", i) for i in items)


def build_gguf(version, alignment, kv, tensors, data_bytes, payloads=None):
    """Same layout as the reference tests' build_gguf; payloads optionally fill tensor bytes."""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv)))
    for k, v in kv:
        out += _str(k) + v
    for name, shape, kind, offset in tensors:
        out += _str(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<IQ", kind, offset)
    if tensors:
        base = (len(out) + alignment - 1) // alignment * alignment
        out += bytes(base - len(out) + data_bytes)
        for (name, shape, kind, offset), data in zip(tensors, payloads or [None] * len(tensors)):
            if data is not None:
                out[base + offset:base + offset + len(data)] = bytes(data)
    return bytes(out)


def write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def asr_policy(**kw):
    # stream_index.rs asr_policy: bounded budget, overheads, no Prism types, an allowlist.
    allowed = np.array([0, 1, 2, 3, 6, 7, 8, 12, 13, 14, 30], np.uint32)
    fields = dict(allow_zero_metadata=0, max_file_bytes=8 << 30, max_tensors=8192, max_metadata=65536,
                  metadata_budget=64 << 20, max_key_bytes=1024, max_string_bytes=65536, max_array_string_bytes=4096,
                  max_retained_string_array_bytes=0, max_array_items=262144, max_alignment=4096,
                  reject_nonfinite_floats=0, reject_interior_nul_strings=0, kv_overhead_bytes=128,
                  string_overhead_bytes=32, tensor_overhead_bytes=512, charge_skipped_scalar_arrays=1)
    fields.update(kw)
    p = ph.GgufPolicy.default(**fields)
    p.allowed_types = allowed.ctypes.data_as(ph.ctypes.POINTER(ph.ctypes.c_uint32))
    p.allowed_type_count = len(allowed)
    p._keep = allowed  # the array must outlive the policy
    return p


def tts_policy(**kw):
    allowed = np.array([0, 1, 8, 12, 14], np.uint32)
    p = ph.GgufPolicy.default(allow_v2=1, allow_positive_i32_alignment=1, **kw)
    p.allowed_types = allowed.ctypes.data_as(ph.ctypes.POINTER(ph.ctypes.c_uint32))
    p.allowed_type_count = len(allowed)
    p._keep = allowed
    return p


def test_index_resolves_layouts_and_skips_scalar_arrays(tmp_path):
    data = build_gguf(3, 32, [(b"unrelated", kv_u32(7)), (b"skipped_i32", kv_i32_array([1, 2, 3, 4]))],
                      [(b"q8", [32, 2], 8, 32), (b"f32", [3], 0, 0)], 100)
    with ph.Gguf(write(tmp_path, "a.gguf", data), asr_policy()) as g:
        t = g.tensors()
        assert t["q8"]["bytes"] == 68 and t["f32"]["bytes"] == 12
        assert t["q8"]["offset"] - t["f32"]["offset"] == 32
        m = g.metadata()
        assert (m["skipped_i32"]["element_type"], m["skipped_i32"]["count"], m["skipped_i32"]["retained"]) == (5, 4, False)
        assert g.int("unrelated") == 7
        s = g.summary()
        assert s["version"] == 3 and s["alignment"] == 32 and s["data_offset"] % 32 == 0
        assert list(t) == sorted(t)  # name order


def test_index_charges_empty_string_arrays_against_the_budget(tmp_path):
    data = build_gguf(3, 32, [(b"t", kv_str_array([b"", b""]))], [(b"w", [1], 0, 0)], 4)
    with pytest.raises(ph.GgufError):
        ph.Gguf(write(tmp_path, "b.gguf", data), asr_policy(metadata_budget=63, allow_zero_metadata=1))


@pytest.mark.parametrize("what,data", [
    ("overlapping", build_gguf(3, 32, [(b"k", kv_u32(1))], [(b"a", [2], 0, 0), (b"b", [32], 8, 0)], 100)),
    ("unaligned", build_gguf(3, 32, [(b"k", kv_u32(1))], [(b"b", [32], 8, 1)], 100)),
    ("truncated", build_gguf(3, 32, [(b"k", kv_u32(1))], [(b"b", [32], 8, 32)], 65)),
    ("fractional", build_gguf(3, 32, [(b"k", kv_u32(1))], [(b"b", [31], 8, 32)], 100)),
    ("prism type outside the dialect", build_gguf(3, 32, [(b"k", kv_u32(1))], [(b"b", [128], 142, 0)], 100)),
    ("duplicate key", build_gguf(3, 32, [(b"k", kv_u32(1)), (b"k", kv_u32(2))], [(b"w", [1], 0, 0)], 4)),
    ("nested array", build_gguf(3, 32, [(b"nested", struct.pack("<IIQ", 9, 9, 0))], [(b"w", [1], 0, 0)], 4)),
])
def test_index_rejects_bad_layouts(tmp_path, what, data):
    with pytest.raises(ph.GgufError):
        ph.Gguf(write(tmp_path, "c.gguf", data), asr_policy())


def test_index_version2_large_alignment_and_string_arrays(tmp_path):
    data = build_gguf(2, 1 << 20, [(b"general.alignment", kv_i32(1 << 20)),
                                   (b"tokenizer.ggml.tokens", kv_str_array([b"alpha", b"beta"])),
                                   (b"codec.rates", kv_i32_array([8, 5, 4, 3])), (b"flag", kv_bool(1))],
                      [(b"w", [1], 0, 0)], 4)
    path = write(tmp_path, "d.gguf", data)
    with ph.Gguf(path, tts_policy()) as g:
        s = g.summary()
        assert s["version"] == 2 and s["alignment"] == 1 << 20
        assert [g.string("tokenizer.ggml.tokens", i) for i in range(2)] == ["alpha", "beta"]
        m = g.metadata()
        assert (m["codec.rates"]["element_type"], m["codec.rates"]["count"]) == (5, 4)
        assert g.int("flag") == 1
    with pytest.raises(ph.GgufError):  # version 2 and I32 alignment are policy opt-ins
        ph.Gguf(path)


@pytest.mark.parametrize("bad_item", [b"bad\0nul", b"\xfe\xff"])
def test_index_rejects_nul_and_invalid_utf8_in_skipped_string_arrays(tmp_path, bad_item):
    data = build_gguf(3, 32, [(b"other.strings", kv_str_array([bad_item]))], [(b"w", [1], 0, 0)], 4)
    with pytest.raises(ph.GgufError):
        ph.Gguf(write(tmp_path, "e.gguf", data), tts_policy(retain_string_arrays=0))


@pytest.mark.parametrize("what,kv", [
    ("scalar bool 2", [(b"flag", kv_bool(2))]),
    ("bool array with 255", [(b"flags", struct.pack("<IIQ", 9, 7, 2) + bytes([0, 255]))]),
    ("negative alignment", [(b"general.alignment", kv_i32(-32))]),
    ("alignment 3", [(b"general.alignment", kv_u32(3))]),
    ("alignment over the cap", [(b"general.alignment", kv_u32(2 << 20))]),
])
def test_index_rejects_bad_booleans_and_alignments(tmp_path, what, kv):
    data = build_gguf(3, 32, kv, [(b"w", [1], 0, 0)], 4)
    with pytest.raises(ph.GgufError):
        ph.Gguf(write(tmp_path, "f.gguf", data), tts_policy())


def test_index_zero_tensors_only_with_the_opt_in(tmp_path):
    data = build_gguf(3, 32, [], [], 0)
    assert len(data) == 24
    path = write(tmp_path, "z.gguf", data)
    with pytest.raises(ph.GgufError):
        ph.Gguf(path, tts_policy())
    with ph.Gguf(path, tts_policy(allow_zero_tensors=1)) as g:
        assert g.tensors() == {} and g.summary()["data_offset"] == 24


def _prism_file(tmp_path, name, file_type=141, levels=3, seed=3):
    """A Prism-dialect model: two PQ2 matrices around an F32 norm vector (GGML order dims)."""
    a = synth.pq2_weights(4, 256, seed, levels)          # 4 rows x 256
    b = synth.pq2_weights(3, 384, seed + 1, levels)      # 3 rows x 384
    norm = np.arange(5, dtype=np.float32) * 0.25
    sizes = [a.size, norm.nbytes, b.size]
    offs, off = [], 0
    for n in sizes:
        offs.append(off)
        off = (off + n + 31) // 32 * 32
    data = build_gguf(3, 32, [(b"general.architecture", kv_string(b"synthetic")),
                              (b"general.file_type", kv_u32(file_type))],
                      [(b"blk.0.ffn_up.weight", [256, 4], 142, offs[0]), (b"blk.0.norm", [5], 0, offs[1]),
                       (b"blk.0.ffn_down.weight", [384, 3], 142, offs[2])], off,
                      payloads=[a, norm.view(np.uint8), b])
    return write(tmp_path, name, data), {"blk.0.ffn_up.weight": a, "blk.0.norm": norm.view(np.uint8),
                                         "blk.0.ffn_down.weight": b}


def test_prism_dialect_reads_tensor_payloads(tmp_path):
    path, payloads = _prism_file(tmp_path, "p.gguf")
    with pytest.raises(ph.GgufError):
        ph.Gguf(path)  # PQ2 needs the dialect
    with ph.Gguf(path, ph.GgufPolicy.default(prism_dialect=1)) as g:
        assert g.string("general.architecture") == "synthetic" and g.int("general.file_type") == 141
        for name, data in payloads.items():
            assert np.array_equal(g.read(name), data), name
        t = g.tensors()["blk.0.ffn_down.weight"]
        assert t["type_id"] == 142 and t["dims"] == [384, 3] and t["bytes"] == 3 * 3 * 34


def test_export_repacks_pq2_losslessly(tmp_path):
    import oracle

    src, payloads = _prism_file(tmp_path, "src.gguf")
    dst = str(tmp_path / "dst.gguf")
    receipt = ph.gguf_export_ptq1(src, dst)
    out = open(dst, "rb").read()
    assert receipt["OutputSha256"] == hashlib.sha256(out).hexdigest()
    assert receipt["OutputBytes"] == len(out) and receipt["ConvertedTensorCount"] == 2
    assert receipt["ConvertedBlocks"] == 4 * 2 + 3 * 3
    with ph.Gguf(dst, ph.GgufPolicy.default(prism_dialect=1)) as g:
        assert g.int("general.file_type") == 143
        t = g.tensors()
        assert t["blk.0.norm"]["type_id"] == 0
        assert np.array_equal(g.read("blk.0.norm"), payloads["blk.0.norm"])
        for name in ("blk.0.ffn_up.weight", "blk.0.ffn_down.weight"):
            assert t[name]["type_id"] == 143
            got = g.read(name)
            pq2 = payloads[name]
            want = b"".join(oracle.pack_ptq(pq2[34 * k:34 * (k + 1)]) for k in range(pq2.size // 34))
            assert got.tobytes() == want, name
            assert b"".join(oracle.unpack_ptq(got[28 * k:28 * (k + 1)]) for k in range(got.size // 28)) == pq2.tobytes()
        assert len(out) % 32 == 0
    with pytest.raises(ph.GgufError):  # never overwrites
        ph.gguf_export_ptq1(src, dst)


@pytest.mark.parametrize("what", ["code 3", "no file type", "signed file type"])
def test_export_rejects(tmp_path, what):
    if what == "code 3":
        src, _ = _prism_file(tmp_path, "s.gguf", levels=4, seed=11)  # 4-level codes include 3 (+2)
    elif what == "no file type":
        data = build_gguf(3, 32, [(b"general.architecture", kv_string(b"x"))],
                          [(b"w", [128], 142, 0)], 64, payloads=[synth.pq2_weights(1, 128, 1, 3)])
        src = write(tmp_path, "s.gguf", data)
    else:
        data = build_gguf(3, 32, [(b"general.file_type", kv_i32(141))],
                          [(b"w", [128], 142, 0)], 64, payloads=[synth.pq2_weights(1, 128, 1, 3)])
        src = write(tmp_path, "s.gguf", data)
    with pytest.raises(ph.GgufError):
        ph.gguf_export_ptq1(src, str(tmp_path / "o.gguf"))


@pytest.mark.gpu
def test_gpu_weight_from_gguf_matches_oracle(tmp_path):
    """A PTQ1 tensor uploaded from an exported file runs the same matvec as the oracle."""
    import oracle

    src, _ = _prism_file(tmp_path, "src.gguf")
    dst = str(tmp_path / "dst.gguf")
    ph.gguf_export_ptq1(src, dst)
    ctx = ph.Context(0)
    try:
        with ph.Gguf(dst, ph.GgufPolicy.default(prism_dialect=1)) as g:
            wid = ctx.weight_from_gguf(g, "blk.0.ffn_down.weight", key=77)
            w = g.read("blk.0.ffn_down.weight")
            x = synth.activations(384, seed=5)
            ref = oracle.matvec(ph.KIND_PTQ1, 384, 3, w, x, False)
            got = ctx.project_f32(wid, 3, x)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
            assert ctx.weight_from_gguf(g, "blk.0.ffn_down.weight", key=77) == wid  # residency by key
    finally:
        ctx.close()
