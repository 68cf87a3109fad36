"""ctypes binding of libprism_hip.so (include/prism_hip.h).

The library is the product; this module only marshals numpy arrays and torch
device tensors across its C ABI.  Importing it never falls back to anything: if
the shared library is missing or fails to load, every entry point raises.
"""

from __future__ import annotations

import ctypes
import itertools
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libprism_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "prism_hip.h")

KIND_Q8_0 = 8
KIND_Q2_K = 10
KIND_TQ1_0 = 34
KIND_TQ2_0 = 35
KIND_PQ2 = 142
KIND_PTQ1 = 143
LAYOUT = {KIND_Q8_0: (32, 34), KIND_Q2_K: (256, 84), KIND_PQ2: (128, 34), KIND_PTQ1: (128, 28),
          KIND_TQ1_0: (256, 54), KIND_TQ2_0: (256, 66)}

OK = 0
ERR_INVALID_INPUT = -1
ERR_RESOURCE = -2
ERR_NONFINITE = -3
ERR_DEVICE_FAULT = -4
ERR_UNSUPPORTED = -5
ERR_CANCELLED = -6

PATH_Q8K = 0
PATH_Q8 = 1
PATH_F32 = 2

Q8_SOURCE = 0
Q8_PINNED = 1
Q8_PINNED_NATIVE = 2

Q8K_DTYPE = np.dtype([("scale", "<f4"), ("values", "i1", (256,)), ("sums", "<i2", (16,))])
Q8_DTYPE = np.dtype([("scale", "<f4"), ("sum", "<f4"), ("values", "i1", (32,))])


class PrismError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"prism_hip error {code}: {message}")
        self.code = code


def header_symbols() -> list[str]:
    """Every prism_hip_* function declared in include/prism_hip.h."""
    with open(HEADER) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(prism_hip_[a-z0-9_]+)\s*\(", text)))


_lib = None
# Keys for weights registered without an explicit tensor identity: never reused.
_fresh_keys = itertools.count(1 << 62)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with prism-inference_amd/build.py")
    L = ctypes.CDLL(LIB_PATH)
    P, U64, U32, I, I64 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_int64
    sig = {
        "prism_hip_create": (P, [I, U64, U32]),
        "prism_hip_destroy": (None, [P]),
        "prism_hip_identity": (ctypes.c_char_p, [P]),
        "prism_hip_last_error": (ctypes.c_char_p, [P]),
        "prism_hip_faulted": (I, [P]),
        "prism_hip_inject_fault": (I, [P]),
        "prism_hip_operation_capacity": (U64, [P]),
        "prism_hip_operation_count": (I64, [P, U32, U64, U64]),
        "prism_hip_supports": (I, [P, U32, U64, U64, I]),
        "prism_hip_supports_f32_group": (I, [P, P, U32]),
        "prism_hip_supports_f32_ffn_swiglu": (I, [P, P, P]),
        "prism_hip_supports_f32_ffn_chain": (I, [P, P]),
        "prism_hip_supports_f32_ffn_chain_lora": (I, [P, P]),
        "prism_hip_get_statistics": (I, [P, P]),
        "prism_hip_set_cancellation": (I, [P, P]),
        "prism_hip_get_diagnostics": (I, [P, P]),
        "prism_hip_supports_tile_tokens": (I, [P]),
        "prism_hip_weight_tiled_bytes": (U64, [P, U32, U64, U64]),
        "prism_hip_weight_repack_tiled": (I, [P, U32, U64, U64, P, U64, P, U64]),
        "prism_hip_weight_wrap_tiled": (I64, [P, U32, U64, U64, P, U64]),
        "prism_hip_weight_acquire": (I64, [P, U64, U32, U64, U64, P, U64]),
        "prism_hip_weight_acquire_device": (I64, [P, U64, U32, U64, U64, P, U64]),
        "prism_hip_weight_wrap_device": (I64, [P, U32, U64, U64, P, U64]),
        "prism_hip_weight_release": (I, [P, I64]),
        "prism_hip_weight_release_all": (I, [P]),
        "prism_hip_resident_bytes": (U64, [P]),
        "prism_hip_project_q8k": (I, [P, I64, P, U64, U32, I, P]),
        "prism_hip_project_q8": (I, [P, I64, P, U64, U32, I, P]),
        "prism_hip_project_f32": (I, [P, I64, P, U32, I, P]),
        "prism_hip_project_f32_group": (I, [P, P, U32, P, I, P]),
        "prism_hip_project_f32_group_tokens": (I, [P, P, U32, P, U32, I, P]),
        "prism_hip_project_f32_pair_tokens": (I, [P, P, P, U32, I, P, P]),
        "prism_hip_project_f32_triple_tokens": (I, [P, P, P, U32, I, P, P, P]),
        "prism_hip_ffn_swiglu": (I, [P, I64, I64, P, I, P]),
        "prism_hip_ffn_chain": (I, [P, I64, I64, I64, P, P, U32, I, P]),
        "prism_hip_ffn_chain_lora": (I, [P, I64, I64, I64, P, P, U32, P, I, P, P]),
        "prism_hip_ffn_swiglu_tokens": (I, [P, I64, I64, P, U32, I, P]),
        "prism_hip_ffn_chain_tokens": (I, [P, I64, I64, I64, P, P, U32, U32, I, P]),
        "prism_hip_prefill": (I, [P, I64, P, U32, I, P]),
        "prism_hip_mul_mat": (I, [P, I64, P, U32, P]),
        "prism_hip_quantize_q8k_device": (I, [P, P, U64, U32, I, P, P]),
        "prism_hip_quantize_q8_device": (I, [P, P, U64, U32, I, P, P]),
        "prism_hip_project_device": (I, [P, I64, I, P, U32, I, P, P]),
        "prism_hip_project_device_noalloc": (I, [P, I64, I, P, U32, I, P, P]),
        "prism_hip_ffn_chain_device": (I, [P, I64, I64, I64, P, P, U32, I, P, P, P]),
        "prism_hip_sync": (I, [P, P]),
        "prism_hip_stream": (P, [P]),
        "prism_hip_decoder_create": (P, [P, P, U32]),
        "prism_hip_decoder_destroy": (None, [P]),
        "prism_hip_decoder_set_layer": (I, [P, U32, P, P, P, P, P, P, P, P, P]),
        "prism_hip_decoder_set_cache": (I, [P, U32, P, P, U64]),
        "prism_hip_decoder_set_head": (I, [P, P, P]),
        "prism_hip_decoder_generate": (I, [P, U32, U64, U32, I, P, P, P]),
        "prism_hip_decoder_profile": (I, [P, U32, U64, U32, P]),
        "prism_hip_decoder_time_family": (I, [P, ctypes.c_char_p, U32, P, P]),
        "prism_gguf_default_policy": (None, [P]),
        "prism_gguf_open": (I, [ctypes.c_char_p, P, P]),
        "prism_gguf_close": (None, [P]),
        "prism_gguf_last_error": (ctypes.c_char_p, []),
        "prism_gguf_summary": (I, [P, P, P, P, P, P, P]),
        "prism_gguf_tensor_at": (I, [P, U64, P, P]),
        "prism_gguf_find_tensor": (I, [P, ctypes.c_char_p, P]),
        "prism_gguf_metadata_at": (I, [P, U64, P, P, P, P, P]),
        "prism_gguf_metadata_int": (I, [P, ctypes.c_char_p, P]),
        "prism_gguf_metadata_float": (I, [P, ctypes.c_char_p, P]),
        "prism_gguf_metadata_string": (I, [P, ctypes.c_char_p, U64, P, P]),
        "prism_gguf_read_tensor": (I, [P, ctypes.c_char_p, P, U64]),
        "prism_hip_weight_from_gguf": (I64, [P, P, ctypes.c_char_p, U64]),
        "prism_gguf_export_ptq1": (I, [ctypes.c_char_p, ctypes.c_char_p, P, ctypes.c_size_t]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


class Statistics(ctypes.Structure):
    """prism_hip_statistics (include/prism_hip.h): MatvecStatistics, src/kernels.rs:1792-1830."""
    _fields_ = [(n, ctypes.c_uint64) for n in ("preparations", "preparation_failures", "matrix_attempts",
                                               "matrix_successes", "rejected_before_dispatch", "device_operations",
                                               "grouped_dispatches")]

    def as_dict(self) -> dict:
        return {n: getattr(self, n) for n, _ in self._fields_}


class Diagnostics(ctypes.Structure):
    """prism_hip_diagnostics (include/prism_hip.h): MatvecDiagnostics, src/kernels.rs:1725-1750."""
    _fields_ = [("dispatched", ctypes.c_int32), ("succeeded", ctypes.c_int32)]


class GgufPolicy(ctypes.Structure):
    """prism_gguf_policy (include/prism_hip.h): IndexPolicy, tools/gguf/src/stream.rs:44-131."""
    _fields_ = [("allow_v2", ctypes.c_int), ("allow_zero_tensors", ctypes.c_int), ("allow_zero_metadata", ctypes.c_int),
                ("max_file_bytes", ctypes.c_uint64), ("max_tensors", ctypes.c_uint64),
                ("max_metadata", ctypes.c_uint64), ("metadata_budget", ctypes.c_uint64),
                ("max_key_bytes", ctypes.c_uint64), ("max_string_bytes", ctypes.c_uint64),
                ("max_array_string_bytes", ctypes.c_uint64), ("max_retained_string_array_bytes", ctypes.c_uint64),
                ("max_array_items", ctypes.c_uint64), ("max_alignment", ctypes.c_uint64),
                ("allow_positive_i32_alignment", ctypes.c_int), ("reject_nonfinite_floats", ctypes.c_int),
                ("reject_interior_nul_keys", ctypes.c_int), ("reject_interior_nul_strings", ctypes.c_int),
                ("kv_overhead_bytes", ctypes.c_uint64), ("string_overhead_bytes", ctypes.c_uint64),
                ("tensor_overhead_bytes", ctypes.c_uint64), ("charge_skipped_scalar_arrays", ctypes.c_int),
                ("prism_dialect", ctypes.c_int), ("retain_string_arrays", ctypes.c_int),
                ("allowed_types", ctypes.POINTER(ctypes.c_uint32)), ("allowed_type_count", ctypes.c_size_t)]

    @classmethod
    def default(cls, **overrides):
        p = cls()
        lib().prism_gguf_default_policy(ctypes.byref(p))
        for k, v in overrides.items():
            setattr(p, k, v)
        return p


class GgufTensor(ctypes.Structure):
    _fields_ = [("type_id", ctypes.c_uint32), ("ndims", ctypes.c_uint32), ("dims", ctypes.c_uint64 * 4),
                ("relative_offset", ctypes.c_uint64), ("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64),
                ("elements", ctypes.c_uint64)]


class GgufError(RuntimeError):
    pass


class Gguf:
    """A validated GGUF index (prism_gguf_open); tensors and metadata in name order."""

    def __init__(self, path: str, policy: GgufPolicy | None = None):
        self._h = None
        h = ctypes.c_void_p()
        rc = lib().prism_gguf_open(str(path).encode(), ctypes.byref(policy) if policy is not None else None,
                                   ctypes.byref(h))
        if rc:
            raise GgufError(lib().prism_gguf_last_error().decode())
        self._h = h

    def close(self):
        if self._h:
            lib().prism_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()

    def summary(self) -> dict:
        v = ctypes.c_uint32()
        a, d, t, m, b = (ctypes.c_uint64() for _ in range(5))
        lib().prism_gguf_summary(self._h, *(ctypes.byref(x) for x in (v, a, d, t, m, b)))
        return {"version": v.value, "alignment": a.value, "data_offset": d.value, "tensors": t.value,
                "metadata": m.value, "remaining_budget": b.value}

    @staticmethod
    def _info(t: GgufTensor) -> dict:
        return {"type_id": t.type_id, "dims": list(t.dims)[:t.ndims], "relative_offset": t.relative_offset,
                "offset": t.offset, "bytes": t.bytes, "elements": t.elements}

    def tensors(self) -> dict:
        out = {}
        for i in range(self.summary()["tensors"]):
            name = ctypes.c_char_p()
            t = GgufTensor()
            lib().prism_gguf_tensor_at(self._h, i, ctypes.byref(name), ctypes.byref(t))
            out[name.value.decode()] = self._info(t)
        return out

    def metadata(self) -> dict:
        out = {}
        for i in range(self.summary()["metadata"]):
            key = ctypes.c_char_p()
            ty, el = ctypes.c_uint32(), ctypes.c_uint32()
            cnt, ret = ctypes.c_uint64(), ctypes.c_int()
            lib().prism_gguf_metadata_at(self._h, i, ctypes.byref(key), ctypes.byref(ty), ctypes.byref(el),
                                         ctypes.byref(cnt), ctypes.byref(ret))
            out[key.value.decode()] = {"type": ty.value, "element_type": el.value, "count": cnt.value,
                                       "retained": bool(ret.value)}
        return out

    def int(self, key: str) -> int:
        v = ctypes.c_int64()
        if lib().prism_gguf_metadata_int(self._h, key.encode(), ctypes.byref(v)):
            raise KeyError(key)
        return v.value

    def float(self, key: str) -> float:
        v = ctypes.c_double()
        if lib().prism_gguf_metadata_float(self._h, key.encode(), ctypes.byref(v)):
            raise KeyError(key)
        return v.value

    def string(self, key: str, element: int = 0) -> str:
        p, n = ctypes.c_char_p(), ctypes.c_uint64()
        if lib().prism_gguf_metadata_string(self._h, key.encode(), element, ctypes.byref(p), ctypes.byref(n)):
            raise KeyError(key)
        return ctypes.string_at(p, n.value).decode()

    def read(self, name: str) -> np.ndarray:
        t = GgufTensor()
        if lib().prism_gguf_find_tensor(self._h, name.encode(), ctypes.byref(t)):
            raise KeyError(name)
        out = np.empty(t.bytes, np.uint8)
        if lib().prism_gguf_read_tensor(self._h, name.encode(), _ptr(out), t.bytes):
            raise GgufError(lib().prism_gguf_last_error().decode())
        return out


def gguf_export_ptq1(src: str, dst: str) -> dict:
    """Lossless PQ2 -> PTQ1 export into a new file; returns the receipt."""
    import json

    buf = ctypes.create_string_buffer(1024)
    if lib().prism_gguf_export_ptq1(str(src).encode(), str(dst).encode(), buf, len(buf)):
        raise GgufError(lib().prism_gguf_last_error().decode())
    return json.loads(buf.value.decode())


class TensorDesc(ctypes.Structure):
    """prism_tensor_desc: a tensor's kind and dimensions [cols, rows]."""
    _fields_ = [("kind", ctypes.c_uint32), ("cols", ctypes.c_uint64), ("rows", ctypes.c_uint64)]


def _descs(tensors):
    arr = (TensorDesc * len(tensors))()
    for i, (kind, cols, rows) in enumerate(tensors):
        arr[i] = TensorDesc(kind, cols, rows)
    return arr


def _ptr(a):
    if a is None:
        return None
    if hasattr(a, "data_ptr"):  # torch tensor
        return ctypes.c_void_p(a.data_ptr())
    assert a.flags["C_CONTIGUOUS"], "arrays must be C contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


class Context:
    """One prism_hip context (one per host thread), mirroring an installed executor."""

    def __init__(self, device: int = 0, max_resident_bytes: int = 0):
        self._h = lib().prism_hip_create(device, max_resident_bytes, 0)
        if not self._h:
            raise RuntimeError(f"prism_hip_create({device}) failed")

    def close(self):
        if self._h:
            lib().prism_hip_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- plumbing --
    def _check(self, rc: int):
        if rc != OK:
            raise PrismError(rc, lib().prism_hip_last_error(self._h).decode())

    @property
    def handle(self):
        return self._h

    @property
    def identity(self) -> str:
        return lib().prism_hip_identity(self._h).decode()

    @property
    def last_error(self) -> str:
        return lib().prism_hip_last_error(self._h).decode()

    @property
    def faulted(self) -> bool:
        return bool(lib().prism_hip_faulted(self._h))

    def inject_fault(self) -> None:
        """Latch this context's device fault from the host (a test hook)."""
        self._check(lib().prism_hip_inject_fault(self._h))

    def operation_capacity(self) -> int:
        return lib().prism_hip_operation_capacity(self._h)

    def operation_count(self, kind: int, cols: int, rows: int) -> int:
        return lib().prism_hip_operation_count(self._h, kind, cols, rows)

    def supports(self, kind: int, cols: int, rows: int, path: int) -> bool:
        return bool(lib().prism_hip_supports(self._h, kind, cols, rows, path))

    def supports_f32_group(self, tensors) -> bool:
        """tensors: [(kind, cols, rows), ...]"""
        return bool(lib().prism_hip_supports_f32_group(self._h, _descs(tensors), len(tensors)))

    def supports_f32_ffn_swiglu(self, gate, up) -> bool:
        d = _descs([gate, up])
        return bool(lib().prism_hip_supports_f32_ffn_swiglu(self._h, ctypes.byref(d[0]), ctypes.byref(d[1])))

    def supports_f32_ffn_chain(self, gate, up, down) -> bool:
        return bool(lib().prism_hip_supports_f32_ffn_chain(self._h, _descs([gate, up, down])))

    def supports_f32_ffn_chain_lora(self, gate, up, down) -> bool:
        return bool(lib().prism_hip_supports_f32_ffn_chain_lora(self._h, _descs([gate, up, down])))

    def set_cancellation(self, flag) -> None:
        """Registers a one-element int32 numpy array as the request's cancellation flag (None
        unregisters); the array is kept alive here while registered."""
        self._cancel = flag
        self._check(lib().prism_hip_set_cancellation(self._h, _ptr(flag) if flag is not None else None))

    def statistics(self) -> dict:
        st = Statistics()
        self._check(lib().prism_hip_get_statistics(self._h, ctypes.byref(st)))
        return st.as_dict()

    def diagnostics(self) -> dict:
        d = Diagnostics()
        self._check(lib().prism_hip_get_diagnostics(self._h, ctypes.byref(d)))
        return {"dispatched": bool(d.dispatched), "succeeded": bool(d.succeeded)}

    def supports_tile_tokens(self) -> bool:
        return bool(lib().prism_hip_supports_tile_tokens(self._h))

    def stream(self) -> int:
        return lib().prism_hip_stream(self._h)

    # -- weights --
    def weight(self, kind: int, cols: int, rows: int, data, key: int | None = None) -> int:
        buf = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray)) else data,
                                   dtype=np.uint8)
        key = next(_fresh_keys) if key is None else key
        wid = lib().prism_hip_weight_acquire(self._h, key & 0xFFFFFFFFFFFFFFFF, kind, cols, rows, _ptr(buf), buf.size)
        if wid < 0:
            self._check(int(wid))
        return int(wid)

    def weight_from_device(self, kind: int, cols: int, rows: int, tensor, key: int | None = None) -> int:
        """Context-owned copy (tiled where supported) of native bytes in device memory."""
        nbytes = tensor.numel() * tensor.element_size()
        key = next(_fresh_keys) if key is None else key
        wid = lib().prism_hip_weight_acquire_device(self._h, key & 0xFFFFFFFFFFFFFFFF, kind, cols, rows, _ptr(tensor),
                                                    nbytes)
        if wid < 0:
            self._check(int(wid))
        return int(wid)

    def weight_from_gguf(self, g: "Gguf", name: str, key: int | None = None) -> int:
        key = next(_fresh_keys) if key is None else key
        wid = lib().prism_hip_weight_from_gguf(self._h, g._h, name.encode(), key & 0xFFFFFFFFFFFFFFFF)
        if wid < 0:
            self._check(int(wid))
        return wid

    def weight_device(self, kind: int, cols: int, rows: int, tensor) -> int:
        nbytes = tensor.numel() * tensor.element_size()
        wid = lib().prism_hip_weight_wrap_device(self._h, kind, cols, rows, _ptr(tensor), nbytes)
        if wid < 0:
            self._check(int(wid))
        return int(wid)

    def tiled_bytes(self, kind: int, cols: int, rows: int) -> int:
        return lib().prism_hip_weight_tiled_bytes(self._h, kind, cols, rows)

    def repack_tiled(self, kind: int, cols: int, rows: int, native, tiled):
        """Writes the tiled image of native device bytes into the caller's device buffer."""
        self._check(lib().prism_hip_weight_repack_tiled(self._h, kind, cols, rows, _ptr(native), native.nbytes,
                                                        _ptr(tiled), tiled.nbytes))

    def weight_tiled_device(self, kind: int, cols: int, rows: int, tiled) -> int:
        """Registers a caller-owned device buffer holding the tiled image (no copy)."""
        wid = lib().prism_hip_weight_wrap_tiled(self._h, kind, cols, rows, _ptr(tiled), tiled.nbytes)
        if wid < 0:
            self._check(int(wid))
        return int(wid)

    def release(self, wid: int):
        self._check(lib().prism_hip_weight_release(self._h, wid))

    def release_all(self):
        self._check(lib().prism_hip_weight_release_all(self._h))

    def resident_bytes(self) -> int:
        return lib().prism_hip_resident_bytes(self._h)

    # -- synchronous host projections; return (code, out) when check=False --
    def _run(self, rc: int, out, check: bool):
        if check:
            self._check(rc)
            return out
        return rc, out

    def project_q8k(self, wid: int, rows: int, act: np.ndarray, tokens: int = 1, fused: bool = False, check=True):
        out = np.full(rows * tokens, 7.0, np.float32)
        rc = lib().prism_hip_project_q8k(self._h, wid, _ptr(act), act.size, tokens, int(fused), _ptr(out))
        return self._run(rc, out.reshape(tokens, rows) if tokens > 1 else out, check)

    def project_q8(self, wid: int, rows: int, act: np.ndarray, tokens: int = 1, pinned: bool = False, check=True):
        out = np.full(rows * tokens, 7.0, np.float32)
        rc = lib().prism_hip_project_q8(self._h, wid, _ptr(act), act.size, tokens, int(pinned), _ptr(out))
        return self._run(rc, out.reshape(tokens, rows) if tokens > 1 else out, check)

    def project_f32(self, wid: int, rows: int, x, tokens: int = 1, pinned: bool = False, check=True):
        x = np.ascontiguousarray(x, np.float32)
        out = np.full(rows * tokens, 7.0, np.float32)
        rc = lib().prism_hip_project_f32(self._h, wid, _ptr(x), tokens, int(pinned), _ptr(out))
        return self._run(rc, out.reshape(tokens, rows) if tokens > 1 else out, check)

    def prefill(self, wid: int, rows: int, X, pinned: bool = False, check=True):
        X = np.ascontiguousarray(X, np.float32)
        out = np.full(X.shape[0] * rows, 7.0, np.float32)
        rc = lib().prism_hip_prefill(self._h, wid, _ptr(X), X.shape[0], int(pinned), _ptr(out))
        return self._run(rc, out.reshape(X.shape[0], rows), check)

    def mul_mat(self, wid: int, rows: int, B, check=True):
        B = np.ascontiguousarray(B, np.float32)
        out = np.full(B.shape[0] * rows, 7.0, np.float32)
        rc = lib().prism_hip_mul_mat(self._h, wid, _ptr(B), B.shape[0], _ptr(out))
        return self._run(rc, out.reshape(B.shape[0], rows), check)

    def project_f32_group(self, wids, rows_list, x, pinned: bool = False, check=True):
        x = np.ascontiguousarray(x, np.float32)
        outs = [np.full(r, 7.0, np.float32) for r in rows_list]
        ids = np.array(wids, np.int64)
        ptrs = (ctypes.c_void_p * len(outs))(*[o.ctypes.data for o in outs])
        rc = lib().prism_hip_project_f32_group(self._h, _ptr(ids), len(outs), _ptr(x), int(pinned), ptrs)
        return self._run(rc, outs, check)

    def project_f32_group_tokens(self, wids, rows_list, X, pinned: bool = False, check=True):
        X = np.ascontiguousarray(X, np.float32)
        tokens = X.shape[0]
        outs = [np.full((tokens, r), 7.0, np.float32) for r in rows_list]
        ids = np.array(wids, np.int64)
        if len(outs) == 2:
            rc = lib().prism_hip_project_f32_pair_tokens(self._h, _ptr(ids), _ptr(X), tokens, int(pinned),
                                                         _ptr(outs[0]), _ptr(outs[1]))
        elif len(outs) == 3:
            rc = lib().prism_hip_project_f32_triple_tokens(self._h, _ptr(ids), _ptr(X), tokens, int(pinned),
                                                           _ptr(outs[0]), _ptr(outs[1]), _ptr(outs[2]))
        else:
            ptrs = (ctypes.c_void_p * len(outs))(*[o.ctypes.data for o in outs])
            rc = lib().prism_hip_project_f32_group_tokens(self._h, _ptr(ids), len(outs), _ptr(X), tokens,
                                                          int(pinned), ptrs)
        return self._run(rc, outs, check)

    def ffn_swiglu_tokens(self, g: int, u: int, ffn: int, X, pinned: bool = False, check=True):
        X = np.ascontiguousarray(X, np.float32)
        out = np.full((X.shape[0], ffn), 7.0, np.float32)
        rc = lib().prism_hip_ffn_swiglu_tokens(self._h, g, u, _ptr(X), X.shape[0], int(pinned), _ptr(out))
        return self._run(rc, out, check)

    def ffn_chain_tokens(self, g: int, u: int, d: int, hidden: int, X, residual=None, pinned: bool = False,
                         check=True, hadamard_block: int = 0):
        """hadamard_block: the chain's hadamard_block_size (0 = None)."""
        X = np.ascontiguousarray(X, np.float32)
        res = np.ascontiguousarray(residual, np.float32) if residual is not None else None
        out = np.full((X.shape[0], hidden), 7.0, np.float32)
        rc = lib().prism_hip_ffn_chain_tokens(self._h, g, u, d, _ptr(X), _ptr(res), X.shape[0], hadamard_block,
                                              int(pinned), _ptr(out))
        return self._run(rc, out, check)

    def ffn_swiglu(self, g: int, u: int, ffn: int, x, pinned: bool = False, check=True):
        x = np.ascontiguousarray(x, np.float32)
        out = np.full(ffn, 7.0, np.float32)
        rc = lib().prism_hip_ffn_swiglu(self._h, g, u, _ptr(x), int(pinned), _ptr(out))
        return self._run(rc, out, check)

    def ffn_chain(self, g: int, u: int, d: int, hidden: int, x, residual=None, pinned: bool = False, check=True,
                  hadamard_block: int = 0):
        """hadamard_block: the chain's hadamard_block_size (0 = None)."""
        x = np.ascontiguousarray(x, np.float32)
        res = np.ascontiguousarray(residual, np.float32) if residual is not None else None
        out = np.full(hidden, 7.0, np.float32)
        rc = lib().prism_hip_ffn_chain(self._h, g, u, d, _ptr(x), _ptr(res), hadamard_block, int(pinned), _ptr(out))
        return self._run(rc, out, check)

    def ffn_chain_lora(self, g: int, u: int, d: int, hidden: int, x, lora_a, residual=None, pinned: bool = False,
                       check=True, hadamard_block: int = 0):
        """Returns (out, lora_dot); out is zero-filled and the dot 0 on failure."""
        x = np.ascontiguousarray(x, np.float32)
        la = np.ascontiguousarray(lora_a, np.float32) if lora_a is not None else None
        res = np.ascontiguousarray(residual, np.float32) if residual is not None else None
        out = np.full(hidden, 7.0, np.float32)
        dot = np.full(1, 7.0, np.float32)
        rc = lib().prism_hip_ffn_chain_lora(self._h, g, u, d, _ptr(x), _ptr(res), hadamard_block, _ptr(la),
                                            int(pinned), _ptr(out), _ptr(dot))
        return self._run(rc, out, check), dot[0]

    # -- device-pointer dispatch (torch tensors) --
    def quantize_q8k_device(self, x, cols: int, tokens: int, pinned: bool, out, stream=None):
        self._check(lib().prism_hip_quantize_q8k_device(self._h, _ptr(x), cols, tokens, int(pinned), _ptr(out), stream))

    def quantize_q8_device(self, x, cols: int, tokens: int, contract: int, out, stream=None):
        self._check(lib().prism_hip_quantize_q8_device(self._h, _ptr(x), cols, tokens, contract, _ptr(out), stream))

    def project_device(self, wid: int, path: int, act, tokens: int, pinned: bool, out, stream=None):
        self._check(lib().prism_hip_project_device(self._h, wid, path, _ptr(act), tokens, int(pinned), _ptr(out), stream))

    def project_device_noalloc(self, wid: int, path: int, act, tokens: int, pinned: bool, out, stream=None,
                               check: bool = True) -> int:
        rc = lib().prism_hip_project_device_noalloc(self._h, wid, path, _ptr(act), tokens, int(pinned), _ptr(out),
                                                    stream)
        if check:
            self._check(rc)
        return rc

    def ffn_chain_device(self, g, u, d, x, residual, pinned, out, h=None, stream=None, hadamard_block: int = 0):
        self._check(lib().prism_hip_ffn_chain_device(self._h, g, u, d, _ptr(x), _ptr(residual), hadamard_block,
                                                     int(pinned), _ptr(out), _ptr(h), stream))

    def sync(self, stream=None) -> int:
        return lib().prism_hip_sync(self._h, stream)


class DecoderLaunchTime(ctypes.Structure):
    """prism_decoder_launch_time."""
    _fields_ = [("name", ctypes.c_char_p), ("launches", ctypes.c_uint32), ("total_us", ctypes.c_double),
                ("bytes", ctypes.c_uint64)]


DECODER_FAMILIES = 9


class DecoderGeometry(ctypes.Structure):
    """prism_decoder_geometry."""
    _fields_ = [(n, ctypes.c_uint64) for n in ("hidden", "ffn", "heads", "kv_heads", "head_dim", "rope", "vocab",
                                                "layers", "max_tokens")] + [
        ("rope_sections", ctypes.c_uint64 * 4), ("rope_base", ctypes.c_float), ("eps", ctypes.c_float)]


class Decoder:
    """A resident full-attention decoder (prism_hip_decoder_*) built from a model dict
    (synth.decoder_model): weights uploaded and repacked once, KV caches prefilled."""

    def __init__(self, ctx: Context, model: dict, max_steps: int = 128):
        g = model["geometry"]
        self.ctx = ctx
        self.g = g
        geo = DecoderGeometry(g["hidden"], g["ffn"], g["heads"], g["kv_heads"], g["head_dim"], g["rope"], g["vocab"],
                              g["layers"], g["max_tokens"], (ctypes.c_uint64 * 4)(*g["rope_sections"]),
                              g["rope_base"], g["eps"])
        self._h = lib().prism_hip_decoder_create(ctx._h, ctypes.byref(geo), max_steps)
        if not self._h:
            code = ERR_DEVICE_FAULT if lib().prism_hip_faulted(ctx._h) else ERR_INVALID_INPUT
            raise PrismError(code, lib().prism_hip_last_error(ctx._h).decode())
        try:
            self.set_weights(model)
            for i, L in enumerate(model["layers"]):
                k = np.ascontiguousarray(L["k_prefill"], np.uint16)
                v = np.ascontiguousarray(L["v_prefill"], np.uint16)
                self._check(lib().prism_hip_decoder_set_cache(self._h, i, _ptr(k), _ptr(v), L["kv_prefill"]))
        except Exception:
            self.close()
            raise

    def set_weights(self, model: dict) -> None:
        """Uploads every layer's tensors and the LM head / final norm."""
        for i, L in enumerate(model["layers"]):
            arrs = [np.ascontiguousarray(L[n]) for n in ("qkv", "o", "gate", "up", "down")]
            norms = [np.ascontiguousarray(L[n], np.float32) for n in ("norm", "post_norm", "q_norm", "k_norm")]
            self._check(lib().prism_hip_decoder_set_layer(self._h, i, *(_ptr(a) for a in arrs + norms)))
        lm = np.ascontiguousarray(model["lm_head"])
        on = np.ascontiguousarray(model["output_norm"], np.float32)
        self._check(lib().prism_hip_decoder_set_head(self._h, _ptr(lm), _ptr(on)))

    def _check(self, rc: int) -> None:
        if rc != OK:
            raise PrismError(rc, lib().prism_hip_last_error(self.ctx._h).decode())

    def generate(self, token: int, pos: int, steps: int, graph: bool = True, logits: bool = False):
        """Greedy decode: returns (tokens[steps], logits[steps][vocab] or None, device seconds)."""
        toks = np.zeros(steps, np.uint32)
        lg = np.zeros((steps, self.g["vocab"]), np.float32) if logits else None
        secs = ctypes.c_double(0.0)
        self._check(lib().prism_hip_decoder_generate(self._h, token, pos, steps, int(graph), _ptr(toks),
                                                     _ptr(lg) if logits else None, ctypes.byref(secs)))
        return toks, lg, secs.value

    def profile(self, token: int, pos: int, steps: int) -> list[dict]:
        """Eager steps with an event before every launch: per launch family, the launches
        timed, their summed microseconds (dispatch gaps included) and bytes per launch."""
        st = (DecoderLaunchTime * DECODER_FAMILIES)()
        self._check(lib().prism_hip_decoder_profile(self._h, token, pos, steps, st))
        return [{"family": s.name.decode(), "launches": int(s.launches), "total_us": float(s.total_us),
                 "bytes_per_launch": int(s.bytes)} for s in st]

    def time_family(self, family: str, reps: int) -> tuple[float, int]:
        """Back-to-back launches of one family (layers cycled): (mean us per launch, bytes)."""
        us, nb = ctypes.c_double(0.0), ctypes.c_uint64(0)
        self._check(lib().prism_hip_decoder_time_family(self._h, family.encode(), reps, ctypes.byref(us),
                                                        ctypes.byref(nb)))
        return us.value, int(nb.value)

    def close(self) -> None:
        if self._h:
            lib().prism_hip_decoder_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
