"""ctypes binding for the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.

The C functions restate the reference's scalar Rust kernels; see the header of
prism_oracle.c for what pins each one.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

KIND_Q8_0 = 8
KIND_Q2_K = 10
KIND_Q8_K = 15
KIND_TQ1_0 = 34
KIND_TQ2_0 = 35
KIND_PQ2 = 142
KIND_PTQ1 = 143

Q8_SOURCE = 0
Q8_PINNED = 1
Q8_PINNED_NATIVE = 2

OK = 0
ERR_INVALID_INPUT = -1
ERR_RESOURCE = -2
ERR_NONFINITE = -3
ERR_UNSUPPORTED = -5

LAYOUT = {KIND_Q8_0: (32, 34), KIND_Q2_K: (256, 84), KIND_Q8_K: (256, 292), KIND_PQ2: (128, 34), KIND_PTQ1: (128, 28),
          KIND_TQ1_0: (256, 54), KIND_TQ2_0: (256, 66)}

# numpy mirrors of the C structs (tools/ternary/src/lib.rs:27-39; src/kernels.rs:528-535)
Q8K_DTYPE = np.dtype([("scale", "<f4"), ("values", "i1", (256,)), ("sums", "<i2", (16,))])
Q8_DTYPE = np.dtype([("scale", "<f4"), ("sum", "<f4"), ("values", "i1", (32,))])
assert Q8K_DTYPE.itemsize == 292 and Q8_DTYPE.itemsize == 40


class OracleError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what} failed with code {code}")
        self.code = code


def build() -> None:
    """Compile liboracle.so with oracle/Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        S = ctypes.c_size_t
        I = ctypes.c_int
        U = ctypes.c_uint32
        sig = {
            "po_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
            "po_half_to_float_bits": (ctypes.c_uint32, [ctypes.c_uint16]),
            "po_float_to_half": (ctypes.c_uint16, [ctypes.c_float]),
            "po_round_f16": (ctypes.c_float, [ctypes.c_float]),
            "po_decode_ptq_trits": (None, [P, P]),
            "po_pack_ptq": (I, [P, P]),
            "po_unpack_ptq": (I, [P, P]),
            "po_quantize_q8k": (I, [P, S, I, P]),
            "po_quantize_q8_0": (I, [P, S, I, P]),
            "po_quantize_row": (I, [U, P, S, P, S]),
            "po_decode_row": (I, [U, S, P, P]),
            "po_dot_pq2": (I, [P, S, P, I, P]),
            "po_dot_q8_groups": (I, [U, P, S, P, P]),
            "po_dot_q8_groups_pinned": (I, [U, P, S, P, P]),
            "po_dot_q2k": (I, [P, S, P, P]),
            "po_dot_q8_0": (I, [P, S, P, P]),
            "po_dot_ptq1_q8k": (I, [P, S, P, P]),
            "po_packed_dot": (I, [U, S, P, S, P, S, P]),
            "po_activation_contract": (I, [U, S, I]),
            "po_matvec": (I, [U, S, S, P, P, I, P, I]),
            "po_project_q8k": (I, [U, S, S, P, P, I, P, I]),
            "po_project_q8": (I, [U, S, S, P, P, I, P, I]),
            "po_vector_exp": (ctypes.c_float, [ctypes.c_float]),
            "po_silu": (None, [P, S, I]),
            "po_swiglu": (None, [P, P, S, I]),
            "po_lora_a_dot": (I, [P, P, S, I, P]),
            "po_ffn": (I, [U, S, S, P, P, P, P, P, I, P, P, I]),
            "po_hadamard": (I, [P, S, U]),
            "po_ffn_rotated": (I, [U, S, S, P, P, P, P, P, U, I, P, P, I]),
            "po_rms_norm": (I, [P, P, S, ctypes.c_float, P]),
            "po_rope_frequencies": (None, [S, P, P, ctypes.c_float, P, P]),
            "po_norm_rope_f16": (I, [P, P, S, S, P, P, ctypes.c_float]),
            "po_softmax_round_f16": (I, [P, S]),
            "po_attention_head": (I, [P, P, P, S, S, S, P, P, S, P, P]),
            "po_decoder_step": (I, [P, P, P, P, U, S, P, I]),
            "po_argmax": (S, [P, S]),
            "po_tq_codes": (None, [U, P, P]),
            "po_dot_tq": (I, [U, P, S, P, P]),
            "po_quantize_tq": (I, [U, P, S, P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(bytes(a), dtype=np.uint8) if isinstance(a, (bytes, bytearray)) else a, dtype=np.uint8)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _check(rc: int, what: str) -> None:
    if rc != OK:
        raise OracleError(rc, what)


def half_to_float(h: int) -> float:
    return lib().po_half_to_float(h)


def half_to_float_bits(h: int) -> int:
    return lib().po_half_to_float_bits(h)


def float_to_half(f: float) -> int:
    return lib().po_float_to_half(f)


def decode_ptq_trits(block) -> np.ndarray:
    b = _u8(block)
    assert b.size == 28
    out = np.zeros(128, np.int16)
    lib().po_decode_ptq_trits(_p(b), _p(out))
    return out


def pack_ptq(pq2) -> bytes:
    b = _u8(pq2)
    out = np.zeros(28, np.uint8)
    _check(lib().po_pack_ptq(_p(b), _p(out)), "pack_ptq")
    return out.tobytes()


def unpack_ptq(ptq) -> bytes:
    b = _u8(ptq)
    out = np.zeros(34, np.uint8)
    _check(lib().po_unpack_ptq(_p(b), _p(out)), "unpack_ptq")
    return out.tobytes()


def quantize_q8k(x, pinned: bool) -> np.ndarray:
    x = _f32(x)
    out = np.zeros(x.size // 256, Q8K_DTYPE)
    _check(lib().po_quantize_q8k(_p(x), x.size, int(pinned), _p(out)), "quantize_q8k")
    return out


def quantize_q8_0(x, contract: int) -> np.ndarray:
    x = _f32(x)
    out = np.zeros(x.size // 32, Q8_DTYPE)
    _check(lib().po_quantize_q8_0(_p(x), x.size, contract, _p(out)), "quantize_q8_0")
    return out


def quantize_row(kind: int, x) -> bytes:
    x = _f32(x)
    g, bb = LAYOUT[kind]
    out = np.zeros(x.size // g * bb, np.uint8)
    _check(lib().po_quantize_row(kind, _p(x), x.size, _p(out), out.size), "quantize_row")
    return out.tobytes()


def decode_row(kind: int, count: int, data) -> np.ndarray:
    d = _u8(data)
    out = np.zeros(count, np.float32)
    _check(lib().po_decode_row(kind, count, _p(d), _p(out)), "decode_row")
    return out


def _f(fn, *args) -> float:
    out = np.zeros(1, np.float32)
    _check(fn(*args, _p(out)), fn.__name__)
    return out


def dot_pq2(row, act: np.ndarray, fused: bool) -> np.float32:
    r = _u8(row)
    return _f(lib().po_dot_pq2, _p(r), r.size // 34, _p(act), int(fused))[0]


def dot_q8_groups(kind: int, row, act: np.ndarray, pinned: bool = False) -> np.float32:
    r = _u8(row)
    bb = 34 if kind == KIND_PQ2 else 28
    fn = lib().po_dot_q8_groups_pinned if pinned else lib().po_dot_q8_groups
    return _f(fn, kind, _p(r), r.size // bb, _p(act))[0]


def dot_q2k(row, act: np.ndarray) -> np.float32:
    r = _u8(row)
    return _f(lib().po_dot_q2k, _p(r), r.size // 84, _p(act))[0]


def dot_q8_0(row, act: np.ndarray) -> np.float32:
    r = _u8(row)
    return _f(lib().po_dot_q8_0, _p(r), r.size // 34, _p(act))[0]


def tq_codes(kind: int, block) -> np.ndarray:
    """The 256 signed digits of one TQ1_0 / TQ2_0 block, in element order."""
    b = _u8(block)
    out = np.zeros(256, np.int16)
    lib().po_tq_codes(kind, _p(b), _p(out))
    return out


def dot_tq(kind: int, row, act: np.ndarray) -> np.float32:
    w = _u8(row)
    return _f(lib().po_dot_tq, kind, _p(w), act.size, _p(act))[0]


def dot_ptq1_q8k(row, act: np.ndarray) -> np.float32:
    r = _u8(row)
    return _f(lib().po_dot_ptq1_q8k, _p(r), r.size // 28, _p(act))[0]


def packed_dot(kind: int, count: int, weights, activations) -> np.float32:
    w = _u8(weights)
    a = _u8(activations)
    return _f(lib().po_packed_dot, kind, count, _p(w), w.size, _p(a), a.size)[0]


def activation_contract(kind: int, cols: int, pinned: bool) -> int:
    return lib().po_activation_contract(kind, cols, int(pinned))


def matvec(kind: int, cols: int, rows: int, w, x, pinned: bool = False, threads: int = 1) -> np.ndarray:
    w = _u8(w)
    x = _f32(x)
    out = np.zeros(rows, np.float32)
    _check(lib().po_matvec(kind, cols, rows, _p(w), _p(x), int(pinned), _p(out), threads), "matvec")
    return out


def matvec_rc(kind: int, cols: int, rows: int, w, x, pinned: bool = False, threads: int = 1):
    """Like matvec but returns (code, output) instead of raising."""
    w = _u8(w)
    x = _f32(x)
    out = np.full(rows, 7.0, np.float32)
    rc = lib().po_matvec(kind, cols, rows, _p(w), _p(x), int(pinned), _p(out), threads)
    return rc, out


def project_q8k(kind: int, cols: int, rows: int, w, act: np.ndarray, fused: bool, threads: int = 1) -> np.ndarray:
    w = _u8(w)
    out = np.zeros(rows, np.float32)
    _check(lib().po_project_q8k(kind, cols, rows, _p(w), _p(act), int(fused), _p(out), threads), "project_q8k")
    return out


def project_q8(kind: int, cols: int, rows: int, w, act: np.ndarray, pinned: bool, threads: int = 1) -> np.ndarray:
    w = _u8(w)
    out = np.zeros(rows, np.float32)
    _check(lib().po_project_q8(kind, cols, rows, _p(w), _p(act), int(pinned), _p(out), threads), "project_q8")
    return out


def vector_exp(x: float) -> float:
    return lib().po_vector_exp(x)


def silu(x, pinned: bool) -> np.ndarray:
    v = _f32(x).copy()
    lib().po_silu(_p(v), v.size, int(pinned))
    return v


def swiglu(gate, up, pinned: bool) -> np.ndarray:
    g = _f32(gate)
    u = _f32(up).copy()
    lib().po_swiglu(_p(g), _p(u), g.size, int(pinned))
    return u


def lora_a_dot(a, h, pinned: bool) -> np.float32:
    """lora_a_dot (src/kernels.rs:2336-2357) of the LoRA A factor with the SwiGLU vector."""
    a, h = _f32(a), _f32(h)
    out = np.zeros(1, np.float32)
    _check(lib().po_lora_a_dot(_p(a), _p(h), a.size, int(pinned), _p(out)), "lora_a_dot")
    return out[0]


def hadamard(values, block: int) -> np.ndarray:
    """Blockwise normalized Walsh-Hadamard rotation (src/kernels.rs:3952-3987)."""
    v = _f32(values).copy()
    _check(lib().po_hadamard(_p(v), v.size, block), "hadamard")
    return v


def ffn(kind: int, hidden: int, ffn_dim: int, wg, wu, wd, x, residual=None, pinned: bool = False, threads: int = 1,
        hadamard_block: int = 0):
    """The FFN chain; returns (out, the unrotated SwiGLU vector)."""
    wg, wu, wd = _u8(wg), _u8(wu), _u8(wd)
    x = _f32(x)
    out = np.zeros(hidden, np.float32)
    h = np.zeros(ffn_dim, np.float32)
    res = _f32(residual) if residual is not None else None
    rc = lib().po_ffn_rotated(kind, hidden, ffn_dim, _p(wg), _p(wu), _p(wd), _p(x),
                              _p(res) if res is not None else None, hadamard_block, int(pinned), _p(out), _p(h),
                              threads)
    _check(rc, "ffn")
    return out, h


def prefill(kind: int, cols: int, rows: int, w, X, pinned: bool = False, threads: int = 1) -> np.ndarray:
    """Tiled prefill semantics: each token row equals its own matvec (src/kernels/prefill.rs:829-887)."""
    X = _f32(X)
    return np.stack([matvec(kind, cols, rows, w, X[m], pinned, threads) for m in range(X.shape[0])])


# ---- full-attention decode step (decoder_oracle.c) ---------------------------------

class DecoderGeometry(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in ("hidden", "ffn", "heads", "kv_heads", "head_dim", "rope", "vocab",
                                                "layers", "max_tokens")] + [
        ("rope_sections", ctypes.c_size_t * 4), ("rope_base", ctypes.c_float), ("eps", ctypes.c_float)]


class DecoderLayer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("qkv", "o", "gate", "up", "down", "norm", "post_norm", "q_norm",
                                                "k_norm", "kcache", "vcache")]


def rms_norm(x, w, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.zeros_like(x)
    _check(lib().po_rms_norm(_p(x), _p(w), x.size, eps, _p(out)), "rms_norm")
    return out


def rope_frequencies(rope: int, sections, positions, base: float):
    sec = (ctypes.c_size_t * 4)(*sections)
    pos = (ctypes.c_size_t * 4)(*positions)
    c = np.zeros(rope // 2, np.float32)
    s = np.zeros(rope // 2, np.float32)
    lib().po_rope_frequencies(rope, sec, pos, base, _p(c), _p(s))
    return c, s


def norm_rope_f16(v, w, rope: int, cosines, sines, eps: float) -> np.ndarray:
    v = _f32(v).copy()
    w, c, s = _f32(w), _f32(cosines), _f32(sines)
    _check(lib().po_norm_rope_f16(_p(v), _p(w), v.size, rope, _p(c), _p(s), eps), "norm_rope_f16")
    return v


def softmax_round_f16(v) -> np.ndarray:
    v = _f32(v).copy()
    _check(lib().po_softmax_round_f16(_p(v), v.size), "softmax_round_f16")
    return v


def attention_head(q, kc, vc, stride: int, offset: int, past: int, kcur, vcur) -> np.ndarray:
    q, kcur, vcur = _f32(q), _f32(kcur), _f32(vcur)
    kc = np.ascontiguousarray(kc, np.uint16)
    vc = np.ascontiguousarray(vc, np.uint16)
    scores = np.zeros(past + 1, np.float32)
    out = np.zeros(q.size, np.float32)
    _check(lib().po_attention_head(_p(q), _p(kc), _p(vc), stride, offset, past, _p(kcur), _p(vcur), q.size,
                                   _p(scores), _p(out)), "attention_head")
    return out


def argmax(v) -> int:
    v = _f32(v)
    return int(lib().po_argmax(_p(v), v.size))


class Decoder:
    """The decode step over a model dict (see prism_hip.synth decoder models): holds its
    own binary16 KV caches, which every step appends to."""

    def __init__(self, model: dict, threads: int = 1):
        g = model["geometry"]
        self.model = model
        self.threads = threads
        self.g = DecoderGeometry(g["hidden"], g["ffn"], g["heads"], g["kv_heads"], g["head_dim"], g["rope"],
                                 g["vocab"], g["layers"], g["max_tokens"], (ctypes.c_size_t * 4)(*g["rope_sections"]),
                                 g["rope_base"], g["eps"])
        kw = g["kv_heads"] * g["head_dim"]
        self.kcache, self.vcache = [], []
        keep = []
        layers = (DecoderLayer * g["layers"])()
        for i, L in enumerate(model["layers"]):
            k = np.zeros((g["max_tokens"], kw), np.uint16)
            v = np.zeros((g["max_tokens"], kw), np.uint16)
            n = L["kv_prefill"]
            k[:n] = L["k_prefill"]
            v[:n] = L["v_prefill"]
            self.kcache.append(k)
            self.vcache.append(v)
            arrs = {name: np.ascontiguousarray(L[name]) for name in ("qkv", "o", "gate", "up", "down", "norm",
                                                                       "post_norm", "q_norm", "k_norm")}
            keep.append(arrs)
            layers[i] = DecoderLayer(*(_p(arrs[n]) for n in ("qkv", "o", "gate", "up", "down", "norm", "post_norm",
                                                              "q_norm", "k_norm")), _p(k), _p(v))
        self.layers = layers
        self._keep = keep
        self.lm_head = np.ascontiguousarray(model["lm_head"])
        self.output_norm = _f32(model["output_norm"])

    def step(self, token: int, pos: int) -> np.ndarray:
        logits = np.zeros(self.g.vocab, np.float32)
        rc = lib().po_decoder_step(ctypes.byref(self.g), self.layers, _p(self.lm_head), _p(self.output_norm),
                                   token, pos, _p(logits), self.threads)
        _check(rc, "decoder_step")
        return logits
