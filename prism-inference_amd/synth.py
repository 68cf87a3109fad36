"""Seeded synthetic packed tensors and activations for the benchmark configurations.

Distributions follow the workload definitions: ternary weights with codes
{-1,0,+1} drawn with p=1/3 each and one binary16 scale |N(0,0.02)| per 128-weight
block; 2-bit Q2_K super-blocks with uniform codes, uniform 4-bit sub-block
scales/mins, d=|N(0,0.02)| and dmin=N(0,0.01); Q8_0 blocks quantized from
N(0,0.02) floats; activations N(0,1).  Every tensor is produced in the
reference's native byte layout (src/kernels.rs:88-119).
"""

from __future__ import annotations

import numpy as np

KIND_Q8_0 = 8
KIND_Q2_K = 10
KIND_TQ1_0 = 34
KIND_TQ2_0 = 35
KIND_PQ2 = 142
KIND_PTQ1 = 143
LAYOUT = {KIND_Q8_0: (32, 34), KIND_Q2_K: (256, 84), KIND_PQ2: (128, 34), KIND_PTQ1: (128, 28),
          KIND_TQ1_0: (256, 54), KIND_TQ2_0: (256, 66)}


def row_bytes(kind: int, cols: int) -> int:
    g, b = LAYOUT[kind]
    assert cols % g == 0
    return cols // g * b


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(v.astype(np.float16)).view(np.uint8).reshape(-1, 2)


def _scales(rng, n: int, sigma: float = 0.02, signed: bool = False) -> np.ndarray:
    s = rng.normal(0.0, sigma, n)
    return _f16_bytes(s if signed else np.abs(s))


def pack_ptq1(codes: np.ndarray, scale_bytes: np.ndarray) -> np.ndarray:
    """Canonical PTQ1 bytes for blocks of 128 codes in {0,1,2} (trit+1).

    Digit 0 is most significant and each byte is ceil(q*256/243) of its base-3
    group (tools/ternary/src/lib.rs:163-189).
    """
    nb = codes.shape[0]
    c = codes.astype(np.int64)
    p5 = np.array([81, 27, 9, 3, 1], np.int64)
    q16 = np.einsum("bnm,n->bm", c[:, :80].reshape(nb, 5, 16), p5)
    q8 = np.einsum("bnm,n->bm", c[:, 80:120].reshape(nb, 5, 8), p5)
    qt = np.einsum("bnm,n->bm", c[:, 120:128].reshape(nb, 4, 2), p5[1:])
    out = np.empty((nb, 28), np.uint8)
    out[:, 0:16] = (q16 * 256 + 242) // 243
    out[:, 16:24] = (q8 * 256 + 242) // 243
    out[:, 24:26] = (qt * 3 * 256 + 242) // 243
    out[:, 26:28] = scale_bytes
    return out


def pack_pq2(codes: np.ndarray, scale_bytes: np.ndarray) -> np.ndarray:
    """PQ2 blocks: f16 scale then 2-bit codes, element i at byte 2+i/4, bits 2*(i%4)."""
    nb = codes.shape[0]
    c = codes.astype(np.uint8).reshape(nb, 32, 4)
    out = np.empty((nb, 34), np.uint8)
    out[:, 0:2] = scale_bytes
    out[:, 2:] = c[:, :, 0] | (c[:, :, 1] << 2) | (c[:, :, 2] << 4) | (c[:, :, 3] << 6)
    return out


def ptq1_weights(rows: int, cols: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    nb = rows * cols // 128
    codes = rng.integers(0, 3, (nb, 128), dtype=np.int8)
    return pack_ptq1(codes, _scales(rng, nb)).reshape(-1)


def pq2_weights(rows: int, cols: int, seed: int, levels: int = 3) -> np.ndarray:
    """levels=3: ternary codes {0,1,2}; levels=4 also draws the +2 code."""
    rng = np.random.default_rng(seed)
    nb = rows * cols // 128
    codes = rng.integers(0, levels, (nb, 128), dtype=np.int8)
    return pack_pq2(codes, _scales(rng, nb)).reshape(-1)


def q2k_weights(rows: int, cols: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    nb = rows * cols // 256
    out = np.empty((nb, 84), np.uint8)
    out[:, 0:16] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)  # 4-bit scale | 4-bit min
    out[:, 16:80] = rng.integers(0, 256, (nb, 64), dtype=np.uint8)  # 2-bit codes
    out[:, 80:82] = _scales(rng, nb)
    out[:, 82:84] = _scales(rng, nb, 0.01, signed=True)
    return out.reshape(-1)


def q8_0_weights(rows: int, cols: int, seed: int) -> np.ndarray:
    """Q8_0 blocks from N(0,0.02) floats: d = max/127, codes rounded half away from zero."""
    rng = np.random.default_rng(seed)
    nb = rows * cols // 32
    out = np.empty((nb, 34), np.uint8)
    step = 1 << 20
    for s in range(0, nb, step):
        e = min(nb, s + step)
        x = rng.normal(0.0, 0.02, (e - s, 32)).astype(np.float32)
        d = np.abs(x).max(axis=1) / np.float32(127.0)
        inv = np.where(d == 0, np.float32(0), np.float32(1.0) / np.where(d == 0, 1, d)).astype(np.float32)
        p = x * inv[:, None]
        q = np.clip(np.sign(p) * np.floor(np.abs(p) + np.float32(0.5)), -127, 127).astype(np.int8)
        out[s:e, 0:2] = _f16_bytes(d)
        out[s:e, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def tq_weights(kind: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """TQ1_0 / TQ2_0 blocks: uniform code bytes (every byte is a valid code: TQ1_0 base-3
    digits of any byte, TQ2_0 2-bit fields 0..3) and one binary16 scale |N(0,0.02)|."""
    rng = np.random.default_rng(seed)
    _, bb = LAYOUT[kind]
    nb = rows * cols // 256
    out = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
    out[:, bb - 2:] = _f16_bytes(np.abs(rng.normal(0.0, 0.02, nb)).astype(np.float32)).reshape(nb, 2)
    return out.reshape(-1)


def weights(kind: int, rows: int, cols: int, seed: int) -> np.ndarray:
    if kind == KIND_PTQ1:
        return ptq1_weights(rows, cols, seed)
    if kind == KIND_PQ2:
        return pq2_weights(rows, cols, seed)
    if kind == KIND_Q2_K:
        return q2k_weights(rows, cols, seed)
    if kind == KIND_Q8_0:
        return q8_0_weights(rows, cols, seed)
    if kind in (KIND_TQ1_0, KIND_TQ2_0):
        return tq_weights(kind, rows, cols, seed)
    raise ValueError(kind)


def activations(n: int, seed: int, tokens: int = 1) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((tokens, n)).astype(np.float32)
    return x[0] if tokens == 1 else x


# ---- full-attention decode step ------------------------------------------------------

# The 28-layer decode workload: hidden 2048, 16 query / 4 KV heads of 128, FFN 6144,
# tied 151936-token Q8_0 LM head, binary16 KV cache prefilled to 1024 tokens with room
# for 128 more.  RoPE on 64 of each head's 128 dimensions with base 1e7 and M-RoPE
# sections (11, 11, 10, 0), the reference's Qwen35 test geometry (src/graph.rs:7321-7322).
DECODE_GEOMETRY = {
    "hidden": 2048, "ffn": 6144, "heads": 16, "kv_heads": 4, "head_dim": 128, "rope": 64,
    "rope_sections": (11, 11, 10, 0), "rope_base": 10_000_000.0, "eps": 1e-6,
    "vocab": 151936, "layers": 28, "max_tokens": 1024 + 128,
}


def _norm_weights(rng, n: int) -> np.ndarray:
    """RMSNorm weights 1 + 0.1 N(0,1) (binary32)."""
    return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)


def decoder_model(seed: int = 0, kv_prefill: int = 1024, **overrides) -> dict:
    """Seeded synthetic decoder: every linear layer PTQ1 (the ternary distribution
    above), q/k/v stacked into one matrix of (heads + 2 kv_heads) * head_dim rows, a
    Q8_0 LM head from N(0,0.02) floats that doubles as the token embedding, RMSNorm
    weights around 1, and binary16 KV caches prefilled with N(0,1) values."""
    g = dict(DECODE_GEOMETRY)
    g.update(overrides)
    H, F, D = g["hidden"], g["ffn"], g["head_dim"]
    QW, KW = g["heads"] * D, g["kv_heads"] * D
    assert kv_prefill <= g["max_tokens"]
    rng = np.random.default_rng(seed)
    layers = []
    for layer in range(g["layers"]):
        s = 1_000_003 * seed + 16 * layer
        layers.append({
            "qkv": ptq1_weights(QW + 2 * KW, H, s + 1),
            "o": ptq1_weights(H, QW, s + 2),
            "gate": ptq1_weights(F, H, s + 3),
            "up": ptq1_weights(F, H, s + 4),
            "down": ptq1_weights(H, F, s + 5),
            "norm": _norm_weights(rng, H),
            "post_norm": _norm_weights(rng, H),
            "q_norm": _norm_weights(rng, D),
            "k_norm": _norm_weights(rng, D),
            "kv_prefill": kv_prefill,
            "k_prefill": rng.standard_normal((kv_prefill, KW)).astype(np.float16).view(np.uint16),
            "v_prefill": rng.standard_normal((kv_prefill, KW)).astype(np.float16).view(np.uint16),
        })
    return {
        "geometry": g,
        "layers": layers,
        "lm_head": q8_0_weights(g["vocab"], H, 1_000_003 * seed + 999_983),
        "output_norm": _norm_weights(rng, H),
    }
