"""The oracle's decode-step pieces against what the mathematics fixes: RMS
normalization, RoPE as a rotation, the softmax, one attention head, and the layer
composition against an independent float64 evaluation (projections through the
oracle's pinned matvec)."""

import numpy as np
import pytest

import synth


def f64_rms(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(w, np.float64)


def test_rms_norm_closed_forms(oracle):
    # [3, 4]: mean square 12.5
    got = oracle.rms_norm(np.array([3, 4], np.float32), np.array([1, 2], np.float32), 0.0)
    np.testing.assert_allclose(got, [3 / np.sqrt(12.5), 8 / np.sqrt(12.5)], rtol=2e-7)
    # epsilon enters under the root: zeros with eps 1 give zeros, scale 1
    assert np.array_equal(oracle.rms_norm(np.zeros(8, np.float32), np.ones(8, np.float32), 1.0), np.zeros(8))
    # zeros with eps 0 have no finite scale; a non-finite input is rejected
    for x in (np.zeros(4, np.float32), np.array([1, np.inf, 0, 0], np.float32)):
        with pytest.raises(oracle.OracleError):
            oracle.rms_norm(x, np.ones(4, np.float32), 0.0)
    rng = np.random.default_rng(0)
    x = rng.standard_normal(2048).astype(np.float32) * 3
    w = (1 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
    np.testing.assert_allclose(oracle.rms_norm(x, w, 1e-6), f64_rms(x, w, 1e-6), rtol=1e-6, atol=1e-7)


def test_rope_is_the_rotation(oracle):
    rope, base = 64, 1e7
    c0, s0 = oracle.rope_frequencies(rope, (11, 11, 10, 0), (0, 0, 0, 0), base)
    assert np.all(c0 == 1) and np.all(s0 == 0)
    pos = 1037
    c, s = oracle.rope_frequencies(rope, (11, 11, 10, 0), (pos, pos, pos, 0), base)
    i = np.arange(rope // 2)
    ang = pos * base ** (-2.0 * i / rope)
    np.testing.assert_allclose(c, np.cos(ang), atol=5e-4)
    np.testing.assert_allclose(s, np.sin(ang), atol=5e-4)
    # sections past 3*section fall back to the fourth position (0): no rotation there
    c2, s2 = oracle.rope_frequencies(rope, (1, 1, 1, 0), (pos, pos, pos, 0), base)
    assert np.all(c2[3:] == 1) and np.all(s2[3:] == 0) and s2[1] != 0
    rng = np.random.default_rng(1)
    x = rng.standard_normal(128).astype(np.float32)
    w = np.ones(128, np.float32)
    got = oracle.norm_rope_f16(x, w, rope, c, s, 1e-6)
    n = f64_rms(x, w, 1e-6)
    want = n.copy()
    want[:32] = n[:32] * c - n[32:64] * s
    want[32:64] = n[:32] * s + n[32:64] * c
    np.testing.assert_allclose(got, want, atol=4e-3)           # binary16 output
    assert np.array_equal(got, got.astype(np.float16).astype(np.float32))
    # a rotation keeps every pair's length
    np.testing.assert_allclose(np.hypot(got[:32], got[32:64]), np.hypot(n[:32], n[32:64]), rtol=4e-3)


def test_softmax_round_f16(oracle):
    rng = np.random.default_rng(2)
    v = (rng.standard_normal(1025) * 3).astype(np.float32)
    p = oracle.softmax_round_f16(v)
    e = np.exp(v.astype(np.float64) - v.max())
    ref = e / e.sum()
    np.testing.assert_allclose(p, ref, rtol=2 ** -10, atol=2 ** -24)
    assert np.array_equal(p, p.astype(np.float16).astype(np.float32))
    assert abs(p.astype(np.float64).sum() - 1) < 1e-3
    # equal logits: every probability is binary16(1/n)
    assert np.all(oracle.softmax_round_f16(np.full(7, 2.5, np.float32)) == np.float32(np.float16(1 / 7)))
    for bad in ([np.nan, 0.0], [np.inf, 0.0], [-np.inf, -np.inf]):
        with pytest.raises(oracle.OracleError):
            oracle.softmax_round_f16(np.array(bad, np.float32))


def test_attention_head_matches_float64(oracle):
    rng = np.random.default_rng(3)
    D, past, kvh = 128, 300, 2
    q = rng.standard_normal(D).astype(np.float16).astype(np.float32)
    kc = rng.standard_normal((past, kvh * D)).astype(np.float16)
    vc = rng.standard_normal((past, kvh * D)).astype(np.float16)
    kcur = rng.standard_normal(D).astype(np.float16).astype(np.float32)
    vcur = rng.standard_normal(D).astype(np.float16).astype(np.float32)
    off = D  # second KV head
    got = oracle.attention_head(q, kc.view(np.uint16), vc.view(np.uint16), kvh * D, off, past, kcur, vcur)
    K = np.vstack([kc[:, off:off + D].astype(np.float64), kcur.astype(np.float64)])
    V = np.vstack([vc[:, off:off + D].astype(np.float64), vcur.astype(np.float64)])
    s = K @ q.astype(np.float64) / np.sqrt(D)
    p = np.exp(s - s.max())
    p /= p.sum()
    np.testing.assert_allclose(got, p @ V, atol=2e-3)


def f64_decoder_step(oracle, model, kc, vc, token, pos):
    """Independent float64 evaluation of one step (projections via oracle.matvec)."""
    g = model["geometry"]
    H, D, F = g["hidden"], g["head_dim"], g["ffn"]
    QW, KW = g["heads"] * D, g["kv_heads"] * D
    group = g["heads"] // g["kv_heads"]
    c, s = oracle.rope_frequencies(g["rope"], g["rope_sections"], (pos, pos, pos, 0), g["rope_base"])
    r = g["rope"] // 2

    def mv(kind, w, cols, rows, x):
        return oracle.matvec(kind, cols, rows, w, np.asarray(x, np.float32)).astype(np.float64)

    def rot(x):
        y = x.copy()
        y[:r] = x[:r] * c - x[r:2 * r] * s
        y[r:2 * r] = x[:r] * s + x[r:2 * r] * c
        return y

    h = oracle.decode_row(8, H, model["lm_head"][token * (H // 32) * 34:(token + 1) * (H // 32) * 34]).astype(np.float64)
    for li, L in enumerate(model["layers"]):
        qkv = mv(143, L["qkv"], H, QW + 2 * KW, f64_rms(h, L["norm"], g["eps"]))
        q = [rot(f64_rms(qkv[i * D:(i + 1) * D], L["q_norm"], g["eps"])) for i in range(g["heads"])]
        k = [rot(f64_rms(qkv[QW + i * D:QW + (i + 1) * D], L["k_norm"], g["eps"])) for i in range(g["kv_heads"])]
        v = [qkv[QW + KW + i * D:QW + KW + (i + 1) * D] for i in range(g["kv_heads"])]
        att = []
        for hd in range(g["heads"]):
            kh = hd // group
            K = np.vstack([kc[li][:pos, kh * D:(kh + 1) * D].astype(np.float64), k[kh]])
            V = np.vstack([vc[li][:pos, kh * D:(kh + 1) * D].astype(np.float64), v[kh]])
            sc = K @ q[hd] / np.sqrt(D)
            p = np.exp(sc - sc.max())
            att.append((p / p.sum()) @ V)
        h = h + mv(143, L["o"], QW, H, np.concatenate(att))
        x = f64_rms(h, L["post_norm"], g["eps"])
        gate, up = mv(143, L["gate"], H, F, x), mv(143, L["up"], H, F, x)
        h = h + mv(143, L["down"], F, H, up * gate / (1 + np.exp(-gate)))
    return mv(8, model["lm_head"], H, g["vocab"], f64_rms(h, model["output_norm"], g["eps"]))


def test_decoder_step_composition(oracle):
    """Heads, KV groups, residuals and the FFN chain wired as the float64 evaluation
    wires them, over three steps that append to the caches."""
    model = synth.decoder_model(7, kv_prefill=5, hidden=256, ffn=384, heads=4, kv_heads=2, vocab=96, layers=2,
                                max_tokens=16)
    dec = oracle.Decoder(model)
    kc = [L["k_prefill"].view(np.float16).copy() for L in model["layers"]]
    vc = [L["v_prefill"].view(np.float16).copy() for L in model["layers"]]
    tok = 3
    for step in range(3):
        pos = 5 + step
        got = dec.step(tok, pos)
        want = f64_decoder_step(oracle, model, [dec.kcache[i].view(np.float16) for i in range(2)],
                                [dec.vcache[i].view(np.float16) for i in range(2)], tok, pos)
        assert np.abs(got - want).max() <= 2e-2 * np.abs(want).max()
        # the step appended its key and value at `pos` (binary16) and nothing after
        for i in range(2):
            assert np.any(dec.kcache[i][pos] != 0) and not np.any(dec.kcache[i][pos + 1:])
            assert np.array_equal(dec.kcache[i][:5], model["layers"][i]["k_prefill"])
        tok = oracle.argmax(got)
