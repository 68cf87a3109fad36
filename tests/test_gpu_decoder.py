"""The resident full-attention decoder (prism_hip_decoder_*) against the oracle's
decode step, with teacher forcing: the oracle replays the tokens the GPU chose.

Parity bar for the full step (logits after 2..28 layers), both per step:
- max |gpu - oracle| over the step's logits <= 1e-3 * max |oracle logit|;
- every logit within 1e-3 of its own magnitude, with an absolute floor of 1e-5 of
  the step's largest logit (a logit near zero carries the error of its neighbours);
and every greedy token equal to the oracle's argmax unless the oracle's two logits
are within the first tolerance of each other.  Source SiLU, softmax exp and RoPE
cos/sin come from different libms (every projection and quantizer is bit-exact), so
bit identity is reported, not required.
"""

import numpy as np
import pytest

import prism_hip as ph
import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3
FLOOR = 1e-5  # absolute floor of the per-logit check, relative to the step's largest logit
THREADS = 16

SMALL = dict(hidden=512, ffn=1024, heads=4, kv_heads=2, vocab=2048, layers=2, max_tokens=96)


@pytest.fixture(scope="module")
def ctx():
    c = ph.Context(0)
    yield c
    c.close()


def check_against_oracle(model, pos, first, toks, logits):
    """Teacher-forced steps against the oracle; returns the number of steps whose
    logits were bit-identical."""
    import oracle

    od = oracle.Decoder(model, threads=THREADS)
    tok = first
    identical = 0
    for i in range(len(toks)):
        ref = od.step(tok, pos + i)
        scale = float(np.abs(ref).max())
        diff = np.abs(logits[i].astype(np.float64) - ref.astype(np.float64))
        err = float(diff.max())
        assert err <= TOL * scale, f"step {i}: max |gpu - oracle| = {err} > {TOL} * {scale}"
        bound = TOL * np.abs(ref.astype(np.float64)) + FLOOR * scale
        worst = int(np.argmax(diff - bound))
        assert diff[worst] <= bound[worst], (f"step {i}: logit {worst}: |gpu - oracle| = {diff[worst]} > "
                                             f"{TOL} * |{ref[worst]}| + {FLOOR} * {scale}")
        want = oracle.argmax(ref)
        if int(toks[i]) != want:
            gap = abs(float(ref[want]) - float(ref[int(toks[i])]))
            assert gap <= TOL * scale, f"step {i}: token {toks[i]} vs oracle {want} (gap {gap})"
        identical += int(np.array_equal(logits[i].view(np.uint32), ref.view(np.uint32)))
        tok = int(toks[i])
    return identical


@pytest.mark.parametrize("seed,prefill", [(1, 40), (2, 0), (3, 1)])
def test_gpu_decoder_small_matches_oracle(ctx, seed, prefill):
    """Two layers, small widths: every step's logits and greedy token; the first
    position in a cache (prefill 0) and a single cached token included."""
    model = synth.decoder_model(seed, kv_prefill=prefill, **SMALL)
    dec = ph.Decoder(ctx, model, max_steps=16)
    try:
        toks, logits, _ = dec.generate(7, prefill, 12, graph=False, logits=True)
    finally:
        dec.close()
    check_against_oracle(model, prefill, 7, toks, logits)


@pytest.mark.parametrize("max_tokens,prefill", [(2500, 2100), (4200, 4000)])
def test_gpu_decoder_long_cache_matches_oracle(ctx, max_tokens, prefill):
    """Caches longer than 2048 positions: the value kernel's four- and eight-score-per-thread
    forms, whose positions past 2048 take their probabilities from LDS."""
    model = synth.decoder_model(8, kv_prefill=prefill, **dict(SMALL, max_tokens=max_tokens))
    dec = ph.Decoder(ctx, model, max_steps=4)
    try:
        toks, logits, _ = dec.generate(3, prefill, 3, graph=True, logits=True)
    finally:
        dec.close()
    check_against_oracle(model, prefill, 3, toks, logits)


def test_gpu_decoder_graph_replay_equals_eager(ctx):
    """The captured graph (position and token read from device memory) gives the same
    bits as launching every kernel each step, on a second generate as well."""
    model = synth.decoder_model(4, kv_prefill=33, **SMALL)
    outs = []
    for graph in (False, True, True):
        dec = ph.Decoder(ctx, model, max_steps=16)
        try:
            toks, logits, _ = dec.generate(11, 33, 9, graph=graph, logits=True)
            if graph:  # a second call replays the same graph from a fresh start
                toks2, logits2, _ = dec.generate(11, 33, 9, graph=True, logits=True)
                assert np.array_equal(toks, toks2)
                assert np.array_equal(logits.view(np.uint32), logits2.view(np.uint32))
        finally:
            dec.close()
        outs.append((toks, logits))
    for toks, logits in outs[1:]:
        assert np.array_equal(toks, outs[0][0])
        assert np.array_equal(logits.view(np.uint32), outs[0][1].view(np.uint32))


def test_gpu_decoder_full_width_matches_oracle(ctx):
    """The workload's widths (hidden 2048, 16/4 heads, FFN 6144, 151936-token LM head
    on the row-tile kernel) with two layers and a 1024-token cache."""
    model = synth.decoder_model(5, kv_prefill=1024, layers=2)
    dec = ph.Decoder(ctx, model, max_steps=4)
    try:
        toks, logits, _ = dec.generate(1, 1024, 3, graph=True, logits=True)
    finally:
        dec.close()
    check_against_oracle(model, 1024, 1, toks, logits)


@pytest.mark.parametrize("graph", [False, True])
def test_gpu_decoder_nan_cached_key_is_refused(ctx, graph):
    """A NaN element in a cached key makes that position's score NaN for the query heads
    of its KV head: softmax_round_f16 refuses it (src/kernels.rs:4431-4462), so the step
    reports NONFINITE and the outputs are zero-filled.  The same decoder then runs a
    clean cache again."""
    model = synth.decoder_model(7, kv_prefill=40, **SMALL)
    layer = model["layers"][1]
    clean = np.array(layer["k_prefill"], np.uint16, copy=True)
    bad = clean.copy()
    bad.reshape(40, -1)[17, 3] = 0x7E00  # binary16 NaN: position 17, KV head 0, dimension 3
    layer["k_prefill"] = bad
    dec = ph.Decoder(ctx, model, max_steps=8)
    try:
        with pytest.raises(ph.PrismError) as ei:
            dec.generate(5, 40, 3, graph=graph, logits=True)
        assert ei.value.code == ph.ERR_NONFINITE
        layer["k_prefill"] = clean
        dec.close()
        dec = ph.Decoder(ctx, model, max_steps=8)
        toks, logits, _ = dec.generate(5, 40, 3, graph=graph, logits=True)
    finally:
        dec.close()
    check_against_oracle(model, 40, 5, toks, logits)


def test_gpu_decoder_rejects_bad_arguments(ctx):
    model = synth.decoder_model(6, kv_prefill=8, **SMALL)
    dec = ph.Decoder(ctx, model, max_steps=4)
    try:
        with pytest.raises(ph.PrismError):
            dec.generate(model["geometry"]["vocab"], 8, 2)  # token out of range
        with pytest.raises(ph.PrismError):
            dec.generate(1, SMALL["max_tokens"] - 1, 2)  # past the cache
        with pytest.raises(ph.PrismError):
            dec.generate(1, 8, 5)  # more steps than max_steps
        toks, _, _ = dec.generate(1, 8, 2)  # still usable
        assert toks.shape == (2,)
    finally:
        dec.close()
    bad = synth.decoder_model(6, kv_prefill=0, **dict(SMALL, layers=1))
    bad["geometry"]["head_dim"] = 64
    with pytest.raises(ph.PrismError):
        ph.Decoder(ctx, bad)
    # The greedy launch reduces at most 4096 tiles of 64 vocabulary rows.
    big = synth.decoder_model(6, kv_prefill=0, **dict(SMALL, layers=1))
    big["geometry"]["vocab"] = 262144 + 1
    with pytest.raises(ph.PrismError):
        ph.Decoder(ctx, big)


def test_gpu_decoder_detects_released_weights(ctx):
    """prism_hip_weight_release_all drops the decoder's tensors too: generate must then
    fail with INVALID_INPUT (not read freed memory), and setting the tensors again makes
    the decoder usable."""
    model = synth.decoder_model(7, kv_prefill=8, **SMALL)
    dec = ph.Decoder(ctx, model, max_steps=4)
    try:
        toks, _, _ = dec.generate(1, 8, 2, graph=True)
        ctx.release_all()
        with pytest.raises(ph.PrismError) as e:
            dec.generate(1, 8, 2, graph=True)
        assert e.value.code == ph.ERR_INVALID_INPUT
        assert not ctx.faulted
        dec.set_weights(model)
        again, _, _ = dec.generate(1, 8, 2, graph=True)
        assert np.array_equal(toks, again)
    finally:
        dec.close()


def test_gpu_decoder_profile_and_family_timing(ctx):
    """The measurement hooks: an eager profile times every launch of every family
    (six per layer, three for the head) and leaves the decoder generating the same bits;
    a family timed back to back reports its algorithmic bytes; 'greedy' (which advances
    the state) and unknown names are rejected."""
    model = synth.decoder_model(5, kv_prefill=20, **SMALL)
    g = model["geometry"]
    dec = ph.Decoder(ctx, model, max_steps=16)
    try:
        toks, logits, _ = dec.generate(3, 20, 4, graph=True, logits=True)
        fams = dec.profile(3, 20, 2)
        names = [f["family"] for f in fams]
        assert names == ["qkv", "attn_scores", "attn_values", "o", "gate_up", "down", "lm_prep", "lm_head", "greedy"]
        for f in fams:
            want = 2 * (g["layers"] if f["family"] in names[:6] else 1)
            assert f["launches"] == want, f
            assert f["total_us"] > 0.0 and f["bytes_per_launch"] > 0, f
        D, H, F = g["head_dim"], g["hidden"], g["ffn"]
        qkv = (g["heads"] + 2 * g["kv_heads"]) * D
        by = {f["family"]: f["bytes_per_launch"] for f in fams}
        assert by["qkv"] == qkv * H // 128 * 28 + 8 * H + 4 * qkv
        # The LM head also writes one (largest logit, first row) pair of 8 bytes per 64-row
        # tile; the greedy launch reads those pairs, the Q8_0 input and the embedding row.
        tiles = (g["vocab"] + 63) // 64
        assert by["lm_head"] == g["vocab"] * (H // 32) * 34 + H // 32 * 34 + 4 * g["vocab"] + 8 * tiles
        assert by["greedy"] == 8 * tiles + H // 32 * 34 + 4 * H
        assert by["gate_up"] == 2 * F * H // 128 * 28 + 8 * H + F // 32 * 34
        toks2, logits2, _ = dec.generate(3, 20, 4, graph=True, logits=True)
        assert np.array_equal(toks, toks2)
        assert np.array_equal(logits.view(np.uint32), logits2.view(np.uint32))
        for fam in ("qkv", "attn_values", "down", "lm_head"):
            us, nb = dec.time_family(fam, 3)
            assert us > 0.0, (fam, us)
            if not fam.startswith("attn"):  # attention bytes grow with the position
                assert nb == by[fam], (fam, nb)
        for bad in ("greedy", "nope"):
            with pytest.raises(ph.PrismError) as e:
                dec.time_family(bad, 1)
            assert e.value.code == ph.ERR_INVALID_INPUT
        toks3, logits3, _ = dec.generate(3, 20, 4, graph=True, logits=True)
        assert np.array_equal(logits.view(np.uint32), logits3.view(np.uint32))
    finally:
        dec.close()


def test_gpu_cancellation_flag():
    """Cancellation (src/runtime.rs:35-60): with a flag registered and clear, a generate
    runs at most two steps ahead of the device and gives the bits of an unthrottled one;
    once the flag is set, projections and generates return PRISM_ERR_CANCELLED with zeroed
    outputs before launching anything (weight uploads still work), and clearing the flag
    restores service."""
    c = ph.Context(0)
    try:
        model = synth.decoder_model(5, kv_prefill=20, **SMALL)
        dec = ph.Decoder(c, model, max_steps=16)
        try:
            ref_toks, ref_logits, _ = dec.generate(3, 20, 10, graph=True, logits=True)
            flag = np.zeros(1, np.int32)
            c.set_cancellation(flag)
            toks, logits, _ = dec.generate(3, 20, 10, graph=True, logits=True)
            assert np.array_equal(toks, ref_toks)
            assert np.array_equal(logits.view(np.uint32), ref_logits.view(np.uint32))
            flag[0] = 1
            cols, rows = 2048, 128
            wid = c.weight(ph.KIND_PTQ1, cols, rows, synth.ptq1_weights(rows, cols, seed=1))
            rc, out = c.project_f32(wid, rows, synth.activations(cols, seed=2), check=False)
            assert rc == ph.ERR_CANCELLED and not out.any()
            with pytest.raises(ph.PrismError) as e:
                dec.generate(3, 20, 10, graph=True)
            assert e.value.code == ph.ERR_CANCELLED
            flag[0] = 0
            toks, _, _ = dec.generate(3, 20, 10, graph=True)
            assert np.array_equal(toks, ref_toks)
            c.set_cancellation(None)
            assert not c.faulted
        finally:
            dec.close()
    finally:
        c.close()
