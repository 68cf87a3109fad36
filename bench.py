#!/usr/bin/env python3
"""Benchmark of the MI355X packed quantized matmul path.

Headline workload (one "step" = one generated token): the full synthetic Qwen35-shaped
decode step at batch 1 -- 28 layers, hidden 2048, 16 query / 4 KV heads of dim 128,
FFN 6144, every linear layer PTQ1 (ternary, 128-weight blocks), RMSNorm, RoPE, binary16
KV cache prefilled to 1024 tokens, tied 151936-token LM head in Q8_0 -- greedy, from
position 1024, one captured HIP graph replayed per token on the library's stream and
timed with HIP events there.  `value` is tokens/s.

The roofline entry is the step's dominant kernel: launch families that run the same
kernel instantiation are summed (q/k/v and o share one), and the kernel with the largest
time per step in an eager pass with an event around every launch wins.  Each of its
families is then timed back to back over the 28 layers with HIP events on the library
stream; its algorithmic bytes per launch are the packed weights at native size plus
activations, outputs and KV rows read.

Extras: the per-family breakdown of a step, the Q2_K FFN decode step (with its slowest
kernel, the down projection, as its own roofline), the batch-1 matvec sweep, skinny
batches, the prefill GEMM, and the CPU baselines (the oracle, a scalar C restatement of
the reference's CPU kernels, on the host's cores) for every workload.

Prints ONE JSON line on rank 0 (the only rank: this build runs on one GPU).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "prism-inference_amd"))

import numpy as np  # noqa: E402

import hiprt  # noqa: E402
import prism_hip as ph  # noqa: E402
import synth  # noqa: E402

METRIC = "packed matvec HBM GB/s (% peak); prefill int8 TOPS; decode tokens/s at batch 1"
PEAK_HBM = 8.0e12  # MI355X HBM3E, bytes/s
PEAK_I8 = 5.0e15  # MI355X dense int8 MFMA, ops/s
PEAK_F16 = 2.5e15  # MI355X dense f16 MFMA, flop/s
ROTATE_BYTES = 1 << 30
HIDDEN, FFN = 2048, 6144
CPU_THREADS = 16  # the host-core share of one GPU on the measurement box
DECODE_POS = 1024
# Prefill GEMM VALU-issue ceiling: per wavefront and 128-deep block of 32 rows x 64
# tokens, the counted instruction mix is 399 VALU instructions (17 of them MFMA), and a
# SIMD issues one wave64 VALU instruction per 4 cycles (profiles/prefill_gemm_6144x2048.md).
PREFILL_VALU_PER_BLOCK = 399
PREFILL_OPS_PER_BLOCK = 2 * 32 * 64 * 128
ENGINE_HZ = 2.4e9
CUS = 256
# HBM traffic of the decode step's dominant kernel, per dispatch of each launch family:
# rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (KiB as counted) over eager decode steps, and
# the bytes one counted KiB stands for in a plain 256 MiB device copy
# (profiles/decode_projection_traffic.md).
DECODE_TRAFFIC_KIB = {"qkv": (833.0, 12.0), "o": (581.1, 8.0)}
COPY_FETCH_BYTES_PER_KIB, COPY_WRITE_BYTES_PER_KIB = 2047.81, 1024.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_info() -> dict:
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return {"nproc": os.cpu_count(), "cores_available": avail, "cpu_model": model}


def cpu_threads() -> int:
    return max(1, min(CPU_THREADS, host_info()["cores_available"]))


def chunk_for(k: int) -> int:
    for c in (8, 4, 2, 1):
        if k % c == 0:
            return c
    return 1


class Rotation:
    """`copies` context-owned device copies of one packed tensor (identical bytes, distinct
    addresses), each stored in the library's tiled layout."""

    def __init__(self, ctx: ph.Context, kind: int, rows: int, cols: int, data: np.ndarray, copies: int):
        self.nbytes = data.size
        src = hiprt.DeviceBuffer.from_numpy(data)
        self.ids = [ctx.weight_from_device(kind, cols, rows, src) for _ in range(copies)]
        src.free()

    def release(self, ctx: ph.Context):
        for wid in self.ids:
            ctx.release(wid)
        self.ids = []


# ---- headline: the 28-layer decode step ---------------------------------------------

def decode_token_bytes(g: dict, pos: int) -> int:
    """Algorithmic bytes of one decode step at position `pos`: every packed weight at
    its native size once (PTQ1 linears, the Q8_0 LM head), the binary16 K and V rows
    attention reads (pos + 1 tokens per layer), and the embedding row."""
    H, F, D = g["hidden"], g["ffn"], g["head_dim"]
    QW, KW = g["heads"] * D, g["kv_heads"] * D

    def ptq1(rows, cols):
        return rows * cols // 128 * 28

    layer = ptq1(QW + 2 * KW, H) + ptq1(H, QW) + 2 * ptq1(F, H) + ptq1(H, F)
    kv = 2 * (pos + 1) * KW * 2
    return g["layers"] * (layer + kv) + g["vocab"] * H // 32 * 34 + H // 32 * 34


def bench_decode(ctx: ph.Context, model: dict, steps: int, warmup: int, profile: bool = True):
    """Greedy generation of `steps` tokens from position 1024 (KV caches prefilled with
    1024 tokens), one captured HIP graph per step, after `warmup` untimed tokens; then
    an eager pass with an event around every launch (per-family breakdown) and the
    dominant kernel's families timed back to back."""
    g = model["geometry"]
    dec = ph.Decoder(ctx, model, max_steps=max(steps, warmup, 8))
    if warmup:
        dec.generate(1, DECODE_POS, warmup, graph=True)  # capture and warm
    hiprt.synchronize()
    toks, _, secs = dec.generate(1, DECODE_POS, steps, graph=True)
    hiprt.synchronize()
    nbytes = sum(decode_token_bytes(g, DECODE_POS + i) for i in range(steps))
    out = {"tokens_per_s": steps / secs, "ms_per_token": secs / steps * 1e3, "steps": steps,
           "bytes_per_token": nbytes // steps, "GBps": nbytes / secs / 1e9, "frac_hbm": nbytes / secs / PEAK_HBM,
           "first_tokens": [int(t) for t in toks[:8]]}
    if profile:
        psteps = 4
        fams = dec.profile(1, DECODE_POS, psteps)
        for f in fams:
            f["us_per_launch"] = f["total_us"] / max(1, f["launches"])
            f["us_per_step"] = f["total_us"] / psteps
        out["eager_profile"] = {"steps": psteps, "families": fams,
                                "ms_per_token": sum(f["total_us"] for f in fams) / psteps / 1e3,
                                "note": "launches issued one by one, an event before every launch: each time "
                                        "includes the launch's dispatch gap"}
        # Families that launch the same kernel (the same template instantiation) are one
        # kernel here: the dominant kernel is the one with the most time per step.
        per_kernel = {}
        for f in fams:
            per_kernel.setdefault(FAMILY_KERNEL.get(f["family"], f["family"]), []).append(f)
        kernel, members = max(per_kernel.items(), key=lambda kv: sum(f["us_per_step"] for f in kv[1]))
        dec.generate(1, DECODE_POS, 1, graph=True)  # state at a position inside the cache
        timed = []
        for f in members:
            per_layer = f["family"] not in ("lm_prep", "lm_head", "greedy")
            reps = 8 if per_layer else 40
            us, nb = dec.time_family(f["family"], reps)
            timed.append({"family": f["family"], "avg_launch_us": us, "bytes_per_launch": nb,
                          "launches": reps * (g["layers"] if per_layer else 1)})
        # Every member launches once per layer (or once per step): the kernel's mean launch is
        # the members' mean, and its bytes per launch likewise.
        out["dominant"] = {"kernel": kernel, "families": timed,
                           "us_per_step_eager": sum(f["us_per_step"] for f in members),
                           "avg_launch_us": sum(t["avg_launch_us"] for t in timed) / len(timed),
                           "bytes_per_launch": sum(t["bytes_per_launch"] for t in timed) / len(timed),
                           "launches": sum(t["launches"] for t in timed)}
    dec.close()
    return out


# The kernel each decode launch family runs (csrc/decode.hip, csrc/mv_tiled.hip): q/k/v and o
# are the same instantiation (PTQ1 source, quantizing prologue, one matrix, 8 held values).
FAMILY_KERNEL = {
    "qkv": "k_mv_split<PTQ1 source, quantizing prologue, 1 matrix, 8 held> (q/k/v 3072x2048 with RMSNorm; "
           "o 2048x2048 + residual)",
    "o": "k_mv_split<PTQ1 source, quantizing prologue, 1 matrix, 8 held> (q/k/v 3072x2048 with RMSNorm; "
         "o 2048x2048 + residual)",
    "gate_up": "k_mv_split<PTQ1 source, quantizing prologue + RMSNorm, gate+up, 8 held> (2x 6144x2048, SwiGLU, "
               "Q8_0 blocks out)",
    "down": "k_mv_split<PTQ1 source, prepared Q8_0 blocks, 1 matrix> (down 2048x6144 + residual)",
    "attn_scores": "k_attn_scores (q/k norm, RoPE, KV append, 16 heads x 1025 positions)",
    "attn_values": "k_attn_values (softmax_round_f16 + value sums, 16 heads x 1025 positions)",
    "lm_head": "k_mv_rows<Q8_0> (151936x2048 LM head)",
    "lm_prep": "k_lm_prep (final RMSNorm + Q8_0)",
    "greedy": "k_argmax_embed (greedy choice from the LM head tile maxima, next embedding)",
}


def decode_roofline(d: dict) -> dict:
    dom = d["dominant"]
    t = dom["avg_launch_us"] * 1e-6
    achieved = dom["bytes_per_launch"] / t / 1e9
    fams = [f["family"] for f in dom["families"]]
    traffic = None
    if all(f in DECODE_TRAFFIC_KIB for f in fams):
        traffic = round(sum(DECODE_TRAFFIC_KIB[f][0] * COPY_FETCH_BYTES_PER_KIB +
                            DECODE_TRAFFIC_KIB[f][1] * COPY_WRITE_BYTES_PER_KIB for f in fams) / len(fams))
    return {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
            "frac": round(achieved * 1e9 / PEAK_HBM, 4), "traffic": traffic,
            "traffic_unit": "bytes per launch (mean over the families; counted, not live)", "kernel": dom["kernel"],
            "families": [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in f.items()}
                         for f in dom["families"]],
            "bytes_per_launch": round(dom["bytes_per_launch"]), "avg_launch_us": round(dom["avg_launch_us"], 3),
            "launches_timed": dom["launches"],
            "method": "each launch family of the kernel timed back to back over the 28 layers with HIP events on "
                      "the library stream; mean launch and mean algorithmic bytes over the families"}


# ---- config 1: the Q2_K FFN decode step ------------------------------------------------

def ffn_step_bytes() -> int:
    """Algorithmic HBM bytes of one FFN step: packed weights at native block size, the f32
    input, the f32 SwiGLU vector (written by the first kernel, read by the second) and
    the f32 output."""
    w = 3 * FFN * HIDDEN // 256 * 84
    return w + 4 * HIDDEN + 2 * 4 * FFN + 4 * HIDDEN


def down_bytes() -> int:
    """Algorithmic bytes of the down projection: weights, the f32 SwiGLU vector, output."""
    return HIDDEN * FFN // 256 * 84 + 4 * FFN + 4 * HIDDEN


def bench_ffn(ctx: ph.Context, steps: int = 400, warmup: int = 40):
    per_copy = 3 * FFN * HIDDEN // 256 * 84
    chunk = chunk_for(steps)
    copies = math.ceil(ROTATE_BYTES / per_copy / chunk) * chunk
    log(f"ffn: {copies} weight copies ({copies * per_copy / 2**30:.2f} GiB), graph chunk {chunk}")
    g = Rotation(ctx, ph.KIND_Q2_K, FFN, HIDDEN, synth.q2k_weights(FFN, HIDDEN, seed=101), copies)
    u = Rotation(ctx, ph.KIND_Q2_K, FFN, HIDDEN, synth.q2k_weights(FFN, HIDDEN, seed=102), copies)
    d = Rotation(ctx, ph.KIND_Q2_K, HIDDEN, FFN, synth.q2k_weights(HIDDEN, FFN, seed=103), copies)
    x = hiprt.DeviceBuffer.from_numpy(synth.activations(HIDDEN, seed=104))
    out = hiprt.DeviceBuffer(4 * HIDDEN)
    h = hiprt.DeviceBuffer(4 * FFN)
    stream = ctx.stream()
    ctx.ffn_chain_device(g.ids[0], u.ids[0], d.ids[0], x, None, False, out)  # allocates scratch
    assert ctx.sync() == 0

    def enqueue(j):
        def run():
            for i in range(chunk):
                c = j * chunk + i
                ctx.ffn_chain_device(g.ids[c], u.ids[c], d.ids[c], x, None, False, out, None, stream)
        return run

    graphs = [hiprt.Graph(stream, enqueue(j)) for j in range(copies // chunk)]
    for i in range(max(warmup // chunk, len(graphs))):
        graphs[i % len(graphs)].launch()
    assert ctx.sync() == 0
    e0, e1 = hiprt.Event(), hiprt.Event()
    hiprt.synchronize()
    e0.record(stream)
    for i in range(steps // chunk):
        graphs[i % len(graphs)].launch()
    e1.record(stream)
    e1.synchronize()
    hiprt.synchronize()
    assert ctx.sync() == 0
    y = out.to_numpy(np.float32)
    assert np.isfinite(y).all()
    ms = e0.elapsed_ms(e1) / steps
    del graphs
    # The step's slowest kernel alone: the down projection (SwiGLU vector quantized to
    # Q8_K in its prologue), back-to-back launches over the rotated copies.
    ctx.ffn_chain_device(g.ids[0], u.ids[0], 0, x, None, False, h, None, stream)
    for i in range(min(copies, 16)):
        ctx.project_device(d.ids[i], ph.PATH_F32, h, 1, False, out, stream)
    assert ctx.sync() == 0
    launches = 400
    e0.record(stream)
    for i in range(launches):
        ctx.project_device(d.ids[i % copies], ph.PATH_F32, h, 1, False, out, stream)
    e1.record(stream)
    e1.synchronize()
    assert ctx.sync() == 0
    t = e0.elapsed_ms(e1) / launches * 1e-3
    for r in (g, u, d):
        r.release(ctx)
    nbytes = ffn_step_bytes()
    return {"workload": "Qwen35-shaped dense FFN decode step, batch 1: Q2_K gate/up 2048->6144, SwiGLU, "
                        "down 6144->2048, source contract, weights rotated over >= 1 GiB of copies",
            "us_per_step": ms * 1e3, "bytes_per_step": nbytes, "GBps": nbytes / (ms * 1e-3) / 1e9,
            "frac_hbm": nbytes / (ms * 1e-3) / PEAK_HBM, "weight_copies": copies,
            "roofline": {"bound": "hbm", "kernel": "k_mv_split<Q2K, quantizing prologue, 1 matrix, 16 held> "
                                                   "(down 2048x6144)",
                         "avg_launch_us": t * 1e6, "bytes_per_launch": down_bytes(),
                         "achieved": down_bytes() / t / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                         "frac": down_bytes() / t / PEAK_HBM}}


def calibrate_copy(nbytes: int = 256 << 20, reps: int = 10) -> int:
    """A plain device-to-device copy of known size, for scaling FETCH_SIZE / WRITE_SIZE."""
    a, b = hiprt.DeviceBuffer(nbytes), hiprt.DeviceBuffer(nbytes)
    for _ in range(reps):
        hiprt.copy_d2d(b.ptr, a.ptr, nbytes)
    hiprt.synchronize()
    print(json.dumps({"calibrate_copy_bytes": nbytes, "reps": reps}), flush=True)
    return 0


def bench_launch_floor(ctx: ph.Context, launches: int = 400) -> dict:
    """The smallest kernel of the library (Q8_0 quantization of one 32-value block, one
    wavefront), launched back to back on the library stream and timed with HIP events:
    eagerly as the matvec extras are, and replayed from a captured HIP graph.  What a
    dependent launch costs before any work."""
    x = hiprt.DeviceBuffer.from_numpy(synth.activations(32, seed=3))
    out = hiprt.DeviceBuffer(40)
    stream = ctx.stream()

    def launch():
        ctx.quantize_q8_device(x, 32, 1, ph.Q8_SOURCE, out, stream)

    def timed(run) -> float:
        e0, e1 = hiprt.Event(), hiprt.Event()
        e0.record(stream)
        run()
        e1.record(stream)
        e1.synchronize()
        assert ctx.sync() == 0
        return e0.elapsed_ms(e1) * 1e3

    for _ in range(8):
        launch()
    assert ctx.sync() == 0
    eager = timed(lambda: [launch() for _ in range(launches)]) / launches
    chunk = 50
    g = hiprt.Graph(stream, lambda: [launch() for _ in range(chunk)])
    g.launch()
    graph = timed(lambda: [g.launch() for _ in range(launches // chunk)]) / (launches // chunk * chunk)
    del g
    return {"kernel": "k_quantize_q8_0 (32 inputs, one wavefront)", "eager_us": eager, "graph_us": graph,
            "launches": launches}


# ---- configs 0 and 4: batch-1 matvec and skinny batches --------------------------------

def bench_matvec_kernel(ctx: ph.Context, kind: int, rows: int, cols: int, launches: int = 200, tokens: int = 1):
    """Per-launch duration of one matvec kernel (prepared Q8_K/Q8_0 activations of `tokens`
    tokens already in HBM), weights rotated over >= 1 GiB: HIP graphs that launch it once
    per weight copy, replayed until at least `launches` launches, bracketed by HIP events on
    the library stream (`avg_us`); the same launches issued one by one from the host
    (`eager_us`, which for small matrices measures the launch path more than the GPU); and
    100 replayed launches of one copy (`warm_single_copy_us`: its weights stay in the MALL
    and L2 when they fit, so this is not an HBM rate).
    tokens > 1 is the skinny batch: each weight byte is read once per launch."""
    w = synth.weights(kind, rows, cols, seed=7)
    copies = max(2, math.ceil(ROTATE_BYTES / w.size))
    rot = Rotation(ctx, kind, rows, cols, w, copies)
    contract = 0 if kind in (ph.KIND_Q2_K, ph.KIND_TQ1_0, ph.KIND_TQ2_0) or (kind == ph.KIND_PQ2 and cols % 256 == 0) else 1
    x = hiprt.DeviceBuffer.from_numpy(synth.activations(cols, seed=8, tokens=tokens))
    if contract == 0:
        act = hiprt.DeviceBuffer(cols // 256 * 292 * tokens)
        ctx.quantize_q8k_device(x, cols, tokens, False, act)
        path, act_bytes = ph.PATH_Q8K, cols // 256 * 292
    else:
        act = hiprt.DeviceBuffer(cols // 32 * 40 * tokens)
        ctx.quantize_q8_device(x, cols, tokens, ph.Q8_SOURCE, act)
        path, act_bytes = ph.PATH_Q8, cols // 32 * 34
    out = hiprt.DeviceBuffer(4 * rows * tokens)
    stream = ctx.stream()
    for i in range(min(copies, 8)):
        ctx.project_device(rot.ids[i], path, act, tokens, False, out, stream)
    assert ctx.sync() == 0

    def timed(run, n) -> float:
        e0, e1 = hiprt.Event(), hiprt.Event()
        e0.record(stream)
        run()
        e1.record(stream)
        e1.synchronize()
        assert ctx.sync() == 0
        return e0.elapsed_ms(e1) / n * 1e-3

    def eager():
        for i in range(launches):
            ctx.project_device(rot.ids[i % copies], path, act, tokens, False, out, stream)

    t_eager = timed(eager, launches)
    # One pass launches every copy once, 100 launches per graph.
    graphs = [hiprt.Graph(stream, lambda ids=rot.ids[g0:g0 + 100]: [
        ctx.project_device(i, path, act, tokens, False, out, stream) for i in ids]) for g0 in range(0, copies, 100)]
    passes = max(1, math.ceil(launches / copies))

    def replay():
        for _ in range(passes):
            for g in graphs:
                g.launch()

    for g in graphs:
        g.launch()
    t = timed(replay, passes * copies)
    del graphs
    # Warm single copy (weights left in the caches by the previous launch), labelled as such:
    # one graph of 100 launches of the first copy.
    warm = hiprt.Graph(stream, lambda: [ctx.project_device(rot.ids[0], path, act, tokens, False, out, stream)
                                        for _ in range(100)])
    warm.launch()
    t_warm = timed(warm.launch, 100)
    del warm
    nbytes = w.size + (act_bytes + 4 * rows) * tokens
    rot.release(ctx)
    return {"kind": kind, "rows": rows, "cols": cols, "tokens": tokens, "bytes_per_launch": int(nbytes),
            "copies": copies, "launches": passes * copies, "avg_us": t * 1e6, "eager_us": t_eager * 1e6,
            "warm_single_copy_us": t_warm * 1e6, "us_per_token": t * 1e6 / tokens, "GBps": nbytes / t / 1e9,
            "frac_hbm": nbytes / t / PEAK_HBM}


# ---- config 2: the tiled prefill GEMM ----------------------------------------------------

def bench_prefill(ctx: ph.Context, M: int, rows: int = 6144, cols: int = 2048, reps: int = 20,
                  pinned: bool = False, kind: int = ph.KIND_PTQ1):
    """The prefill GEMM (quantization prep + GEMM) in the source or the pinned contract."""
    w = synth.weights(kind, rows, cols, seed=9)
    wid = ctx.weight(kind, cols, rows, w)
    X = hiprt.DeviceBuffer.from_numpy(synth.activations(cols, seed=10, tokens=M))
    out = hiprt.DeviceBuffer(4 * rows * M)
    stream = ctx.stream()
    ctx.project_device(wid, ph.PATH_F32, X, M, pinned, out, stream)
    assert ctx.sync() == 0
    e0, e1 = hiprt.Event(), hiprt.Event()
    e0.record(stream)
    for _ in range(reps):
        ctx.project_device(wid, ph.PATH_F32, X, M, pinned, out, stream)
    e1.record(stream)
    e1.synchronize()
    assert ctx.sync() == 0
    t = e0.elapsed_ms(e1) / reps * 1e-3
    ops = 2.0 * M * rows * cols
    ctx.release(wid)
    valu_ceiling = PREFILL_OPS_PER_BLOCK * 4 / (PREFILL_VALU_PER_BLOCK * 4) * CUS * ENGINE_HZ
    r = {"M": M, "contract": "pinned" if pinned else "source", "ms": t * 1e3, "TOPS": ops / t / 1e12,
         "frac_int8_peak": ops / t / PEAK_I8, "frac_f16_peak": ops / t / PEAK_F16}
    if kind != ph.KIND_PTQ1 or (rows, cols) != (6144, 2048):
        r.update(kind=kind, rows=rows, cols=cols)
    elif not pinned:  # the instruction-mix ceiling was counted for the source kernel
        r.update(valu_issue_ceiling_TOPS=valu_ceiling / 1e12, frac_valu_ceiling=ops / t / valu_ceiling)
    return r


# ---- test-backend-ops' MUL_MAT performance cases -------------------------------------

def bench_backend_ops(ctx: ph.Context, rotate_bytes: int = 512 << 20, calls: int = 40) -> list:
    """The reference's MUL_MAT performance cases for the path's formats (test-backend-ops'
    Perf list, tests/upstream_prism/backend-ops-geometries.json, filtered into
    tests/golden/backend-ops-mulmat.json): A [m][k] packed, B [n][k] F32 in HBM, the whole
    op as the reference runs it (src/backend/ops.rs:444-466: the GPU quantizes B in the
    public contract, then the projection), through prism_hip_project_device.  Weights
    rotated over >= rotate_bytes of copies (beyond the 256 MB MALL); `calls` calls issued one
    by one from the host and timed with HIP events on the library stream."""
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "golden",
                           "backend-ops-mulmat.json")) as f:
        perf = json.load(f)["Perf"]
    cases = []
    for e in perf:
        a = e["Arguments"]
        g = (a[0], a[2], a[3], a[4])
        if g not in cases:
            cases.append(g)
    shapes = []
    for kind, m, n, k in cases:
        if (kind, m, k) not in shapes:
            shapes.append((kind, m, k))
    stream = ctx.stream()
    res = []
    for kind, m, k in shapes:
        w = synth.weights(kind, m, k, seed=17)
        copies = max(2, math.ceil(rotate_bytes / w.size))
        rot = Rotation(ctx, kind, m, k, w, copies)
        for n in [c[2] for c in cases if (c[0], c[1], c[3]) == (kind, m, k)]:
            x = hiprt.DeviceBuffer.from_numpy(synth.activations(k, seed=18, tokens=n))
            out = hiprt.DeviceBuffer(4 * m * n)
            for i in range(min(copies, 4)):
                ctx.project_device(rot.ids[i], ph.PATH_F32, x, n, False, out, stream)
            assert ctx.sync() == 0
            e0, e1 = hiprt.Event(), hiprt.Event()
            e0.record(stream)
            for i in range(calls):
                ctx.project_device(rot.ids[i % copies], ph.PATH_F32, x, n, False, out, stream)
            e1.record(stream)
            e1.synchronize()
            assert ctx.sync() == 0
            t = e0.elapsed_ms(e1) / calls * 1e-3
            nbytes = w.size + 4 * k * n + 4 * m * n
            res.append({"type": kind, "m": m, "n": n, "k": k, "us": t * 1e6, "GBps": nbytes / t / 1e9,
                        "TOPS": 2.0 * m * n * k / t / 1e12, "frac_hbm": nbytes / t / PEAK_HBM})
            x.free()
            out.free()
        rot.release(ctx)
    return res


# ---- CPU baselines (the oracle on the host's cores) --------------------------------------

def _time(fn, budget_s: float = 0.0, min_runs: int = 20, warmups: int = 3):
    """Median seconds of at least `min_runs` timed runs after `warmups` untimed ones
    (more runs while the budget lasts), and the number of timed runs."""
    for _ in range(warmups):
        fn()
    times, t0 = [], time.perf_counter()
    while len(times) < min_runs or time.perf_counter() - t0 < budget_s:
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return float(np.median(times)), len(times)


def cpu_baselines(model: dict, budget_s: float = 1.0):
    """The oracle (scalar C restatement of the reference's CPU kernels, rows split evenly
    over threads as CpuThreadPool does, src/backend/threadpool.rs:190-196) on the same
    workloads, at the box's host-core share and at one thread: the median of at least 20
    runs after 3 warmups (the one-thread decode step: of 3 runs after one warmup)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    T = cpu_threads()
    res = {"host": host_info(), "threads": T, "kind": "port", "configs": []}

    def add(name, unit, work, fn, budget=budget_s, sample=""):
        row = {"config": name, "unit": unit, "sample": sample, "statistic": "median"}
        for threads in (T, 1):
            dt, n = _time(lambda: fn(threads), budget)
            row[f"value_{threads}t" if threads == 1 else "value"] = work / dt
            row[f"ms_{threads}t" if threads == 1 else "ms"] = dt * 1e3
            row[f"runs_{threads}t" if threads == 1 else "runs"] = n
        res["configs"].append(row)
        log(f"cpu {name}: {row['value']:.3f} {unit} at {T} threads, {row['value_1t']:.3f} at 1")

    w0 = synth.ptq1_weights(2048, 2048, seed=7)
    x0 = synth.activations(2048, seed=8)
    add("c0 PTQ1 2048x2048 matvec (Q8_0 source)", "GB/s", (w0.size + 2048 // 32 * 34 + 4 * 2048) / 1e9,
        lambda t: oracle.matvec(oracle.KIND_PTQ1, 2048, 2048, w0, x0, False, t))
    wg = synth.q2k_weights(FFN, HIDDEN, seed=101)
    wu = synth.q2k_weights(FFN, HIDDEN, seed=102)
    wd = synth.q2k_weights(HIDDEN, FFN, seed=103)
    x1 = synth.activations(HIDDEN, seed=104)
    add("c1 Q2_K FFN step 2048->6144->2048", "GB/s", ffn_step_bytes() / 1e9,
        lambda t: oracle.ffn(oracle.KIND_Q2_K, HIDDEN, FFN, wg, wu, wd, x1, None, False, t))
    w2 = synth.ptq1_weights(6144, 2048, seed=9)
    X2 = synth.activations(2048, seed=10, tokens=16)
    add("c2 PTQ1 6144x2048 prefill (16 of the M tokens; per-token cost is independent of M)", "Gop/s",
        2.0 * 16 * 6144 * 2048 / 1e9, lambda t: oracle.prefill(oracle.KIND_PTQ1, 2048, 6144, w2, X2, False, t),
        sample="16 tokens per run")
    add("c2 PTQ1 6144x2048 prefill, pinned contract (16 of the M tokens)", "Gop/s",
        2.0 * 16 * 6144 * 2048 / 1e9, lambda t: oracle.prefill(oracle.KIND_PTQ1, 2048, 6144, w2, X2, True, t),
        sample="16 tokens per run")
    for kind, name in ((oracle.KIND_PTQ1, "PTQ1"), (oracle.KIND_Q2_K, "Q2_K"), (oracle.KIND_Q8_0, "Q8_0")):
        w4 = synth.weights(kind, 12288, 4096, seed=7)
        x4 = synth.activations(4096, seed=8)
        act = 4096 // 256 * 292 if kind == oracle.KIND_Q2_K else 4096 // 32 * 34
        add(f"c4 {name} 12288x4096 matvec", "GB/s", (w4.size + act + 4 * 12288) / 1e9,
            lambda t, w4=w4, x4=x4, kind=kind: oracle.matvec(kind, 4096, 12288, w4, x4, False, t))
    # c3: the decode step of the oracle (every projection through the scalar dots).
    od = oracle.Decoder(model, threads=T)
    pos = [DECODE_POS]

    def step(threads):
        od.threads = threads
        oracle.argmax(od.step(1, pos[0]))

    row = {"config": "c3 28-layer decode step", "unit": "tokens/s", "statistic": "median"}
    dt, n = _time(lambda: step(T))
    row.update(value=1.0 / dt, ms=dt * 1e3, runs=n)
    dt1, n1 = _time(lambda: step(1), min_runs=3, warmups=1)
    row.update(value_1t=1.0 / dt1, ms_1t=dt1 * 1e3, runs_1t=n1)
    res["configs"].append(row)
    log(f"cpu c3: {row['value']:.3f} tokens/s at {T} threads, {row['value_1t']:.4f} at 1")
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="decode tokens timed")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode tokens first")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--prefill-only", default="",
                    help="comma-separated token counts, each optionally ':pinned', ':q2k', ':pq2', ':q8', "
                         "':tq1' or ':tq2' (Q2_K, PQ2, Q8_0, TQ1_0 or TQ2_0 weights, else PTQ1) and ':ROWSxCOLS' (else 6144x2048): time only "
                         "the f32 projection of that many tokens (the prefill GEMM where it applies)")
    ap.add_argument("--matvec-only", default="",
                    help="comma-separated kind:rows:cols[:tokens]: time only these matvecs")
    ap.add_argument("--ffn-only", action="store_true", help="time only the Q2_K FFN step")
    ap.add_argument("--floor-only", action="store_true", help="time only the launch floor")
    ap.add_argument("--backend-ops", action="store_true",
                    help="time only test-backend-ops' MUL_MAT performance cases of the path's formats")
    ap.add_argument("--decode-eager", action="store_true",
                    help="time only decode steps launched kernel by kernel (no graph), for kernel traces")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the path would shard by output rows with an all-gather of the outputs)", file=sys.stderr)
        return 2
    if hiprt.device_count() < 1:
        print("bench.py: no HIP device", file=sys.stderr)
        return 1
    if args.calibrate_copy:
        return calibrate_copy()
    ctx = ph.Context(0)
    log(ctx.identity)
    if args.backend_ops:
        for r in bench_backend_ops(ctx):
            print(json.dumps(r), flush=True)
        ctx.close()
        return 0
    if args.prefill_only or args.matvec_only or args.ffn_only or args.floor_only:
        for spec in filter(None, args.prefill_only.split(",")):
            # "2048", "2048:pinned", "2048:q2k", "2048:pinned:pq2", "16:q2k:151936x4096"
            M, *flags = spec.split(":")
            kinds = {"q2k": ph.KIND_Q2_K, "pq2": ph.KIND_PQ2, "q8": ph.KIND_Q8_0, "tq1": ph.KIND_TQ1_0,
                     "tq2": ph.KIND_TQ2_0}
            kind = next((kinds[f] for f in flags if f in kinds), ph.KIND_PTQ1)
            shape = next(([int(v) for v in f.split("x")] for f in flags if "x" in f), [6144, 2048])
            print(json.dumps(bench_prefill(ctx, int(M), rows=shape[0], cols=shape[1], pinned="pinned" in flags,
                                           kind=kind)), flush=True)
        for spec in filter(None, args.matvec_only.split(",")):
            kind, rows, cols, *tok = (int(v) for v in spec.split(":"))
            print(json.dumps(bench_matvec_kernel(ctx, kind, rows, cols, tokens=tok[0] if tok else 1)), flush=True)
        if args.ffn_only:
            print(json.dumps(bench_ffn(ctx)), flush=True)
        if args.floor_only:
            print(json.dumps(bench_launch_floor(ctx)), flush=True)
        ctx.close()
        return 0
    t0 = time.perf_counter()
    model = synth.decoder_model(0)
    log(f"decode model generated in {time.perf_counter() - t0:.1f} s")
    if args.decode_eager:
        dec = ph.Decoder(ctx, model, max_steps=args.steps)
        _, _, secs = dec.generate(1, DECODE_POS, args.steps, graph=False)
        dec.close()
        print(json.dumps({"decode_eager_ms_per_token": secs / args.steps * 1e3}), flush=True)
        ctx.close()
        return 0
    dec = bench_decode(ctx, model, args.steps, args.warmup, profile=True)
    log(f"decode: {dec['ms_per_token']:.3f} ms/token, {dec['tokens_per_s']:.1f} tok/s; dominant kernel "
        f"{dec['dominant']['kernel']} {dec['dominant']['avg_launch_us']:.2f} us/launch")
    extras = {"decode_breakdown": dec["eager_profile"]}
    if not args.no_extras:
        extras["ffn_decode_step"] = bench_ffn(ctx)
        log(f"ffn step: {extras['ffn_decode_step']['us_per_step']:.2f} us")
        extras["matvec"] = []
        for kind, rows, cols in [(ph.KIND_PTQ1, 2048, 2048), (ph.KIND_PQ2, 2048, 2048), (ph.KIND_Q2_K, HIDDEN, FFN),
                                 (ph.KIND_PTQ1, 12288, 4096), (ph.KIND_Q2_K, 12288, 4096), (ph.KIND_Q8_0, 12288, 4096),
                                 (ph.KIND_PTQ1, 151936, 4096), (ph.KIND_Q2_K, 151936, 4096),
                                 (ph.KIND_Q8_0, 151936, 4096), (ph.KIND_TQ1_0, 12288, 4096),
                                 (ph.KIND_TQ2_0, 12288, 4096), (ph.KIND_TQ1_0, 151936, 4096),
                                 (ph.KIND_TQ2_0, 151936, 4096)]:
            r = bench_matvec_kernel(ctx, kind, rows, cols, launches=100)
            log(f"matvec kind={kind} {rows}x{cols}: {r['avg_us']:.2f} us, {r['GBps']:.1f} GB/s")
            extras["matvec"].append(r)
        extras["launch_floor"] = bench_launch_floor(ctx)
        log(f"launch floor: {extras['launch_floor']['eager_us']:.2f} us eager, "
            f"{extras['launch_floor']['graph_us']:.2f} us in a graph")
        extras["skinny_batch"] = []
        for kind, rows, cols in [(ph.KIND_PTQ1, 12288, 4096), (ph.KIND_Q2_K, 12288, 4096), (ph.KIND_Q8_0, 12288, 4096),
                                 (ph.KIND_PTQ1, 151936, 4096), (ph.KIND_Q2_K, 151936, 4096),
                                 (ph.KIND_Q8_0, 151936, 4096)]:
            for B in (4, 16):
                r = bench_matvec_kernel(ctx, kind, rows, cols, launches=50, tokens=B)
                log(f"skinny kind={kind} {rows}x{cols} B={B}: {r['avg_us']:.2f} us "
                    f"({r['us_per_token']:.2f} us/token), {r['GBps']:.1f} GB/s")
                extras["skinny_batch"].append(r)
        extras["prefill_ptq1_6144x2048"] = []
        for pinned in (False, True):
            for M in (128, 512, 2048):
                r = bench_prefill(ctx, M, pinned=pinned)
                log(f"prefill {r['contract']} M={M}: {r['ms']:.3f} ms, {r['TOPS']:.2f} TOPS")
                extras["prefill_ptq1_6144x2048"].append(r)
        extras["prefill_q2k_6144x2048"] = []
        for M in (128, 512, 2048):
            r = bench_prefill(ctx, M, kind=ph.KIND_Q2_K)
            log(f"prefill Q2_K M={M}: {r['ms']:.3f} ms, {r['TOPS']:.2f} TOPS")
            extras["prefill_q2k_6144x2048"].append(r)
    ctx.close()
    cpu = None
    if not args.no_cpu:
        cb = cpu_baselines(model)
        extras["cpu_baselines"] = cb
        c3 = next(r for r in cb["configs"] if r["config"].startswith("c3"))
        cpu = {"value": c3["value"], "unit": "tokens/s", "cores": cb["threads"], "kind": "port",
               "value_1_thread": c3["value_1t"], "nproc": cb["host"]["nproc"],
               "cores_available": cb["host"]["cores_available"], "cpu_model": cb["host"]["cpu_model"],
               "sample": f"median of {c3['runs']} decode steps at {cb['threads']} threads (after 3 warmups) and "
                         f"of {c3['runs_1t']} at one thread (after one) of the scalar C restatement (every "
                         f"projection through the reference's dot order), rows split evenly over the threads"}
    ms = dec["ms_per_token"]
    line = {
        "metric": METRIC,
        "value": round(dec["tokens_per_s"], 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "ternary/int8 x int8 -> int32, f32 chains; f16 KV",
        "data": "synthetic (seeded random-init weights of the stated architecture; KV cache prefilled N(0,1))",
        "config": {"workload": "28-layer synthetic decode step, batch 1, greedy: hidden 2048, 16/4 heads x 128, "
                               "FFN 6144, PTQ1 linears, RMSNorm, RoPE, f16 KV cache prefilled to 1024 tokens, "
                               "tied Q8_0 LM head 151936",
                   "layers": 28, "hidden": HIDDEN, "ffn": FFN, "vocab": 151936, "kv_prefill": DECODE_POS,
                   "bytes_per_token": dec["bytes_per_token"], "GBps": round(dec["GBps"], 1),
                   "frac_hbm_peak": round(dec["frac_hbm"], 4), "first_tokens": dec["first_tokens"]},
        "roofline": decode_roofline(dec),
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
