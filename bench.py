#!/usr/bin/env python3
"""Benchmark of the MI355X packed quantized matmul path.

Headline workload (one "step"): the Qwen35-shaped dense FFN decode step at batch 1
with Q2_K weights -- quantize x (f32 -> Q8_K), gate and up matvecs 2048->6144,
SwiGLU, quantize h, down matvec 6144->2048 -- in the public (source) arithmetic
contract.  It runs as two kernels (gate+up+SwiGLU, down).  Weights are rotated over
>= 1 GiB of distinct device copies so every step streams them from HBM; steps are
captured in HIP graphs on the library's stream and timed with HIP events there.

The roofline entry is the step's dominant kernel, the fused gate+up+SwiGLU launch,
timed with HIP events around back-to-back launches on the same stream.  Its HBM
traffic comes from the rocprof FETCH_SIZE / WRITE_SIZE summaries committed under
profiles/ (scaled by a plain device copy of known size; --calibrate-copy runs it).

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
ROTATE_BYTES = 1 << 30
HIDDEN, FFN = 2048, 6144


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


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


def ffn_step_bytes() -> int:
    """Algorithmic HBM bytes of one FFN step: packed weights at native block size, the f32
    input, the f32 SwiGLU vector (written by the first kernel, read by the second) and
    the f32 output."""
    w = 3 * FFN * HIDDEN // 256 * 84
    return w + 4 * HIDDEN + 2 * 4 * FFN + 4 * HIDDEN


def gateup_bytes() -> int:
    """Algorithmic bytes of the gate+up+SwiGLU kernel: both weight matrices, x, and h."""
    return 2 * FFN * HIDDEN // 256 * 84 + 4 * HIDDEN + 4 * FFN


def bench_ffn(ctx: ph.Context, steps: int, warmup: int):
    per_copy = 3 * FFN * HIDDEN // 256 * 84
    chunk = chunk_for(steps)
    copies = math.ceil(ROTATE_BYTES / per_copy / chunk) * chunk
    log(f"ffn: {copies} weight copies ({copies * per_copy / 2**30:.2f} GiB), graph chunk {chunk}")
    g = Rotation(ctx, ph.KIND_Q2_K, FFN, HIDDEN, synth.q2k_weights(FFN, HIDDEN, seed=101), copies)
    u = Rotation(ctx, ph.KIND_Q2_K, FFN, HIDDEN, synth.q2k_weights(FFN, HIDDEN, seed=102), copies)
    d = Rotation(ctx, ph.KIND_Q2_K, HIDDEN, FFN, synth.q2k_weights(HIDDEN, FFN, seed=103), copies)
    x = hiprt.DeviceBuffer.from_numpy(synth.activations(HIDDEN, seed=104))
    out = hiprt.DeviceBuffer(4 * HIDDEN)
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
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps // chunk):
        graphs[i % len(graphs)].launch()
    e1.record(stream)
    e1.synchronize()
    hiprt.synchronize()
    wall = time.perf_counter() - t0
    rc = ctx.sync()
    assert rc == 0, ctx.last_error
    y = out.to_numpy(np.float32)
    assert np.isfinite(y).all()
    ms = e0.elapsed_ms(e1) / steps
    del graphs
    for r in (g, u, d):
        r.release(ctx)
    return ms, wall / steps * 1e3, copies


def bench_gateup_kernel(ctx: ph.Context, launches: int = 400):
    """The FFN step's dominant kernel alone: gate+up+SwiGLU (x quantized in its prologue),
    back-to-back launches over rotated weight copies, HIP events on the library stream."""
    per_copy = 2 * FFN * HIDDEN // 256 * 84
    copies = math.ceil(ROTATE_BYTES / per_copy)
    g = Rotation(ctx, ph.KIND_Q2_K, FFN, HIDDEN, synth.q2k_weights(FFN, HIDDEN, seed=111), copies)
    u = Rotation(ctx, ph.KIND_Q2_K, FFN, HIDDEN, synth.q2k_weights(FFN, HIDDEN, seed=112), copies)
    x = hiprt.DeviceBuffer.from_numpy(synth.activations(HIDDEN, seed=113))
    h = hiprt.DeviceBuffer(4 * FFN)
    stream = ctx.stream()
    for i in range(min(copies, 16)):
        ctx.ffn_chain_device(g.ids[i], u.ids[i], 0, x, None, False, h, None, stream)
    assert ctx.sync() == 0
    e0, e1 = hiprt.Event(), hiprt.Event()
    e0.record(stream)
    for i in range(launches):
        ctx.ffn_chain_device(g.ids[i % copies], u.ids[i % copies], 0, x, None, False, h, None, stream)
    e1.record(stream)
    e1.synchronize()
    assert ctx.sync() == 0
    t = e0.elapsed_ms(e1) / launches * 1e-3
    g.release(ctx)
    u.release(ctx)
    return {"avg_us": t * 1e6, "bytes_per_launch": gateup_bytes(), "GBps": gateup_bytes() / t / 1e9,
            "copies": copies}


def measured_traffic(name: str):
    """HBM bytes per launch of a kernel from a committed rocprof summary
    (profiles/<name>): lines 'fetch_kib_per_dispatch: X', 'write_kib_per_dispatch: Y',
    'copy_fetch_scale: A', 'copy_write_scale: B' (counter KiB -> bytes of a plain copy).
    None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for line in f:
            if ":" in line:
                k, v = line.split(":", 1)
                try:
                    vals[k.strip().strip("-* `")] = float(v.strip().strip("`"))
                except ValueError:
                    pass
    need = ("fetch_kib_per_dispatch", "write_kib_per_dispatch", "copy_fetch_scale", "copy_write_scale")
    if not all(k in vals for k in need):
        return None
    return vals["fetch_kib_per_dispatch"] * vals["copy_fetch_scale"] + \
        vals["write_kib_per_dispatch"] * vals["copy_write_scale"]


def calibrate_copy(nbytes: int = 256 << 20, reps: int = 10) -> int:
    """A plain device-to-device copy of known size, for scaling FETCH_SIZE / WRITE_SIZE."""
    a, b = hiprt.DeviceBuffer(nbytes), hiprt.DeviceBuffer(nbytes)
    for _ in range(reps):
        hiprt.copy_d2d(b.ptr, a.ptr, nbytes)
    hiprt.synchronize()
    print(json.dumps({"calibrate_copy_bytes": nbytes, "reps": reps}), flush=True)
    return 0


def bench_matvec_kernel(ctx: ph.Context, kind: int, rows: int, cols: int, launches: int = 200, tokens: int = 1):
    """Per-launch duration of one matvec kernel (prepared Q8_K/Q8_0 activations of `tokens`
    tokens already in HBM), bracketed by HIP events on the library stream, weights rotated
    over >= 1 GiB.  tokens > 1 is the skinny batch: each weight byte is read once per launch."""
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
    e0, e1 = hiprt.Event(), hiprt.Event()
    e0.record(stream)
    for i in range(launches):
        ctx.project_device(rot.ids[i % copies], path, act, tokens, False, out, stream)
    e1.record(stream)
    e1.synchronize()
    assert ctx.sync() == 0
    t = e0.elapsed_ms(e1) / launches * 1e-3
    nbytes = w.size + (act_bytes + 4 * rows) * tokens
    rot.release(ctx)
    return {"kind": kind, "rows": rows, "cols": cols, "tokens": tokens, "bytes_per_launch": int(nbytes),
            "copies": copies, "avg_us": t * 1e6, "us_per_token": t * 1e6 / tokens, "GBps": nbytes / t / 1e9,
            "frac_hbm": nbytes / t / PEAK_HBM}


def bench_prefill(ctx: ph.Context, M: int, rows: int = 6144, cols: int = 2048, reps: int = 20):
    w = synth.ptq1_weights(rows, cols, seed=9)
    wid = ctx.weight(ph.KIND_PTQ1, cols, rows, w)
    X = hiprt.DeviceBuffer.from_numpy(synth.activations(cols, seed=10, tokens=M))
    out = hiprt.DeviceBuffer(4 * rows * M)
    stream = ctx.stream()
    ctx.project_device(wid, ph.PATH_F32, X, M, False, out, stream)
    assert ctx.sync() == 0
    e0, e1 = hiprt.Event(), hiprt.Event()
    e0.record(stream)
    for _ in range(reps):
        ctx.project_device(wid, ph.PATH_F32, X, M, False, out, stream)
    e1.record(stream)
    e1.synchronize()
    assert ctx.sync() == 0
    t = e0.elapsed_ms(e1) / reps * 1e-3
    ops = 2.0 * M * rows * cols
    ctx.release(wid)
    return {"M": M, "ms": t * 1e3, "TOPS": ops / t / 1e12, "frac_int8_peak": ops / t / PEAK_I8}


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


def bench_decode(ctx: ph.Context, steps: int = 128, cpu_steps: int = 2, graph: bool = True):
    """The 28-layer synthetic decode step: greedy generation of `steps` tokens from
    position 1024 (KV caches prefilled with 1024 tokens), one captured HIP graph per
    step, timed with HIP events on the library stream; the oracle's step timed beside
    it on the host for `cpu_steps` tokens."""
    t0 = time.perf_counter()
    model = synth.decoder_model(0)
    g = model["geometry"]
    log(f"decode model generated in {time.perf_counter() - t0:.1f} s")
    dec = ph.Decoder(ctx, model, max_steps=steps)
    dec.generate(1, 1024, 8, graph=graph)  # capture and warm
    toks, _, secs = dec.generate(1, 1024, steps, graph=graph)
    dec.close()
    nbytes = sum(decode_token_bytes(g, 1024 + i) for i in range(steps))
    out = {"workload": "28-layer synthetic decode, hidden 2048, 16/4 heads x 128, FFN 6144, PTQ1 linears, "
                       "tied Q8_0 LM head 151936, f16 KV prefilled to 1024, greedy",
           "steps": steps, "graph": graph, "tokens_per_s": steps / secs, "ms_per_token": secs / steps * 1e3,
           "bytes_per_token": nbytes // steps, "GBps": nbytes / secs / 1e9, "frac_hbm": nbytes / secs / PEAK_HBM,
           "first_tokens": [int(t) for t in toks[:8]]}
    if cpu_steps:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle

        threads = min(16, os.cpu_count() or 1)
        od = oracle.Decoder(model, threads=threads)
        tok, cpu_toks, t0 = 1, [], time.perf_counter()
        for i in range(cpu_steps):
            tok = oracle.argmax(od.step(tok, 1024 + i))
            cpu_toks.append(tok)
        dt = (time.perf_counter() - t0) / cpu_steps
        out["cpu_baseline"] = {"tokens_per_s": 1.0 / dt, "cores": threads, "kind": "port",
                               "sample": f"{cpu_steps} decode steps of the scalar C restatement, rows split over "
                                         f"{threads} threads",
                               "same_tokens": cpu_toks == [int(t) for t in toks[:cpu_steps]]}
    return out


def cpu_baseline(budget_s: float = 12.0):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    threads = min(16, os.cpu_count() or 1)
    wg = synth.q2k_weights(FFN, HIDDEN, seed=101)
    wu = synth.q2k_weights(FFN, HIDDEN, seed=102)
    wd = synth.q2k_weights(HIDDEN, FFN, seed=103)
    x = synth.activations(HIDDEN, seed=104)
    oracle.ffn(oracle.KIND_Q2_K, HIDDEN, FFN, wg, wu, wd, x, None, False, threads)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        oracle.ffn(oracle.KIND_Q2_K, HIDDEN, FFN, wg, wu, wd, x, None, False, threads)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return {"value": ffn_step_bytes() / dt / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "ms_per_step": dt * 1e3,
            "sample": f"{n} FFN decode steps (Q2_K 2048->6144->2048, source contract) on one weight copy, "
                      f"scalar C restatement, rows split over {threads} threads"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--prefill-only", default="", help="comma-separated token counts: time only the prefill GEMM")
    ap.add_argument("--matvec-only", default="",
                    help="comma-separated kind:rows:cols[:tokens]: time only these matvecs")
    ap.add_argument("--decode-only", action="store_true", help="time only the 28-layer decode step")
    ap.add_argument("--decode-eager", action="store_true",
                    help="with --decode-only: launch every kernel each step instead of replaying a HIP graph")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the path would shard by output rows, see DESIGN.md)", file=sys.stderr)
        return 2
    if hiprt.device_count() < 1:
        print("bench.py: no HIP device", file=sys.stderr)
        return 1
    if args.calibrate_copy:
        return calibrate_copy()
    ctx = ph.Context(0)
    log(ctx.identity)
    if args.decode_only:
        print(json.dumps(bench_decode(ctx, cpu_steps=0, graph=not args.decode_eager)), flush=True)
        ctx.close()
        return 0
    if args.prefill_only or args.matvec_only:
        for M in filter(None, args.prefill_only.split(",")):
            print(json.dumps(bench_prefill(ctx, int(M))), flush=True)
        for spec in filter(None, args.matvec_only.split(",")):
            kind, rows, cols, *tok = (int(v) for v in spec.split(":"))
            print(json.dumps(bench_matvec_kernel(ctx, kind, rows, cols, tokens=tok[0] if tok else 1)), flush=True)
        ctx.close()
        return 0
    ms, wall_ms, copies = bench_ffn(ctx, args.steps, args.warmup)
    nbytes = ffn_step_bytes()
    value = nbytes / (ms * 1e-3) / 1e9
    log(f"ffn step: {ms * 1e3:.2f} us/step (wall {wall_ms * 1e3:.2f}), {value:.1f} GB/s")
    kern = bench_gateup_kernel(ctx)
    log(f"gate+up+SwiGLU kernel: {kern['avg_us']:.2f} us, {kern['GBps']:.1f} GB/s")
    extras = {}
    if not args.no_extras:
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
        for M in (128, 512, 2048):
            r = bench_prefill(ctx, M)
            log(f"prefill M={M}: {r['ms']:.3f} ms, {r['TOPS']:.2f} TOPS")
            extras["prefill_ptq1_6144x2048"].append(r)
        r = bench_decode(ctx)
        log(f"decode: {r['ms_per_token']:.3f} ms/token, {r['tokens_per_s']:.1f} tok/s, {r['GBps']:.1f} GB/s")
        extras["decode_28_layer"] = r
    cpu = None if args.no_cpu else cpu_baseline()
    if cpu:
        log(f"cpu baseline: {cpu['value']:.2f} GB/s on {cpu['cores']} threads")
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int2xint8->int32, f32 chain",
        "data": "synthetic (seeded; weights rotated over distinct device copies)",
        "config": {"workload": "Qwen35-shaped dense FFN decode step, batch 1: Q2_K gate/up 2048->6144, "
                               "SwiGLU, down 6144->2048, source contract",
                   "hidden": HIDDEN, "ffn": FFN, "format": "Q2_K x Q8_K", "weight_copies": copies,
                   "bytes_per_step": nbytes, "frac_hbm_peak": round(value * 1e9 / PEAK_HBM, 4),
                   "tokens_per_s": round(1e3 / ms, 1)},
        "roofline": {"bound": "hbm", "achieved": round(kern["GBps"], 2), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                     "frac": round(kern["GBps"] * 1e9 / PEAK_HBM, 4),
                     "traffic": measured_traffic("ffn_gateup_traffic.md"),
                     "kernel": "k_mv_split<Q2K, quantizing prologue, gate+up> (FFN gate+up+SwiGLU, 2x 6144x2048 Q2_K)",
                     "bytes_per_launch": kern["bytes_per_launch"], "avg_launch_us": round(kern["avg_us"], 3)},
        "cpu_baseline": cpu,
    }
    if extras:
        line["extras"] = extras
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
