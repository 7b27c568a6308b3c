#!/usr/bin/env python3
"""Benchmark of the gfx950 hot path on one MI355X: the Q4_K decode GEMV (
4096x4096) and 8B-shaped Q4_K_M decode at bs=1.

A step is one greedy decode token of a random-init 8B-shaped decoder (34 blocks of the
BASELINE configs[1] decode-step linear layers — Q/K/O/gate/up Q4_K, V/down Q6_K, d_model
4096, FFN 12288, 32/8 heads x 128 — plus RMSNorm/RoPE/SwiGLU/residual glue, f16-KV GQA
attention, the Q6_K 131072x4096 output and the on-device argmax), replayed as one HIP graph
with weights and KV resident in HBM. `value` is tokens/s over exactly --steps timed steps.

Also reported on the same line:
  roofline      the metric's GEMV: Q4_K 4096x4096 with x ~ N(0,1), launched back to
                back over the model's 68 distinct Q and O weights (642 MB, beyond the 256 MB
                MALL), timed with HIP events on the backend stream;
  config        the 12288x4096 gate/up-shape GEMV, the C3 prefill GEMMs, a 128-token prefill
                (a short prompt: one chunk over the Q4_K/Q6_K weights), a 2048-token prefill
                (one chunk of the policy's size, over the FP16 weight copies), the C4 attention
                cases and the C5 14B-shaped decoder (512-token prefill, greedy decode);
  cpu_baseline  the CPU oracle (a C++ restatement of the reference's AVX2 CPU kernels) on all
                host cores: greedy decode steps of the same 8B model, resumed from the GPU's
                512-token KV cache, for a bounded time; plus the C1 GEMV and C4 decode attention.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K GEMV GB/s (% HBM peak); 8B-shaped Q4_K_M decode tok/s at bs=1"
HBM_PEAK_GBPS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0

# HBM bytes per launch of the roofline kernel (gh_gemv_q4k_r2_d at 4096x4096), from the two
# rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) over `bench.py --traffic-probe`, each scaled by
# the same counter's reading for a 256 MiB device-to-device copy (profiles/q4k_gemv_c1_4096x4096.txt).
# Re-measure whenever the kernel changes.
ROOFLINE_TRAFFIC_BYTES = 9596715
# Mean traced duration of the same kernel under `rocprofv3 --kernel-trace --stats -- python3
# bench.py --roofline-only` (profiles/q4k_gemv_c1_4096x4096.txt); the tracer's timestamps add
# 0.2-0.6 us per dispatch against the untraced back-to-back period that `achieved` uses
# (profiles/stream_probe_floor_9mb_94mb.txt). Re-measure whenever the kernel changes.
ROOFLINE_TRACED_US = 4.667


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def weight_bytes(shape):
    """Algorithmic weight bytes streamed per decode token (blocks + output; embedding row)."""
    from graph_horizon_amd import synth

    per_block = 0
    for t, fmt in synth.LAYER_FORMATS.items():
        ind, outd = synth.tensor_dims(shape, t)
        per_block += outd * (ind // 256) * (144 if fmt == 12 else 210)
    out = shape.vocab_size * (shape.embedding_length // 256) * 210
    return per_block, shape.block_count * per_block + out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            return next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except Exception:
        return "unknown CPU"


def cpu_baseline(shape, tensors, kv, kv_context, prompt_len, first, seconds):
    """The oracle on every core of the affinity set: greedy decode steps of the bench's 8B model
    resumed from the GPU's KV cache of the prompt (positions < prompt_len), for about `seconds`
    (the oracle's own cache has room for 1024 steps past the prompt); then the C1 GEMV over
    distinct Q/O weights and C4 decode attention at ctx 4096 / 32768. Every figure is the
    median of the timed calls."""
    import oracle as O
    from graph_horizon_amd import synth
    from graph_horizon_amd import _ffi as F

    cores = len(os.sched_getaffinity(0))
    O.lib().gho_set_threads(cores)
    table = {("g", tid) if layer == F.NO_LAYER else (layer, tid): (fmt, data)
             for layer, tid, fmt, data in tensors}
    y = synth.yarn_params(shape)
    cfg = O.ModelCfg(shape.block_count, max(kv_context, 32768), shape.embedding_length,
                     shape.feed_forward_length, shape.head_count, shape.kv_head_count,
                     shape.head_dim, shape.head_dim, shape.vocab_size, 1e-5, O.Yarn(**y))
    cpu_ctx = prompt_len + 1024
    om = O.Model(cfg, table, cpu_ctx)
    om.load_kv(kv[0], kv[1], kv_context, prompt_len)
    tok, pos, times = first, prompt_len, []
    t0 = time.perf_counter()
    while (len(times) < 4 or time.perf_counter() - t0 < seconds) and pos < cpu_ctx:
        ts = time.perf_counter()
        om.token(tok, pos)
        tok = int(np.argmax(om.logits()))
        times.append(time.perf_counter() - ts)
        pos += 1
    steps = len(times)
    dt = float(np.median(times))
    om.close()
    _, per_token = weight_bytes(shape)
    # C1: Q4_K 4096x4096 GEMV over the model's distinct Q and O weights (FP32 out, logits)
    d = shape.embedding_length
    ws = [data for layer, tid, fmt, data in tensors
          if layer != F.NO_LAYER and tid in (F.T_ATTN_Q, F.T_ATTN_OUTPUT)]
    rng = np.random.default_rng(3)
    x16 = O.f16(rng.standard_normal(d).astype(np.float32))
    c1_times, t1 = [], time.perf_counter()
    while len(c1_times) < len(ws) or time.perf_counter() - t1 < 2.0:
        ts = time.perf_counter()
        O.logits(F.FMT_Q4_K, x16, ws[len(c1_times) % len(ws)], d, d)
        c1_times.append(time.perf_counter() - ts)
    c1_s = float(np.median(c1_times))
    c1_bytes = d * (d // 256) * 144 + d * 2 + d * 4
    # C4: decode attention, 32 q / 8 kv heads x 128, f16 KV N(0,1), pos = ctx - 1
    attn = {}
    for ctx in (4096, 32768):
        kc = O.f16(rng.standard_normal(ctx * 8 * 128).astype(np.float32))
        vc = O.f16(rng.standard_normal(ctx * 8 * 128).astype(np.float32))
        q = O.f16(rng.standard_normal(32 * 128).astype(np.float32))
        at, t2 = [], time.perf_counter()
        while len(at) < 3 or time.perf_counter() - t2 < 1.0:
            ts = time.perf_counter()
            O.attention_decode(q, kc, vc, 128, 8, 32, ctx - 1, 0, ctx)
            at.append(time.perf_counter() - ts)
        us = float(np.median(at)) * 1e6
        attn[f"decode_{ctx}"] = {"median_us": round(us, 1), "calls": len(at),
                                 "gbps": round(2 * ctx * 8 * 128 * 2 / (us * 1e-6) / 1e9, 2)}
    model = cpu_model()
    log(f"bench: CPU baseline: {cores} threads ({model}): {1 / dt:.2f} tok/s, C1 "
        f"{c1_bytes / c1_s / 1e9:.1f} GB/s, attention ctx 4096 {attn['decode_4096']['median_us']:.0f} us")
    return {"value": round(1.0 / dt, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"{steps} greedy decode steps of the bench's 8B-shaped model (34 blocks with "
                      f"attention, output GEMV and argmax) at context {prompt_len}..{pos - 1}, "
                      f"resumed from the GPU's prompt KV cache, {sum(times):.1f} s in all: median "
                      f"{dt * 1e3:.1f} ms/token ({per_token / dt / 1e9:.1f} GB/s of weights); "
                      f"{cores} threads (nproc of the affinity set), {model}",
            "q4k_gemv_c1": {"median_us": round(c1_s * 1e6, 1), "gbps": round(c1_bytes / c1_s / 1e9, 2),
                            "calls": len(c1_times)},
            "attention_c4": attn,
            "label": "C++ restatement of the graph_horizon CPU reference (AVX2 kernels)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=512, help="prefilled context before decode")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-c5", action="store_true", help="skip the 14B-shaped decoder (configs[4])")
    ap.add_argument("--launch", choices=("graph", "stream"), default="graph",
                    help="decode steps as one replayed HIP graph (default) or as direct "
                         "stream launches of the same kernels (for kernel tracers)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the roofline GEMV's timed launches (for rocprofv3 --kernel-trace)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch the roofline kernel (4 distinct weights) and a 256 MiB "
                         "device copy of known size, for rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE")
    ap.add_argument("--gemm-probe", action="store_true",
                    help="only the C3 prefill GEMMs (512 tokens, 8 random weights each), for "
                         "rocprofv3 --pmc passes")
    ap.add_argument("--attn-probe", action="store_true",
                    help="only the C4 attention cases (bench.py c4_attention), for rocprofv3 "
                         "--pmc passes")
    ap.add_argument("--floor-probe", action="store_true",
                    help="only plain streaming reads (gh_stream_probe) of --probe-bytes with "
                         "--probe-groups workgroups and the C1 GEMV, back to back over distinct "
                         "memory: the floor of one launch of each size, and (under rocprofv3 "
                         "--kernel-trace) the tracer's per-dispatch cost")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="calibration only: the vendor library's dense FP16 GEMM (torch.matmul, "
                         "hipBLASLt) at the C3 shapes beside this build's dequantizing GEMMs, "
                         "same box, same timing")
    ap.add_argument("--probe-tokens", type=int, default=512,
                    help="token rows of --gemm-probe's GEMMs (512: the C3 shape; 8-128 run the "
                         "128-token tiles)")
    ap.add_argument("--probe-bytes", default="9437184,94371840",
                    help="comma-separated read sizes for --floor-probe")
    ap.add_argument("--probe-groups", default="256,512,1024,2048",
                    help="comma-separated workgroup counts for --floor-probe")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path shards by rows/heads across GPUs only by design).", file=sys.stderr)
        sys.exit(2)

    from graph_horizon_amd import HipBackend, HipModel, synth
    from graph_horizon_amd import _ffi as F

    if args.traffic_probe:
        traffic_probe(synth.SHAPES["8b"])
        return
    if args.gemm_probe:
        gemm_probe(synth.SHAPES["8b"], args.probe_tokens)
        return
    if args.floor_probe:
        floor_probe([int(v) for v in args.probe_bytes.split(",")],
                    [int(v) for v in args.probe_groups.split(",")])
        return
    if args.vendor_gemm:
        vendor_gemm(synth.SHAPES["8b"])
        return
    if args.attn_probe:
        hip = HipBackend(0)
        log(f"bench: attention probe {json.dumps(c4_attention(hip))}")
        hip.close()
        return
    shape = synth.SHAPES["8b"]
    per_block, per_token = weight_bytes(shape)
    kv_context = args.prompt + args.warmup + args.steps + 8
    hip = HipBackend(0)
    flags = F.MODEL_NO_GRAPH if args.launch == "stream" else 0
    model = HipModel(hip, synth.model_config(shape, kv_context, prefill_rows=512, flags=flags))
    t0 = time.perf_counter()
    tensors = list(synth.model_tensors(shape, seed=2024))
    for layer, tid, fmt, data in tensors:
        model.load_tensor(layer, tid, fmt, data)
    log(f"bench: generated and loaded {shape.name} weights in {time.perf_counter() - t0:.1f} s")
    if args.roofline_only:
        log(f"bench: roofline {json.dumps(c1_roofline(hip, model, shape))}")
        return

    rng = np.random.default_rng(7)
    prompt = rng.integers(0, shape.vocab_size, args.prompt).astype(np.uint32)
    # one untimed prefill of the same length first: its first use grows the split-K workspace
    # (a synchronizing allocation) that every later prefill of this length reuses
    model.prefill(prompt, 0)
    hip.synchronize()
    hip.timer_start()
    model.prefill(prompt, 0)
    prefill_ms = hip.timer_stop()
    log(f"bench: prefill {args.prompt} tokens in {prefill_ms:.2f} ms "
        f"({args.prompt / (prefill_ms / 1e3):.0f} tok/s)")
    first = model.read_argmax()
    kv = model.kv()
    n_kv = shape.block_count * kv_context * shape.kv_head_count * shape.head_dim
    kv_host = (hip.download(kv.k, np.uint16, n_kv), hip.download(kv.v, np.uint16, n_kv))
    pos = args.prompt
    tok = first
    if args.warmup:
        out = model.decode_greedy(tok, pos, args.warmup)
        tok, pos = int(out[-1]), pos + args.warmup
    hip.synchronize()
    hip.timer_start()
    toks = model.decode_greedy(tok, pos, args.steps)
    ms = hip.timer_stop()
    tok_s = args.steps / (ms / 1e3)
    log(f"bench: {args.steps} decode steps in {ms:.2f} ms -> {tok_s:.1f} tok/s")
    merge_ab = xcd_merge_ab(hip, model, tok, pos, args.steps, args.warmup, toks, tok_s)

    roofline = c1_roofline(hip, model, shape)
    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random-init Q4_K_M weights, random prompt ids)",
        "config": {
            "workload": f"8b-shaped Q4_K_M decoder, greedy decode bs=1 ({shape.block_count} "
                        f"blocks of BASELINE configs[1]: d {shape.embedding_length}, FFN "
                        f"{shape.feed_forward_length}, 32/8 heads x 128, Q/K/O/gate/up Q4_K, "
                        f"V/down Q6_K; Q6_K output {shape.vocab_size}x{shape.embedding_length}); "
                        f"context {args.prompt}..{pos + args.steps}; {args.launch} launch",
            "weight_bytes_per_token": per_token,
            "prefill": {"tokens": args.prompt, "ms": round(prefill_ms, 3),
                        "tok_s": round(args.prompt / (prefill_ms / 1e3), 1)},
            "decode_weight_roofline_frac": round(per_token * tok_s / (HBM_PEAK_GBPS * 1e9), 4),
            "q4k_gemv_12288x4096": gemv_gate_shape(hip, model, shape),
            "attention_merge_ab": merge_ab,
        },
        "roofline": roofline,
    }
    result["config"]["prefill_gemm_c3"] = prefill_gemm(hip, model, shape, tensors, 512)
    result["config"]["prefill_128"] = prefill_short(hip, model, shape, 128)
    model.close()
    result["config"]["prefill_2048"] = prefill_long(hip, HipModel, shape, tensors, 2048)
    # the same prefills with no FP16 weight copies: the GEMMs dequantize the Q4_K/Q6_K weights
    result["config"]["prefill_dequantizing"] = {
        str(t): prefill_long(hip, HipModel, shape, tensors, t, copies=False) for t in (512, 2048)}
    result["config"]["attention_c4"] = c4_attention(hip)
    if not args.no_c5:
        result["config"]["decoder_c5"] = c5_decoder(hip, HipModel, args.prompt)
    hip.close()
    if not args.no_cpu:
        log("bench: CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(shape, tensors, kv_host, kv_context, args.prompt,
                                              first, args.cpu_seconds)
    print(json.dumps(result), flush=True)


def xcd_merge_ab(hip, model, tok, pos, steps, warmup, toks, tok_s):
    """The same decode steps again with decode attention's split merge through device memory
    instead of one XCD's L2 (same box, same positions): tok/s of both forms, and whether the
    token streams agree (the two merges give the same bits)."""
    if not hip.xcd_count:
        return {"xcds": 0, "note": "dispatch placement not confirmed: device-memory merge only"}
    hip.set_attention_xcd_merge(False)
    try:
        model.decode_greedy(tok, pos, max(warmup, 1))  # records the graphs again
        hip.synchronize()
        hip.timer_start()
        other = model.decode_greedy(tok, pos, steps)
        ms = hip.timer_stop()
    finally:
        hip.set_attention_xcd_merge(True)
    ab = {"xcds": hip.xcd_count, "xcd_local_tok_s": round(tok_s, 2),
          "device_memory_tok_s": round(steps / (ms / 1e3), 2),
          "same_tokens": bool(np.array_equal(toks, other))}
    log(f"bench: attention merge A/B {json.dumps(ab)}")
    return ab


def model_weight(model, layer, tid):
    """The device handle of one model weight (read from the driver's tensor table)."""
    import ctypes as C

    from graph_horizon_amd import _ffi as F

    buf = F.GhBuf()
    rc = model.b.lib.gh_model_weight(model.h, layer, tid, C.byref(buf))
    assert rc == 0, rc
    return buf


def time_gemv(hip, weights, x, y, in_dim, out_dim, reps=3, each=False):
    """gh_matmul launches over `weights` (warm-up pass first), timed with HIP events on the
    backend stream. Returns the average microseconds per launch of back-to-back launches (the
    period, launch gaps included) and, with each=True, of launches bracketed one by one by
    their own event pair (the dispatch's duration, as a kernel tracer reports it)."""
    import ctypes as C

    lib = hip.lib
    enc = hip.begin()
    for w in weights[:4]:
        lib.gh_matmul(hip.h, enc, C.byref(y), C.byref(x), C.byref(w), in_dim, out_dim)
    hip.submit()
    enc = hip.begin()
    hip.timer_start()
    for _ in range(reps):
        for w in weights:
            lib.gh_matmul(hip.h, enc, C.byref(y), C.byref(x), C.byref(w), in_dim, out_dim)
    period = hip.timer_stop() * 1e3 / (reps * len(weights))
    hip.submit()
    if not each:
        return period, None
    total = 0.0
    for _ in range(reps):
        for w in weights:
            enc = hip.begin()
            hip.timer_start()
            lib.gh_matmul(hip.h, enc, C.byref(y), C.byref(x), C.byref(w), in_dim, out_dim)
            total += hip.timer_stop()
            hip.submit()
    return period, total * 1e3 / (reps * len(weights))


def c1_roofline(hip, model, shape):
    """The metric's GEMV: Q4_K 4096x4096, x ~ N(0,1) in FP16, one token,
    over the model's 68 distinct 4096x4096 Q4_K weights (Q and O of 34 blocks, 642 MB)."""
    from graph_horizon_amd import _ffi as F
    from graph_horizon_amd import synth

    d = shape.embedding_length
    ws = [model_weight(model, li, t) for li in range(shape.block_count)
          for t in (F.T_ATTN_Q, F.T_ATTN_OUTPUT)]
    x = hip.from_host(synth.f16_bits(np.random.default_rng(11).standard_normal(d)))
    y = hip.alloc_buffer(d * 2)
    period, single = time_gemv(hip, ws, x, y, d, d, each=True)
    nbytes = d * (d // 256) * 144 + d * 2 + d * 2
    gbps = nbytes / (period * 1e-6) / 1e9
    hip.free_buffer(x)
    hip.free_buffer(y)
    log(f"bench: Q4_K GEMV {d}x{d} (C1): {period:.3f} us per launch back to back, {gbps:.0f} GB/s "
        f"({gbps / HBM_PEAK_GBPS:.1%}); one launch between its own event pair {single:.3f} us")
    return {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": ROOFLINE_TRAFFIC_BYTES,
            "kernel": f"gh_gemv_q4k_r2_d (Q4_K GEMV {d}x{d}, BASELINE configs[0], x ~ N(0,1); "
                      f"{nbytes} algorithmic B/launch: weights {d * (d // 256) * 144} + x + y)",
            "avg_us": round(period, 3), "single_launch_us": round(single, 3),
            "traced_avg_us": ROOFLINE_TRACED_US,
            "traced_frac": round(nbytes / (ROOFLINE_TRACED_US * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
            "launches": 3 * len(ws), "distinct_weights": len(ws),
            "timing": "avg_us: HIP events on the backend stream around back-to-back launches "
                      "(launch gaps included), per launch; single_launch_us: one launch on an "
                      "idle GPU between its own event pair (dispatch ramp and event markers "
                      "included); traced_avg_us: the kernel trace's mean per-dispatch duration "
                      "of the same command (profiles/q4k_gemv_c1_4096x4096.txt), which the "
                      "tracer's timestamps lengthen"}


def gemv_gate_shape(hip, model, shape):
    """The decode GEMV at the FFN gate/up shape (12288x4096) over the 68 distinct gate/up
    weights of the model (1.9 GB)."""
    from graph_horizon_amd import _ffi as F
    from graph_horizon_amd import synth

    d, ffn = shape.embedding_length, shape.feed_forward_length
    ws = [model_weight(model, li, t) for li in range(shape.block_count)
          for t in (F.T_FFN_GATE, F.T_FFN_UP)]
    x = hip.from_host(synth.f16_bits(np.random.default_rng(12).standard_normal(d)))
    y = hip.alloc_buffer(ffn * 2)
    us, _ = time_gemv(hip, ws, x, y, d, ffn)
    nbytes = ffn * (d // 256) * 144 + d * 2 + ffn * 2
    gbps = nbytes / (us * 1e-6) / 1e9
    hip.free_buffer(x)
    hip.free_buffer(y)
    log(f"bench: Q4_K GEMV {ffn}x{d}: {us:.2f} us, {gbps:.0f} GB/s")
    return {"avg_us": round(us, 3), "gbps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "bytes_per_launch": nbytes, "kernel": "gh_gemv_q4k_r1_d"}


def traffic_probe(shape):
    """Roofline kernel launches plus a copy of known size, nothing else (for PMC passes)."""
    import ctypes as C

    from graph_horizon_amd import HipBackend, synth

    hip = HipBackend(0)
    d = shape.embedding_length
    rng = np.random.default_rng(5)
    ws = [hip.load_weight(12, synth.quant_blocks(rng, 12, d, d, 0.02), d, d) for _ in range(4)]
    xb = hip.from_host(synth.f16_bits(rng.standard_normal(d)))
    yb = hip.alloc_buffer(d * 2)
    enc = hip.begin()
    for w in ws:
        hip.lib.gh_matmul(hip.h, enc, C.byref(yb), C.byref(xb), C.byref(w), d, d)
    hip.submit()
    rt = C.CDLL("libamdhip64.so")
    nbytes = 256 << 20
    src, dst = C.c_void_p(), C.c_void_p()
    assert rt.hipMalloc(C.byref(src), C.c_size_t(nbytes)) == 0
    assert rt.hipMalloc(C.byref(dst), C.c_size_t(nbytes)) == 0
    assert rt.hipMemset(src, 1, C.c_size_t(nbytes)) == 0
    for _ in range(2):  # device-to-device: the runtime's blit copy kernel
        assert rt.hipMemcpy(dst, src, C.c_size_t(nbytes), 3) == 0
    assert rt.hipDeviceSynchronize() == 0
    log(f"bench: traffic probe: 4 x gh_matmul {d}x{d} ({d * (d // 256) * 144} B of weights "
        f"each), 2 x copy of {nbytes} B")
    rt.hipFree(src)
    rt.hipFree(dst)
    hip.close()


def floor_probe(sizes, groups, launches=240):
    """Back-to-back plain streaming reads (gh_stream_probe) of each size over distinct offsets
    of a 1 GiB buffer (so the 256 MB MALL cannot serve them), for each workgroup count, then the
    C1 GEMV (gh_gemv_q4k_r2_d, 4096x4096) over 64 distinct random weights (604 MB). Prints the
    HIP-event period per launch of each case (launch gaps included): the untraced figures that
    a kernel trace of the same command is compared with."""
    import ctypes as C

    from graph_horizon_amd import HipBackend, synth

    hip = HipBackend(0)
    lib = hip.lib
    span = 1 << 30
    src, sink = hip.alloc_buffer(span), hip.alloc_buffer(4096)
    out = {"stream": []}
    for nbytes in sizes:
        stride = (nbytes + 4095) // 4096 * 4096
        slots = max(4, (span - nbytes) // stride + 1)
        for g in groups:
            enc = hip.begin()
            for i in range(8):
                lib.gh_stream_probe(hip.h, enc, C.byref(src), (i % slots) * stride, nbytes, C.byref(sink), g)
            hip.submit()
            enc = hip.begin()
            hip.timer_start()
            for i in range(launches):
                rc = lib.gh_stream_probe(hip.h, enc, C.byref(src), (i % slots) * stride, nbytes,
                                         C.byref(sink), g)
                assert rc == 0, rc
            us = hip.timer_stop() * 1e3 / launches
            hip.submit()
            gbps = nbytes / (us * 1e-6) / 1e9
            out["stream"].append({"bytes": nbytes, "workgroups": g, "period_us": round(us, 3),
                                  "gbps": round(gbps, 1), "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4)})
            log(f"bench: stream probe {nbytes} B, {g} workgroups: {us:.3f} us per launch back to "
                f"back ({gbps:.0f} GB/s, {gbps / HBM_PEAK_GBPS:.1%}), {slots} distinct offsets")
    hip.free_buffer(src)
    d = 4096
    rng = np.random.default_rng(5)
    ws = [hip.load_weight(12, synth.quant_blocks(rng, 12, d, d, 0.02), d, d) for _ in range(64)]
    x = hip.from_host(synth.f16_bits(rng.standard_normal(d)))
    y = hip.alloc_buffer(d * 2)
    period, _ = time_gemv(hip, ws, x, y, d, d, reps=4)
    nbytes = d * (d // 256) * 144 + d * 2 + d * 2
    gbps = nbytes / (period * 1e-6) / 1e9
    out["c1_gemv"] = {"kernel": "gh_gemv_q4k_r2_d", "bytes": nbytes, "period_us": round(period, 3),
                      "gbps": round(gbps, 1), "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4),
                      "launches": 4 * len(ws)}
    log(f"bench: C1 GEMV 4096x4096 over 64 distinct weights: {period:.3f} us per launch back to "
        f"back ({gbps:.0f} GB/s, {gbps / HBM_PEAK_GBPS:.1%})")
    print(json.dumps({"floor_probe": out}), flush=True)
    for b in ws + [x, y, sink]:
        hip.free_buffer(b)
    hip.close()


def gemm_probe(shape, n=512):
    """The C3 prefill GEMMs alone: gate/up (Q4_K d -> FFN) then down (Q6_K FFN -> d) over 8
    random weights each, 4 passes, nothing else (for PMC passes)."""
    import ctypes as C

    from graph_horizon_amd import HipBackend, synth

    hip = HipBackend(0)
    d, ffn = shape.embedding_length, shape.feed_forward_length
    rng = np.random.default_rng(3)
    y = hip.alloc_buffer(n * ffn * 2)
    for fmt, ind, outd in ((12, d, ffn), (14, ffn, d)):
        ws = [hip.load_weight(fmt, synth.quant_blocks(rng, fmt, outd, ind, synth.model_d_std(ind)), ind, outd)
              for _ in range(8)]
        a = hip.from_host(synth.f16_bits(rng.standard_normal(n * ind) * 0.5))
        enc = hip.begin()
        for _ in range(4):
            for w in ws:
                hip.lib.gh_matmul_batched(hip.h, enc, C.byref(y), C.byref(a), C.byref(w), ind, outd, n)
        hip.submit()
        hip.synchronize()
        for b in ws + [a]:
            hip.free_buffer(b)
    log(f"bench: gemm probe: 32 x {n}x{d}->{ffn} Q4_K, 32 x {n}x{ffn}->{d} Q6_K")
    hip.close()


def vendor_gemm(shape, sizes=(128, 512, 2048), reps=6):
    """Calibration for the C3 GEMMs: what the vendor library reaches on this chip at the same
    shapes. torch.matmul over dense FP16 weights (hipBLASLt; FP16 in, FP32 accumulation, FP16
    out) and this build's GEMMs over Q4_K (gate/up, d -> FFN) and Q6_K (down, FFN -> d) weights
    that they dequantize tile by tile, each over 8 distinct weights (more bytes than the MALL
    holds), timed back to back with events on the stream each is launched on. The vendor figure
    is a ceiling for the arithmetic at these shapes, not the C3 workload (it reads FP16 weights,
    3.6x the Q4_K bytes)."""
    import ctypes as C

    import torch

    from graph_horizon_amd import HipBackend, synth

    dev = torch.device("cuda", 0)
    hip = HipBackend(0)
    d, ffn = shape.embedding_length, shape.feed_forward_length
    rng = np.random.default_rng(3)
    out = {"vendor": [], "own": []}
    for name, fmt, ind, outd in (("gate_up", 12, d, ffn), ("down", 14, ffn, d)):
        # operands made on the host and copied over: the calibration runs no torch kernel of its
        # own on the device, only the library GEMM
        g = torch.Generator().manual_seed(ind)
        tw = [(torch.randn(ind, outd, generator=g) * 0.02).half().to(dev) for _ in range(8)]
        ws = [hip.load_weight(fmt, synth.quant_blocks(rng, fmt, outd, ind, synth.model_d_std(ind)), ind, outd)
              for _ in range(8)]
        for n in sizes:
            fl = 2.0 * n * ind * outd
            tx = torch.randn(n, ind, generator=g).half().to(dev)
            for w in tw:
                torch.matmul(tx, w)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                for w in tw:
                    torch.matmul(tx, w)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (reps * len(tw))
            tf = fl / (us * 1e-6) / 1e12
            out["vendor"].append({"gemm": name, "shape": f"{n}x{ind}->{outd}", "avg_us": round(us, 2),
                                  "tflops": round(tf, 1), "frac_f16_mfma_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4)})
            log(f"bench: vendor FP16 GEMM {name} {n}x{ind}->{outd}: {us:.1f} us, {tf:.0f} TFLOP/s "
                f"({tf / MFMA_F16_PEAK_TFLOPS:.1%})")
            del tx
            a = hip.from_host(synth_f16(rng, n * ind))
            y = hip.alloc_buffer(n * outd * 2)
            enc = hip.begin()
            for w in ws:
                hip.lib.gh_matmul_batched(hip.h, enc, C.byref(y), C.byref(a), C.byref(w), ind, outd, n)
            hip.submit()
            enc = hip.begin()
            hip.timer_start()
            for _ in range(reps):
                for w in ws:
                    hip.lib.gh_matmul_batched(hip.h, enc, C.byref(y), C.byref(a), C.byref(w), ind, outd, n)
            us = hip.timer_stop() * 1e3 / (reps * len(ws))
            hip.submit()
            tf = fl / (us * 1e-6) / 1e12
            out["own"].append({"gemm": name, "fmt": "Q4_K" if fmt == 12 else "Q6_K", "shape": f"{n}x{ind}->{outd}",
                               "avg_us": round(us, 2), "tflops": round(tf, 1),
                               "frac_f16_mfma_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4)})
            log(f"bench: dequantizing GEMM {name} {n}x{ind}->{outd}: {us:.1f} us, {tf:.0f} TFLOP/s "
                f"({tf / MFMA_F16_PEAK_TFLOPS:.1%})")
            hip.free_buffer(a)
            hip.free_buffer(y)
        for w in ws:
            hip.free_buffer(w)
        del tw
        torch.cuda.empty_cache()
    print(json.dumps({"vendor_gemm": out}), flush=True)
    hip.close()


def prefill_short(hip, model, shape, n):
    """A short prompt (one chunk of n <= 128 rows: the 128-token GEMM tiles over the Q4_K/Q6_K
    weights, no FP16 copies) at position 0 of the bench's model, after its decode leg: the
    median of three timed prefills after an untimed one."""
    prompt = np.random.default_rng(13).integers(0, shape.vocab_size, n).astype(np.uint32)
    model.prefill(prompt, 0)
    times = []
    for _ in range(3):
        hip.synchronize()
        hip.timer_start()
        model.prefill(prompt, 0)
        times.append(hip.timer_stop())
    ms = float(np.median(times))
    log(f"bench: prefill {n} tokens (short prompt) in {ms:.3f} ms ({n / (ms / 1e3):.0f} tok/s)")
    return {"tokens": n, "ms": round(ms, 3), "tok_s": round(n / (ms / 1e3), 1), "fp16_weight_copies": False}


def prefill_long(hip, HipModel, shape, tensors, n, copies=True):
    """A long prompt through the prefill policy's 2048-row chunks: the same 8B-shaped weights in
    a model of n positions, one n-token chunk. Its first prefill (untimed) also makes the FP16
    copies of the layer matrices that the prefill GEMMs read (copies=False: the model keeps
    none, GH_MODEL_NO_F16_WEIGHTS, and the GEMMs dequantize the Q4_K/Q6_K weights tile by
    tile); the second is timed."""
    from graph_horizon_amd import _ffi as F
    from graph_horizon_amd import synth

    flags = 0 if copies else F.MODEL_NO_F16_WEIGHTS
    model = HipModel(hip, synth.model_config(shape, n, prefill_rows=n, flags=flags))
    for layer, tid, fmt, data in tensors:
        model.load_tensor(layer, tid, fmt, data)
    prompt = np.random.default_rng(11).integers(0, shape.vocab_size, n).astype(np.uint32)
    model.prefill(prompt, 0)
    hip.synchronize()
    hip.timer_start()
    model.prefill(prompt, 0)
    ms = hip.timer_stop()
    model.close()
    log(f"bench: prefill {n} tokens (one chunk{'' if copies else ', dequantizing'}) in {ms:.2f} ms "
        f"({n / (ms / 1e3):.0f} tok/s)")
    return {"tokens": n, "chunk_rows": n, "ms": round(ms, 3), "tok_s": round(n / (ms / 1e3), 1),
            "fp16_weight_copies": copies}


def prefill_gemm(hip, model, shape, tensors, n):
    """the n-token prefill GEMMs (gate/up Q4_K d->FFN, down Q6_K FFN->d) on
    the matrix cores, over 8 distinct layers' weights, timed with HIP events. The top-level
    figures are the C3 workload itself: Q4_K/Q6_K weights loaded without FP16 copies, which the
    GEMMs dequantize tile by tile. Beside them, the same GEMMs over the FP16 copies the model's
    prefill made (same output bits; their HBM cost is stated)."""
    import ctypes as C

    from graph_horizon_amd import _ffi as F
    from graph_horizon_amd import synth

    d, ffn = shape.embedding_length, shape.feed_forward_length
    rng = np.random.default_rng(11)
    a_d = hip.from_host(synth_f16(rng, n * d))
    a_f = hip.from_host(synth_f16(rng, n * ffn))
    y = hip.alloc_buffer(n * max(d, ffn) * 2)
    layers = min(8, shape.block_count)
    host = {(layer, tid): (fmt, data) for layer, tid, fmt, data in tensors
            if layer < layers and tid in (F.T_FFN_GATE, F.T_FFN_DOWN)}

    def timed(name, ws, ind, outd, a):
        enc = hip.begin()
        hip.lib.gh_matmul_batched(hip.h, enc, C.byref(y), C.byref(a), C.byref(ws[0]), ind, outd, n)
        hip.submit()
        reps = 4
        enc = hip.begin()
        hip.timer_start()
        for _ in range(reps):
            for w in ws:
                hip.lib.gh_matmul_batched(hip.h, enc, C.byref(y), C.byref(a), C.byref(w), ind, outd, n)
        ms = hip.timer_stop() / (reps * len(ws))
        hip.submit()
        tflops = 2.0 * n * ind * outd / (ms * 1e-3) / 1e12
        log(f"bench: prefill GEMM {name} {n}x{ind}->{outd}: {ms * 1e3:.1f} us, {tflops:.0f} TFLOP/s")
        return {"shape": f"{n}x{ind}->{outd}", "avg_us": round(ms * 1e3, 2), "tflops": round(tflops, 1),
                "frac_f16_mfma_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}

    copy_bytes = 2 * sum(i * o for i, o in (synth.tensor_dims(shape, t) for t in synth.LAYER_FORMATS))
    out = {"weights": f"Q4_K gate/up, Q6_K down of {layers} layers, dequantized tile by tile "
                      f"(the C3 workload)",
           "fp16_weight_copies": {
               "weights": "the same layers' FP16 copies (a prefill of more than 128 rows reads "
                          "these instead; same output bits)",
               "hbm_cost_bytes": copy_bytes * shape.block_count,
               "hbm_cost": f"{copy_bytes * shape.block_count / 1e9:.1f} GB of HBM beside the "
                           f"{weight_bytes(shape)[1] / 1e9:.1f} GB of Q4_K_M weights"}}
    for name, tid, ind, outd, a in (("gate_up_q4k", F.T_FFN_GATE, d, ffn, a_d),
                                    ("down_q6k", F.T_FFN_DOWN, ffn, d, a_f)):
        ws = [hip.load_weight(*host[(li, tid)], ind, outd) for li in range(layers)]
        out[name] = timed(name + " (dequantizing)", ws, ind, outd, a)
        for w in ws:
            hip.free_buffer(w)
        out["fp16_weight_copies"][name] = timed(
            name + " (FP16 copies)", [model_weight(model, li, tid) for li in range(layers)], ind, outd, a)
    for b in (a_d, a_f, y):
        hip.free_buffer(b)
    return out


def c4_attention(hip):
    """GQA attention over the f16 KV cache (32 q / 8 kv heads x 128) — the
    2048-row causal prefill on the matrix cores, and single-token decode at ctx 4096 and 32768.
    Decode rotates over distinct layers of a >= 671 MB cache (40 x 4096 / 5 x 32768 positions),
    so the 256 MB MALL cannot serve the K/V stream. HIP-event timing on the backend stream."""
    import ctypes as C

    from graph_horizon_amd import _ffi as F

    qh, kvh, hd = 32, 8, 128
    rng = np.random.default_rng(13)
    out = {}
    for ctx, layers in ((2048, 8), (4096, 40), (32768, 5)):
        per_layer = ctx * kvh * hd
        k1, v1 = synth_f16(rng, per_layer), synth_f16(rng, per_layer)
        kb, vb = hip.from_host(np.tile(k1, layers)), hip.from_host(np.tile(v1, layers))
        del k1, v1
        kv = F.GhKv(kb, vb, F.KV_F16, layers, ctx, kvh, hd, hd)
        rows = ctx if ctx == 2048 else 1
        qb = hip.from_host(synth_f16(rng, rows * qh * hd))
        ob = hip.alloc_buffer(rows * qh * hd * 2)

        def launch(enc, layer):
            if rows > 1:
                return hip.lib.gh_attention_prefill(hip.h, enc, C.byref(ob), C.byref(qb), C.byref(kv),
                                                    qh, 0, rows, layer)
            return hip.lib.gh_attention_decode(hip.h, enc, C.byref(ob), C.byref(qb), C.byref(kv),
                                               qh, ctx - 1, layer)
        enc = hip.begin()
        launch(enc, 0)
        hip.submit()
        reps = 3 if rows > 1 else 5
        enc = hip.begin()
        hip.timer_start()
        for _ in range(reps):
            for layer in range(layers):
                launch(enc, layer)
        ms = hip.timer_stop() / (reps * layers)
        hip.submit()
        if rows > 1:
            tflops = 4.0 * qh * hd * (rows * (rows + 1) / 2) / (ms * 1e-3) / 1e12
            out["prefill_2048"] = {"avg_us": round(ms * 1e3, 1), "tflops": round(tflops, 1),
                                   "frac_f16_mfma_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}
            log(f"bench: attention prefill 2048 causal rows: {ms * 1e3:.1f} us, {tflops:.0f} TFLOP/s")
        else:
            gbps = 2 * per_layer * 2 / (ms * 1e-3) / 1e9
            out[f"decode_{ctx}"] = {"avg_us": round(ms * 1e3, 2), "gbps": round(gbps, 1),
                                    "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4)}
            log(f"bench: attention decode ctx {ctx}: {ms * 1e3:.2f} us/layer, {gbps:.0f} GB/s")
        for b in (kb, vb, qb, ob):
            hip.free_buffer(b)
    return out


def c5_decoder(hip, HipModel, prompt_len, steps=64):
    """the 14B-shaped decoder (40 blocks, d 5120, FFN 16384, vocab 131072,
    attn_v / ffn_down / output Q6_K, the rest Q4_K): a random-id prompt prefilled in one chunk,
    then greedy decode steps as one replayed HIP graph, timed with HIP events."""
    from graph_horizon_amd import synth

    shape = synth.SHAPES["14b"]
    _, per_token = weight_bytes(shape)
    kv_context = prompt_len + 8 + steps + 8
    model = HipModel(hip, synth.model_config(shape, kv_context, prefill_rows=prompt_len))
    t0 = time.perf_counter()
    for layer, tid, fmt, data in synth.model_tensors(shape, seed=1405):
        model.load_tensor(layer, tid, fmt, data)
    log(f"bench: generated and loaded 14b weights in {time.perf_counter() - t0:.1f} s")
    prompt = np.random.default_rng(1405).integers(0, shape.vocab_size, prompt_len).astype(np.uint32)
    model.prefill(prompt, 0)  # untimed: grows the split-K workspace, as in the 8B leg
    hip.synchronize()
    hip.timer_start()
    model.prefill(prompt, 0)
    prefill_ms = hip.timer_stop()
    out = model.decode_greedy(model.read_argmax(), prompt_len, 8)
    hip.synchronize()
    hip.timer_start()
    model.decode_greedy(int(out[-1]), prompt_len + 8, steps)
    ms = hip.timer_stop()
    model.close()
    tok_s = steps / (ms / 1e3)
    log(f"bench: 14b prefill {prompt_len} tokens {prefill_ms:.2f} ms; decode {tok_s:.1f} tok/s")
    return {"workload": "14b-shaped Q4_K_M decoder (BASELINE configs[4]: 40 blocks, d 5120, FFN "
                        f"16384, vocab 131072), {prompt_len}-token prompt, greedy decode bs=1",
            "prefill_ms": round(prefill_ms, 3), "prefill_tok_s": round(prompt_len / (prefill_ms / 1e3), 1),
            "decode_tok_s": round(tok_s, 2), "decode_ms_per_step": round(ms / steps, 4),
            "weight_bytes_per_token": per_token,
            "decode_weight_roofline_frac": round(per_token * tok_s / (HBM_PEAK_GBPS * 1e9), 4)}


def synth_f16(rng, count):
    from graph_horizon_amd import synth

    return synth.f16_bits(rng.standard_normal(count))


if __name__ == "__main__":
    main()
