#!/usr/bin/env python3
"""Benchmark of the gfx950 hot path: 8B-shaped Q4_K_M decode at bs=1 on one MI355X.

A step is one greedy decode token of a random-init 8B-shaped decoder (34 blocks of the
BASELINE configs[1] decode-step linear layers — Q/K/O/gate/up Q4_K, V/down Q6_K, d_model
4096, FFN 12288, 32/8 heads x 128 — plus RMSNorm/RoPE/SwiGLU/residual glue, f16-KV GQA
attention, the Q6_K 131072x4096 output and the on-device argmax), replayed as one HIP graph
with weights and KV resident in HBM. `value` is tokens/s over exactly --steps timed steps.

Also reported on the same line:
  roofline      the dominant kernel (the Q4_K decode GEMV at the FFN gate/up shape,
                12288x4096) timed with HIP events on the backend stream over the 68 distinct
                gate/up weights of the model (1.9 GB, so the 256 MB MALL cannot serve them);
  cpu_baseline  the CPU oracle (a C++ restatement of the reference's AVX2 CPU kernels) on a
                bounded sample: one block's decode linear layers, scaled to tokens/s.
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


def cpu_baseline(shape, seconds: float):
    """Oracle GEMVs of one block's decode linear layers, rotated over 3 distinct blocks."""
    import oracle as O
    from graph_horizon_amd import synth

    threads = min(len(os.sched_getaffinity(0)), 16)
    O.lib().gho_set_threads(threads)
    rng = np.random.default_rng(99)
    blocks = []
    for _ in range(3):
        mats = []
        for t, fmt in synth.LAYER_FORMATS.items():
            ind, outd = synth.tensor_dims(shape, t)
            mats.append((fmt, synth.quant_blocks(rng, fmt, outd, ind, 0.02), ind, outd))
        blocks.append(mats)
    xs = {n: O.f16(rng.standard_normal(n).astype(np.float32))
          for n in (shape.embedding_length, shape.feed_forward_length,
                    shape.head_count * shape.head_dim)}

    def one(b):
        for fmt, w, ind, outd in blocks[b % 3]:
            O.matmul(fmt, xs[ind], w, ind, outd)

    one(0)
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds:
        one(n)
        n += 1
    dt = (time.perf_counter() - t0) / n
    per_block, per_token = weight_bytes(shape)
    tok_s = 1.0 / (dt * per_token / per_block)
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except Exception:
        pass
    return {"value": round(tok_s, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} passes of one 8B-shaped block's 7 decode GEMVs ({per_block} B, "
                      f"rotated over 3 blocks), {dt * 1e3:.2f} ms/block, scaled by the "
                      f"{per_token} B/token weight stream; {cpu_model}",
            "gbps": round(per_block / dt / 1e9, 2)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=512, help="prefilled context before decode")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--shape", default="8b")
    ap.add_argument("--launch", choices=("graph", "stream"), default="graph",
                    help="decode steps as one replayed HIP graph (default) or as direct "
                         "stream launches of the same kernels (for kernel tracers)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch the roofline kernel (4 distinct weights) and a 256 MiB "
                         "device copy of known size, for rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path shards by rows/heads across GPUs only by design).", file=sys.stderr)
        sys.exit(2)

    from graph_horizon_amd import HipBackend, HipModel, synth
    from graph_horizon_amd import _ffi as F

    if args.traffic_probe:
        traffic_probe(synth.SHAPES[args.shape])
        return
    shape = synth.SHAPES[args.shape]
    per_block, per_token = weight_bytes(shape)
    kv_context = args.prompt + args.warmup + args.steps + 8
    hip = HipBackend(0)
    flags = F.MODEL_NO_GRAPH if args.launch == "stream" else 0
    model = HipModel(hip, synth.model_config(shape, kv_context, prefill_rows=512, flags=flags))
    t0 = time.perf_counter()
    for layer, tid, fmt, data in synth.model_tensors(shape, seed=2024):
        model.load_tensor(layer, tid, fmt, data)
    log(f"bench: loaded {shape.name} weights in {time.perf_counter() - t0:.1f} s")

    rng = np.random.default_rng(7)
    prompt = rng.integers(0, shape.vocab_size, args.prompt).astype(np.uint32)
    model.prefill(prompt[:16], 0)  # first-use costs (workspace growth) outside the timing
    hip.synchronize()
    hip.timer_start()
    model.prefill(prompt, 0)
    prefill_ms = hip.timer_stop()
    log(f"bench: prefill {args.prompt} tokens in {prefill_ms:.2f} ms "
        f"({args.prompt / (prefill_ms / 1e3):.0f} tok/s)")
    first = model.read_argmax()
    pos = args.prompt
    if args.warmup:
        out = model.decode_greedy(first, pos, args.warmup)
        first, pos = int(out[-1]), pos + args.warmup
    hip.synchronize()
    hip.timer_start()
    toks = model.decode_greedy(first, pos, args.steps)
    ms = hip.timer_stop()
    hip.synchronize()
    tok_s = args.steps / (ms / 1e3)
    log(f"bench: {args.steps} decode steps in {ms:.2f} ms -> {tok_s:.1f} tok/s")

    # Dominant kernel: Q4_K decode GEMV at the gate/up shape over the model's own weights.
    d, ffn = shape.embedding_length, shape.feed_forward_length
    xb = hip.from_host(synth.f16_bits(rng.standard_normal(d)))
    yb = hip.alloc_buffer(ffn * 2)
    lib = hip.lib
    import ctypes as C

    weights = []
    for li in range(shape.block_count):
        for tid in (F.T_FFN_GATE, F.T_FFN_UP):
            weights.append(model_weight(model, li, tid))
    enc = hip.begin()
    for w in weights[:4]:
        lib.gh_matmul(hip.h, enc, C.byref(yb), C.byref(xb), C.byref(w), d, ffn)
    hip.submit()
    reps = 3
    enc = hip.begin()
    hip.timer_start()
    for _ in range(reps):
        for w in weights:
            lib.gh_matmul(hip.h, enc, C.byref(yb), C.byref(xb), C.byref(w), d, ffn)
    gemv_ms = hip.timer_stop() / (reps * len(weights))
    hip.submit()
    gemv_bytes = ffn * (d // 256) * 144 + d * 2 + ffn * 2
    gemv_gbps = gemv_bytes / (gemv_ms * 1e-3) / 1e9
    log(f"bench: Q4_K GEMV {ffn}x{d}: {gemv_ms * 1e3:.2f} us, {gemv_gbps:.0f} GB/s")

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
            "workload": f"{shape.name}-shaped Q4_K_M decoder, greedy decode bs=1 "
                        f"({shape.block_count} blocks"
                        f"{' of BASELINE configs[1]' if shape.name == '8b' else ''}"
                        f"{'; BASELINE configs[4]' if shape.name == '14b' else ''}: d {d}, FFN {ffn}, "
                        f"32/8 heads x 128, Q/K/O/gate/up Q4_K, V/down Q6_K; Q6_K output "
                        f"{shape.vocab_size}x{d}); context {args.prompt}..{pos + args.steps}; "
                        f"{args.launch} launch",
            "weight_bytes_per_token": per_token,
            "prefill": {"tokens": args.prompt, "ms": round(prefill_ms, 3),
                        "tok_s": round(args.prompt / (prefill_ms / 1e3), 1)},
            "decode_weight_roofline_frac": round(per_token * tok_s / (HBM_PEAK_GBPS * 1e9), 4),
            "q4k_gemv_c1_shape": None,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gemv_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gemv_gbps / HBM_PEAK_GBPS, 4),
            "traffic": ROOFLINE_TRAFFIC_BYTES if (d, ffn) == (4096, 12288) else None,
            "kernel": f"{gemv_kernel_name(d, ffn)} (Q4_K GEMV {ffn}x{d}, {gemv_bytes} B/launch)",
            "avg_us": round(gemv_ms * 1e3, 3),
        },
    }
    c1 = c1_gemv(hip, model, shape)
    result["config"]["q4k_gemv_c1_shape"] = c1
    result["config"]["prefill_gemm_c3"] = prefill_gemm(hip, model, shape, 512)
    model.close()
    result["config"]["attention_c4"] = c4_attention(hip, shape)
    hip.close()
    if not args.no_cpu:
        log("bench: CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(shape, args.cpu_seconds)
    print(json.dumps(result), flush=True)


def gemv_kernel_name(in_dim, rows):
    """The kernel gh_matmul launches for one token (the host's selection in op_gemv)."""
    if in_dim <= 4096:
        return "gh_gemv_q4k_r1_d" if rows >= 8192 else "gh_gemv_q4k_r2_d"
    return "gh_gemv_q4k_r2_k"


# HBM bytes per launch of the roofline kernel (gh_gemv_q4k_r1_d at 12288x4096), from the two
# rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) over `bench.py --traffic-probe`, each scaled by
# the same counter's reading for a 256 MiB device-to-device copy (FETCH_SIZE x 2.0, WRITE_SIZE
# x 1.0): profiles/q4k_gemv_12288x4096.txt. Re-measure whenever the kernel changes.
ROOFLINE_TRAFFIC_BYTES = 28531416


def traffic_probe(shape):
    """Roofline kernel launches plus a copy of known size, nothing else (for PMC passes)."""
    import ctypes as C

    from graph_horizon_amd import HipBackend, synth

    hip = HipBackend(0)
    d, ffn = shape.embedding_length, shape.feed_forward_length
    rng = np.random.default_rng(5)
    ws = [hip.load_weight(12, synth.quant_blocks(rng, 12, ffn, d, 0.02), d, ffn) for _ in range(4)]
    xb = hip.from_host(synth.f16_bits(rng.standard_normal(d)))
    yb = hip.alloc_buffer(ffn * 2)
    enc = hip.begin()
    for w in ws:
        hip.lib.gh_matmul(hip.h, enc, C.byref(yb), C.byref(xb), C.byref(w), d, ffn)
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
    log(f"bench: traffic probe: 4 x gh_matmul {ffn}x{d} ({ffn * (d // 256) * 144} B of weights "
        f"each), 2 x copy of {nbytes} B")
    rt.hipFree(src)
    rt.hipFree(dst)
    hip.close()


def model_weight(model, layer, tid):
    """The device handle of one model weight (read from the driver's tensor table)."""
    import ctypes as C

    from graph_horizon_amd import _ffi as F

    buf = F.GhBuf()
    rc = model.b.lib.gh_model_weight(model.h, layer, tid, C.byref(buf))
    assert rc == 0, rc
    return buf


MFMA_F16_PEAK_TFLOPS = 2500.0


def prefill_gemm(hip, model, shape, n):
    """the n-token prefill GEMMs (gate/up Q4_K d->FFN, down Q6_K FFN->d) on
    the matrix cores, over 8 distinct layers' weights, timed with HIP events."""
    import ctypes as C

    from graph_horizon_amd import _ffi as F

    d, ffn = shape.embedding_length, shape.feed_forward_length
    rng = np.random.default_rng(11)
    a_d = hip.from_host(synth_f16(rng, n * d))
    a_f = hip.from_host(synth_f16(rng, n * ffn))
    y = hip.alloc_buffer(n * max(d, ffn) * 2)
    out = {}
    for name, tid, ind, outd, a in (("gate_up_q4k", F.T_FFN_GATE, d, ffn, a_d),
                                    ("down_q6k", F.T_FFN_DOWN, ffn, d, a_f)):
        ws = [model_weight(model, li, tid) for li in range(min(8, shape.block_count))]
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
        out[name] = {"shape": f"{n}x{ind}->{outd}", "avg_us": round(ms * 1e3, 2),
                     "tflops": round(tflops, 1), "frac_f16_mfma_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}
        log(f"bench: prefill GEMM {name} {n}x{ind}->{outd}: {ms * 1e3:.1f} us, {tflops:.0f} TFLOP/s")
    for b in (a_d, a_f, y):
        hip.free_buffer(b)
    return out


def c4_attention(hip, shape):
    """GQA attention over the f16 KV cache at the model's heads — the
    2048-row causal prefill on the matrix cores, and single-token decode at ctx 4096 and 32768.
    Decode rotates over distinct layers of a >= 671 MB cache (40 x 4096 / 5 x 32768 positions),
    so the 256 MB MALL cannot serve the K/V stream. HIP-event timing on the backend stream."""
    import ctypes as C

    from graph_horizon_amd import _ffi as F

    qh, kvh, hd = shape.head_count, shape.kv_head_count, shape.head_dim
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


def synth_f16(rng, count):
    from graph_horizon_amd import synth

    return synth.f16_bits(rng.standard_normal(count))


def c1_gemv(hip, model, shape):
    """BASELINE configs[0] shape (Q4_K 4096x4096): the 68 distinct Q and O weights."""
    import ctypes as C

    from graph_horizon_amd import _ffi as F

    d = shape.embedding_length
    if shape.head_count * shape.head_dim != d:
        return None
    ws = [model_weight(model, li, t) for li in range(shape.block_count)
          for t in (F.T_ATTN_Q, F.T_ATTN_OUTPUT)]
    xb = hip.from_host(np.zeros(d, np.uint16))
    yb = hip.alloc_buffer(d * 2)
    enc = hip.begin()
    for w in ws[:4]:
        hip.lib.gh_matmul(hip.h, enc, C.byref(yb), C.byref(xb), C.byref(w), d, d)
    hip.submit()
    enc = hip.begin()
    hip.timer_start()
    reps = 3
    for _ in range(reps):
        for w in ws:
            hip.lib.gh_matmul(hip.h, enc, C.byref(yb), C.byref(xb), C.byref(w), d, d)
    ms = hip.timer_stop() / (reps * len(ws))
    hip.submit()
    nbytes = d * (d // 256) * 144 + d * 2 + d * 2
    gbps = nbytes / (ms * 1e-3) / 1e9
    hip.free_buffer(xb)
    hip.free_buffer(yb)
    return {"shape": f"{d}x{d}", "avg_us": round(ms * 1e3, 3), "gbps": round(gbps, 1),
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "bytes_per_launch": nbytes,
            "distinct_weights": len(ws)}


if __name__ == "__main__":
    main()
