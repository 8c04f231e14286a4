#!/usr/bin/env python3
"""Benchmark: batch-1 decode tokens/s of the Llama-3B-shape model on one
MI355X, plus the roofline of the dominant kernel (the Q4_0 GEMV) and a CPU baseline.

A step is one forward_step (reference model.cpp:1496-1597) of one new token at position 2048 over a
KV cache pre-filled with 2048 positions of N(0,1) F16 values, followed by the greedy argmax — the
tg loop body of the reference's cmd_bench (cmd_bench.cpp:52-59). Every step runs at the same
position so each step is the same workload. Weights are random-init N(0,0.02) quantized to Q4_0 by
the ggml reference quantizer, written to a synthetic GGUF and loaded through load_weights; inputs
are resident in HBM when the timed region starts.

Prints one JSON line (see the "config", "roofline" and "cpu_baseline" keys).
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))

PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
PROFILE_EVERY = 10     # timed steps per step whose dominant-kernel launches carry HIP events


def load_pkg():
    spec = importlib.util.spec_from_file_location("ggml_loader_amd", os.path.join(ROOT, "ggml-loader_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ggml_loader_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def ensure_model(gl, path, config, seed):
    if os.path.exists(path):
        return
    os.makedirs(os.path.dirname(path), exist_ok=True)
    t = time.time()
    gl.synth_model(path + ".tmp", seed=seed, n_threads=min(16, os.cpu_count() or 1), **gl.CONFIGS[config])
    os.replace(path + ".tmp", path)
    log(f"[bench] wrote synthetic {config} model {path} in {time.time() - t:.1f}s")


def cpu_baseline(gl, model_path, n_pos, token, seconds, threads):
    """The oracle (CPU restatement of ggml-cpu, this repository's oracle/) timed on the host cores
    on a bounded sample of the same workload: decode steps at the same position, one untimed warmup
    step, at each thread count (the reference's cmd_bench hard-codes 8, cmd_bench.cpp:107)."""
    spec = importlib.util.spec_from_file_location("gl_test_helpers", os.path.join(ROOT, "tests", "gl.py"))
    helpers = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(helpers)
    helpers.oracle()  # registers the CPU backend
    runs = {}
    for nt in threads:
        with gl.Session(model_path, "cpu", n_ctx=n_pos + 2, n_threads=nt) as c:
            c.kv_fill_random(n_pos, seed=3)
            _, t1 = c.decode_loop(n_pos, token, 1, fixed_pos=True)  # warmup, also sizes the sample
            n = max(1, min(64, int(seconds / len(threads) / max(t1, 1e-6))))
            _, t = c.decode_loop(n_pos, token, n, fixed_pos=True)
        runs[nt] = (n / t, n, t)
        log(f"[bench] cpu baseline {nt} threads: {n} steps in {t:.2f}s -> {n / t:.2f} tok/s")
    main_nt = threads[0]
    v, n, t = runs[main_nt]
    return {"value": round(v, 3), "unit": "tok/s", "cores": main_nt, "kind": "port",
            "sample": f"{n} decode steps at position {n_pos} ({t:.1f}s) of the same synthetic model on the oracle/ "
                      f"CPU restatement of ggml-cpu (restated ggml-cpu semantics; upstream ggml unavailable offline), "
                      f"{main_nt} threads",
            "by_threads": {str(k): round(r[0], 3) for k, r in runs.items()}}


TRAFFIC_JSON = os.path.join(ROOT, "profiles", "gemv_q4_0_llama3b_decode_traffic.json")


def summarize_pmc(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, copy_mb, kernel_prefix):
    """HBM bytes per launch of the kernels whose name starts with kernel_prefix, from four
    rocprofv3 --pmc runs (FETCH_SIZE and WRITE_SIZE in KiB per dispatch, each over the bench and
    over the copy kernel of copy_mb MiB). Each counter is scaled by what it reads for the copy,
    whose bytes are known: scale = copy bytes / counter bytes."""
    import csv
    import glob

    def per_dispatch(d, prefix):
        vals = []
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                name = r["Kernel_Name"]
                if name.startswith(prefix):
                    vals.append(float(r["Counter_Value"]) * 1024.0)
        if not vals:
            raise SystemExit(f"no {prefix} dispatches in {d}")
        return sum(vals) / len(vals), len(vals)

    copy_bytes = copy_mb * (1 << 20)
    cf, _ = per_dispatch(copy_fetch_dir, "cpy_kernel")
    cw, _ = per_dispatch(copy_write_dir, "cpy_kernel")
    f, n = per_dispatch(fetch_dir, kernel_prefix)
    w, _ = per_dispatch(write_dir, kernel_prefix)
    fs, ws = copy_bytes / cf, copy_bytes / cw
    return {"kernel_prefix": kernel_prefix, "dispatches": n,
            "fetch_size_bytes_per_dispatch": round(f), "write_size_bytes_per_dispatch": round(w),
            "fetch_scale": round(fs, 4), "write_scale": round(ws, 4),
            "copy_kernel_bytes": copy_bytes, "traffic_bytes_per_launch": round(f * fs + w * ws)}


def copy_kernel(gl, mb, reps):
    """Runs the backend's own contiguous f32 copy (a ggml_cpy graph node) over mb MiB reps times:
    the known-size kernel that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters."""
    core = gl.libs()["core"]
    n = mb * (1 << 20) // 4
    ctx = core.ggml_init(gl.ggml_init_params(1 << 20, None, True))
    a = core.ggml_new_tensor_1d(ctx, gl.F32, n)
    b = core.ggml_new_tensor_1d(ctx, gl.F32, n)
    out = core.ggml_cpy(ctx, a, b)
    gf = core.ggml_new_graph(ctx)
    core.ggml_build_forward_expand(gf, out)
    be = gl.hip_backend(0)
    buf = core.ggml_backend_alloc_ctx_tensors(ctx, be)
    t = time.time()
    for _ in range(reps):
        assert core.ggml_backend_graph_compute(be, gf) == 0
    dt = time.time() - t
    core.ggml_backend_buffer_free(buf)
    core.ggml_backend_free(be)
    core.ggml_free(ctx)
    print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "reps": reps,
                      "GB/s": round(2 * n * 4 * reps / dt / 1e9, 1)}), flush=True)


def prefill_bench(gl, args):
    """--prefill N: one forward_step of N prompt tokens at position 0 per step (the reference's
    prefill of a 512-token prompt for the phi3 config, model.cpp:1624-1657, which calls forward_step
    once for the hip backend). Prints its own JSON line; the default run's line is the decode metric."""
    cfg = gl.CONFIGS[args.config]
    wname = {gl.Q4_0: "q4_0", gl.Q8_0: "q8_0", gl.Q4_K: "q4_K"}[cfg["wtype"]]
    model_path = os.path.join(args.model_dir, f"{args.config}_{wname}_seed{args.seed}.gguf")
    ensure_model(gl, model_path, args.config, args.seed)
    import numpy as np
    n = args.prefill
    tokens = np.random.default_rng(args.seed).integers(0, cfg["n_vocab"], n).astype(np.int32)
    hipl = gl.libs()["hip"]
    with gl.Session(model_path, "hip", n_ctx=n) as s:
        for _ in range(args.warmup):
            s.forward(0, tokens)
        t = time.perf_counter()
        for _ in range(args.steps):
            s.forward(0, tokens)
        secs = time.perf_counter() - t
        hipl.ggml_backend_hip_set_profile_filter(s.backend, b"")
        hipl.ggml_backend_hip_reset_profile(s.backend)
        hipl.ggml_backend_hip_set_profiling(s.backend, True)
        s.forward(0, tokens)
        hipl.ggml_backend_hip_set_profiling(s.backend, False)
        prof = gl.profile(s.backend)
    prof.pop("host_enqueue", None)
    ms_step = 1000 * secs / args.steps
    log(f"[bench] prefill {n}: {args.steps} steps in {secs:.4f}s -> {n / (secs / args.steps):.1f} tok/s ({ms_step:.3f} ms/step)")
    total_ms = sum(v[1] for v in prof.values())
    breakdown = {}
    for k, (cnt, ms, by) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        log(f"[bench]   {k:22s} {cnt:5d} launches {ms / cnt * 1e3:10.2f} us/launch {100 * ms / total_ms:5.1f}%")
        breakdown[k] = {"launches": cnt, "us_per_launch": round(ms / cnt * 1e3, 2), "ms": round(ms, 3)}
    print(json.dumps({
        "metric": f"prefill tokens/s ({n}-token prompt)", "value": round(n / (secs / args.steps), 1), "unit": "tok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 3),
        "higher_is_better": True, "data": f"synthetic (seeded random-init weights quantized to {wname.upper()})",
        "config": {"workload": f"{args.config}: prefill of {n} tokens at position 0", "n_tokens": n},
        "kernel_ms_per_step": {k: v["ms"] for k, v in breakdown.items()},
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="llama3b")
    ap.add_argument("--n-past", type=int, default=2048)
    ap.add_argument("--prefill", type=int, default=0, help="time forward_step over this many prompt tokens instead")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--model-dir", default=os.environ.get("GL_BENCH_DIR", "/tmp/gl_bench"))
    ap.add_argument("--breakdown-steps", type=int, default=10, help="untimed steps with every kernel timed")
    ap.add_argument("--cpu-seconds", type=float, default=24.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-mb", type=int, default=0, help="only run the copy kernel of this size (counter calibration)")
    ap.add_argument("--summarize-pmc", nargs=4, metavar=("FETCH_DIR", "WRITE_DIR", "COPY_FETCH_DIR", "COPY_WRITE_DIR"),
                    help="print the HBM bytes per launch of the dominant kernel from rocprofv3 --pmc runs")
    ap.add_argument("--copy-mb-of-pmc", type=int, default=256, help="size of the copy kernel of the calibration runs")
    args = ap.parse_args()

    if args.summarize_pmc:
        print(json.dumps(summarize_pmc(*args.summarize_pmc, args.copy_mb_of_pmc, "void gemv_kernel<2,")), flush=True)
        return

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)

    gl = load_pkg()
    if gl.hip_device_count() < 1:
        raise SystemExit("bench.py: no HIP device")
    if args.copy_mb:
        copy_kernel(gl, args.copy_mb, args.steps)
        return
    if args.prefill:
        prefill_bench(gl, args)
        return
    cfg = gl.CONFIGS[args.config]
    wname = {gl.Q4_0: "q4_0", gl.Q8_0: "q8_0", gl.Q4_K: "q4_K"}[cfg["wtype"]]
    model_path = os.path.join(args.model_dir, f"{args.config}_{wname}_seed{args.seed}.gguf")
    ensure_model(gl, model_path, args.config, args.seed)

    n_past = args.n_past
    token = 12345 % cfg["n_vocab"]
    hipl = gl.libs()["hip"]
    dominant = "gemv_" + wname
    with gl.Session(model_path, "hip", n_ctx=n_past + 2) as s:
        s.kv_fill_random(n_past, seed=3)
        s.decode_loop(n_past, token, args.warmup, fixed_pos=True)

        # timed region: K steps. In every 10th step the dominant kernel's launches (and only those)
        # carry HIP events stamped by their own dispatches on the backend's stream, so its launch
        # durations come from these same steps; reading the events back costs host time after a
        # timed step, which the sampling keeps to a tenth of the steps.
        hipl.ggml_backend_hip_set_profile_filter(s.backend, dominant.encode())
        hipl.ggml_backend_hip_set_profile_sampling(s.backend, PROFILE_EVERY)
        hipl.ggml_backend_hip_reset_profile(s.backend)
        hipl.ggml_backend_hip_set_profiling(s.backend, True)
        _, secs = s.decode_loop(n_past, token, args.steps, fixed_pos=True)
        hipl.ggml_backend_hip_set_profiling(s.backend, False)
        hipl.ggml_backend_hip_set_profile_sampling(s.backend, 1)
        timed = gl.profile(s.backend)
        value = args.steps / secs
        log(f"[bench] {args.steps} steps in {secs:.4f}s -> {value:.1f} tok/s ({1000 * secs / args.steps:.3f} ms/step)")

        # untimed breakdown: every kernel bracketed
        hipl.ggml_backend_hip_set_profile_filter(s.backend, b"")
        hipl.ggml_backend_hip_reset_profile(s.backend)
        hipl.ggml_backend_hip_set_profiling(s.backend, True)
        s.decode_loop(n_past, token, args.breakdown_steps, fixed_pos=True)
        hipl.ggml_backend_hip_set_profiling(s.backend, False)
        prof = gl.profile(s.backend)
        weights_bytes = s.get("weights_bytes")

    host = timed.pop("host_enqueue", None)
    prof.pop("host_enqueue", None)
    total_ms = sum(v[1] for v in prof.values())
    breakdown = {}
    for k, (n, ms, by) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        gbs = by / (ms * 1e-3) / 1e9 if ms > 0 and by > 0 else 0.0
        log(f"[bench]   {k:22s} {n / args.breakdown_steps:7.1f}/step {ms / n * 1e3:8.2f} us/launch "
            f"{100 * ms / total_ms:5.1f}%  {gbs:8.1f} GB/s")
        breakdown[k] = {"launches_per_step": round(n / args.breakdown_steps, 2), "us_per_launch": round(ms / n * 1e3, 2),
                        "GB/s": round(gbs, 1)}
    timed_steps = (args.steps + PROFILE_EVERY - 1) // PROFILE_EVERY
    # HBM bytes per launch measured by rocprofv3 --pmc on this workload (profiles/, see its summary)
    traffic = None
    if os.path.exists(TRAFFIC_JSON):
        traffic = json.load(open(TRAFFIC_JSON))["traffic_bytes_per_launch"]
    gemv = [v for k, v in timed.items() if k.startswith(dominant)]
    g_launch = sum(v[0] for v in gemv)
    g_ms = sum(v[1] for v in gemv)
    g_bytes = sum(v[2] for v in gemv)
    achieved = g_bytes / (g_ms * 1e-3) / 1e9 if g_ms > 0 else 0.0
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBS, 4),
        "traffic": traffic,
        "kernel": f"{dominant}* (every quantized-GEMV launch of a step: QKV, O+residual, gate/up+SwiGLU, "
                  "down+residual, LM head)",
        "launches_per_step": round(g_launch / timed_steps, 2),
        "bytes_per_launch": round(g_bytes / g_launch) if g_launch else None,
        "us_per_launch": round(g_ms / g_launch * 1e3, 3) if g_launch else None,
        "share_of_step": round((g_ms / timed_steps) / (secs * 1e3 / args.steps), 4),
    }

    cpu = None
    if not args.no_cpu_baseline:
        try:
            n_cpu = min(16, os.cpu_count() or 1)
            cpu = cpu_baseline(gl, model_path, n_past, token, args.cpu_seconds, [n_cpu, 8] if n_cpu != 8 else [8])
        except Exception as e:  # the baseline is reported, never required
            log(f"[bench] cpu baseline failed: {e}")

    out = {
        "metric": "batch-1 decode tokens/s; quant-GEMV HBM GB/s as % of MI355X peak",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000 * secs / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": f"synthetic (seeded random-init weights N(0,0.02) quantized to {wname.upper()}; KV cache N(0,1) F16)",
        "config": {"workload": f"{args.config}: Llama-arch decode, 1 token at position {n_past}, batch 1 "
                               f"(hidden 3072, 28 layers, 24/8 heads, head_dim 128, FFN 8192, vocab 128256, Q4_0)",
                   "global_batch": 1, "seq_len": n_past + 1, "parallelism": "single GPU",
                   "weights_bytes": weights_bytes,
                   "arithmetic": "Q4_0 weights x Q8_0 activations by int8 dot products, f32 block sums; "
                                 "F16 KV with f64 dot accumulation"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernel_breakdown_us_per_step": {k: round(v["launches_per_step"] * v["us_per_launch"], 1) for k, v in breakdown.items()},
        "host_enqueue_us_per_step": round(host[1] / host[0] * 1e3, 1) if host else None,
    }
    if host:
        log(f"[bench] host enqueue {host[1] / host[0] * 1e3:.1f} us/step (graph walk + kernel submission)")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
