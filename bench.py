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


def cpu_baseline(gl, model_path, n_pos, token, seconds, n_threads):
    """The oracle (CPU restatement of ggml-cpu, this repository's oracle/) timed on the host cores
    on a bounded sample of the same workload: a few decode steps at the same position."""
    spec = importlib.util.spec_from_file_location("gl_test_helpers", os.path.join(ROOT, "tests", "gl.py"))
    helpers = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(helpers)
    helpers.oracle()  # registers the CPU backend
    with gl.Session(model_path, "cpu", n_ctx=n_pos + 2, n_threads=n_threads) as c:
        c.kv_fill_random(n_pos, seed=3)
        _, t1 = c.decode_loop(n_pos, token, 1, fixed_pos=True)  # warmup, also sizes the sample
        n = max(1, min(64, int(seconds / max(t1, 1e-6))))
        _, t = c.decode_loop(n_pos, token, n, fixed_pos=True)
    return {"value": n / t, "unit": "tok/s", "cores": n_threads, "kind": "port",
            "sample": f"{n} decode steps at position {n_pos} ({t:.1f}s), oracle/ CPU restatement of ggml-cpu "
                      f"(upstream ggml unavailable offline), {n_threads} threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="llama3b")
    ap.add_argument("--n-past", type=int, default=2048)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--model-dir", default=os.environ.get("GL_BENCH_DIR", "/tmp/gl_bench"))
    ap.add_argument("--profile-steps", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)

    gl = load_pkg()
    if gl.hip_device_count() < 1:
        raise SystemExit("bench.py: no HIP device")
    cfg = gl.CONFIGS[args.config]
    wname = {gl.Q4_0: "q4_0", gl.Q8_0: "q8_0", gl.Q4_K: "q4_K"}[cfg["wtype"]]
    model_path = os.path.join(args.model_dir, f"{args.config}_{wname}_seed{args.seed}.gguf")
    ensure_model(gl, model_path, args.config, args.seed)

    n_past = args.n_past
    token = 12345 % cfg["n_vocab"]
    hipl = gl.libs()["hip"]
    with gl.Session(model_path, "hip", n_ctx=n_past + 2) as s:
        s.kv_fill_random(n_past, seed=3)
        s.decode_loop(n_past, token, args.warmup, fixed_pos=True)
        _, secs = s.decode_loop(n_past, token, args.steps, fixed_pos=True)
        value = args.steps / secs
        log(f"[bench] {args.steps} steps in {secs:.4f}s -> {value:.1f} tok/s ({1000 * secs / args.steps:.3f} ms/step)")

        # per-kernel HIP-event timing over a second pass of the same steps
        hipl.ggml_backend_hip_set_profiling(s.backend, True)
        hipl.ggml_backend_hip_reset_profile(s.backend)
        s.decode_loop(n_past, token, args.profile_steps, fixed_pos=True)
        prof = gl.profile(s.backend)
        hipl.ggml_backend_hip_set_profiling(s.backend, False)
        weights_bytes = s.get("weights_bytes")

    total_ms = sum(v[1] for v in prof.values())
    for k, (n, ms, by) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        gbs = by / (ms * 1e-3) / 1e9 if ms > 0 and by > 0 else 0.0
        log(f"[bench]   {k:22s} {n / args.profile_steps:7.1f}/step {ms / n * 1e3:8.2f} us/launch "
            f"{100 * ms / total_ms:5.1f}%  {gbs:8.1f} GB/s")
    gemv = [v for k, v in prof.items() if k.startswith("gemv_" + wname)]
    g_launch = sum(v[0] for v in gemv)
    g_ms = sum(v[1] for v in gemv)
    g_bytes = sum(v[2] for v in gemv)
    achieved = g_bytes / (g_ms * 1e-3) / 1e9 if g_ms > 0 else 0.0
    roofline = {
        "bound": "hbm",
        "kernel": f"gemv_{wname} (all launches of a step: fused QKV, O+residual, gate/up+SwiGLU, down+residual, LM head)",
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBS, 4),
        "traffic": None,
        "bytes_per_launch": round(g_bytes / g_launch) if g_launch else None,
        "us_per_launch": round(g_ms / g_launch * 1e3, 3) if g_launch else None,
        "kernel_time_per_step_ms": round(total_ms / args.profile_steps, 4),
    }

    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(gl, model_path, n_past, token, args.cpu_seconds, min(16, os.cpu_count() or 1))
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
        "dtype": "q4_0 weights x q8_0 activations (int8 dot), f32 accumulate, f16 KV",
        "data": "synthetic (seeded random-init weights N(0,0.02) quantized to Q4_0; KV cache N(0,1) F16)",
        "config": {"workload": f"{args.config}: Llama-arch decode, 1 token at position {n_past}, batch 1 "
                               f"(hidden 3072, 28 layers, 24/8 heads, head_dim 128, FFN 8192, vocab 128256, Q4_0)",
                   "global_batch": 1, "seq_len": n_past + 1, "parallelism": "single GPU",
                   "weights_bytes": weights_bytes},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
