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
import ctypes as C
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


# the position each decode configuration is quoted at
DEFAULT_N_PAST = {"llama3b": 2048, "qwen3": 8192, "qwen3moe": 4096, "phi3mini": 2048}
WNAME = {2: "q4_0", 8: "q8_0", 12: "q4_K"}


def model_path_of(gl, args):
    cfg = gl.CONFIGS[args.config]
    shared = "_sharedexp" if cfg.get("n_expert") else ""
    return os.path.join(args.model_dir, f"{args.config}_{WNAME[cfg['wtype']]}_seed{args.seed}{shared}.gguf")


def ensure_model(gl, path, config, seed):
    if os.path.exists(path):
        return
    os.makedirs(os.path.dirname(path), exist_ok=True)
    t = time.time()
    cfg = dict(gl.CONFIGS[config])
    if cfg.get("n_expert"):
        cfg["share_experts"] = True   # layer 0's experts in every layer (routers stay per layer)
    log(f"[bench] writing synthetic {config} model {path}")
    gl.synth_model(path + ".tmp", seed=seed, n_threads=min(16, os.cpu_count() or 1), **cfg)
    os.replace(path + ".tmp", path)
    log(f"[bench] wrote synthetic {config} model {path} in {time.time() - t:.1f}s")


def describe(cfg, n_past, batch):
    """The workload of a decode configuration in words."""
    arch = cfg["arch"]
    ffn = (f"{cfg['n_expert']} experts x FFN {cfg['n_ff_exp']}, top-{cfg['n_expert_used']}" if cfg.get("n_expert")
           else f"FFN {cfg['n_ff']}")
    toks = "1 token" if batch == 1 else f"{batch} tokens"
    return (f"{arch} decode, {toks} at position {n_past}, batch {batch} (hidden {cfg['n_embd']}, "
            f"{cfg['n_layer']} layers, {cfg['n_head']}/{cfg['n_head_kv']} heads, head_dim {cfg['head_dim']}, {ffn}, "
            f"vocab {cfg['n_vocab']}, {WNAME[cfg['wtype']].upper()})")


def timed_reps(run, n_steps, reps):
    """One timed loop of n_steps steps (run(k) -> seconds), which gives the reported value, then
    reps - 1 more loops of the same steps for the spread (cmd_bench.cpp:30-38, 135-147 reports the
    mean and sample standard deviation over its reps). Each loop starts from an idle device, so the
    reps are whole loops rather than slices of one: a slice would expose the pipeline's fill once
    per slice. Returns the first loop's seconds and the statistics over all loops."""
    import statistics
    reps = max(1, reps)
    times = [run(n_steps) for _ in range(reps)]
    rates = [n_steps / t for t in times]
    stats = {"n": reps, "steps_per_rep": n_steps, "steps_per_s_mean": round(statistics.fmean(rates), 3),
             "steps_per_s_stddev": round(statistics.stdev(rates), 3) if reps > 1 else 0.0}
    return times[0], stats


def oracle_helpers():
    """tests/gl.py, whose oracle() registers the oracle's CPU backend (the cpu_baseline leg only)."""
    spec = importlib.util.spec_from_file_location("gl_test_helpers", os.path.join(ROOT, "tests", "gl.py"))
    helpers = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(helpers)
    helpers.oracle()
    return helpers


def physical_cores():
    """Distinct (physical id, core id) pairs of /proc/cpuinfo: the host's physical cores."""
    cores, phys = set(), "0"
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "physical id":
                phys = v
            elif k == "core id":
                cores.add((phys, v))
    except OSError:
        pass
    return len(cores) or (os.cpu_count() or 1)


def cpu_threads():
    """Thread counts of the CPU baseline: every core this process may use (its CPU affinity, at
    most the host's physical cores and at most 16, the CPU share of a one-GPU box), then 8, the
    reference's own count (cmd_bench.cpp:107)."""
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count() or 1
    n = max(1, min(16, allowed, physical_cores()))
    return [n, 8] if n != 8 else [8]


def cpu_baseline(gl, model_path, n_pos, tokens, seconds, threads):
    """The oracle (CPU restatement of ggml-cpu, this repository's oracle/) timed on the host cores
    on a bounded sample of the same workload: steps of len(tokens) new tokens at the same position,
    one untimed warmup step, at each thread count (the reference's cmd_bench hard-codes 8,
    cmd_bench.cpp:107)."""
    oracle_helpers()
    batch = len(tokens)
    runs = {}
    for nt in threads:
        with gl.Session(model_path, "cpu", n_ctx=n_pos + batch + 1, n_threads=nt) as c:
            c.kv_fill_random(n_pos, seed=3)

            def steps(k):
                if batch == 1:
                    return c.decode_loop(n_pos, int(tokens[0]), k, fixed_pos=True)[1]
                t = time.perf_counter()
                for _ in range(k):
                    c.forward(n_pos, tokens)
                return time.perf_counter() - t

            t1 = steps(1)  # warmup, also sizes the sample
            n = max(1, min(64, int(seconds / len(threads) / max(t1, 1e-6))))
            t, reps = timed_reps(steps, max(1, n // 3), 3)
            n = max(1, n // 3)
        runs[nt] = (n * batch / t, n, t, reps)
        log(f"[bench] cpu baseline {nt} threads: {n} steps in {t:.2f}s -> {n * batch / t:.2f} tok/s "
            f"({reps['steps_per_s_mean'] * batch:.2f} +- {reps['steps_per_s_stddev'] * batch:.2f} over {reps['n']} reps)")
    main_nt = threads[0]
    v, n, t, reps = runs[main_nt]
    what = "decode steps" if batch == 1 else f"{batch}-token steps"
    return {"value": round(v, 3), "unit": "tok/s", "cores": main_nt, "kind": "port",
            "reps": {"n": reps["n"], "tok_s_mean": round(reps["steps_per_s_mean"] * batch, 3),
                     "tok_s_stddev": round(reps["steps_per_s_stddev"] * batch, 3)},
            "host_physical_cores": physical_cores(), "host_logical_cpus": os.cpu_count(),
            "sample": f"{n} {what} at position {n_pos} ({t:.1f}s) of the same synthetic model on the oracle/ "
                      f"CPU restatement of ggml-cpu (restated ggml-cpu semantics; upstream ggml unavailable offline), "
                      f"{main_nt} threads",
            "by_threads": {str(k): round(r[0], 3) for k, r in runs.items()}}


def traffic_json(wname, config):
    """HBM bytes per launch of the dominant kernel, from rocprofv3 --pmc runs (profiles/)."""
    return os.path.join(ROOT, "profiles", f"gemv_{wname}_{config}_decode_traffic.json")


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


def summarize_pmc_all(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, copy_mb):
    """Per-kernel HBM bytes per dispatch from the same four rocprofv3 --pmc runs: every kernel name
    (its text before the argument list) with its dispatch count, the scaled FETCH_SIZE and
    WRITE_SIZE and their sum."""
    import csv
    import glob

    def per_kernel(d):
        acc = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                name = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0]
                v = acc.setdefault(name, [0, 0.0])
                v[0] += 1
                v[1] += float(r["Counter_Value"]) * 1024.0
        return acc

    copy_bytes = copy_mb * (1 << 20)
    cf, cw = per_kernel(copy_fetch_dir), per_kernel(copy_write_dir)
    fs = copy_bytes / (cf["cpy_kernel"][1] / cf["cpy_kernel"][0])
    ws = copy_bytes / (cw["cpy_kernel"][1] / cw["cpy_kernel"][0])
    f, w = per_kernel(fetch_dir), per_kernel(write_dir)
    out = {}
    for name, (n, tot) in sorted(f.items(), key=lambda kv: -kv[1][1]):
        wn, wt = w.get(name, (n, 0.0))
        fb, wb = tot / n * fs, wt / max(wn, 1) * ws
        out[name] = {"dispatches": n, "fetch_bytes": round(fb), "write_bytes": round(wb), "traffic_bytes": round(fb + wb)}
    return {"fetch_scale": round(fs, 4), "write_scale": round(ws, 4), "kernels": out}


def summarize_activity(pmc_dir):
    """Per-kernel wave activity from one rocprofv3 --pmc run of SQ_WAVES, SQ_INSTS_VALU,
    SQ_INSTS_LDS, SQ_ACTIVE_INST_VALU, SQ_ACTIVE_INST_ANY and SQ_WAIT_ANY: waves per dispatch, VALU
    and LDS instructions per wave, and the shares of the waves' cycles spent issuing VALU and
    waiting (SQ_WAIT_ANY over SQ_WAIT_ANY + SQ_ACTIVE_INST_ANY)."""
    import csv
    import glob

    acc, disp = {}, {}
    for f in glob.glob(os.path.join(pmc_dir, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            name = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0]
            c = acc.setdefault(name, {})
            c[r["Counter_Name"]] = c.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            disp.setdefault(name, set()).add(r["Dispatch_Id"])
    out = {}
    for name, c in sorted(acc.items(), key=lambda kv: -kv[1].get("SQ_INSTS_VALU", 0.0)):
        waves = max(c.get("SQ_WAVES", 0.0), 1.0)
        cyc = max(c.get("SQ_WAIT_ANY", 0.0) + c.get("SQ_ACTIVE_INST_ANY", 0.0), 1.0)
        out[name] = {"dispatches": len(disp[name]), "waves_per_dispatch": round(waves / len(disp[name])),
                     "valu_per_wave": round(c.get("SQ_INSTS_VALU", 0.0) / waves, 1),
                     "lds_per_wave": round(c.get("SQ_INSTS_LDS", 0.0) / waves, 1),
                     "valu_issue_share": round(c.get("SQ_ACTIVE_INST_VALU", 0.0) / cyc, 3),
                     "wait_share": round(c.get("SQ_WAIT_ANY", 0.0) / cyc, 3)}
    return out


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
    wname = WNAME[cfg["wtype"]]
    model_path = model_path_of(gl, args)
    ensure_model(gl, model_path, args.config, args.seed)
    import numpy as np
    n = args.prefill
    tokens = np.random.default_rng(args.seed).integers(0, cfg["n_vocab"], n).astype(np.int32)
    hipl = gl.libs()["hip"]
    with gl.Session(model_path, "hip", n_ctx=n) as s:
        for _ in range(args.warmup):
            s.forward(0, tokens)
        def run(k):
            t = time.perf_counter()
            for _ in range(k):
                s.forward(0, tokens)
            return time.perf_counter() - t

        secs, reps = timed_reps(run, args.steps, args.reps)
        hipl.ggml_backend_hip_set_profile_filter(s.backend, b"")
        hipl.ggml_backend_hip_reset_profile(s.backend)
        hipl.ggml_backend_hip_set_profiling(s.backend, True)
        s.forward(0, tokens)
        hipl.ggml_backend_hip_set_profiling(s.backend, False)
        prof = gl.profile(s.backend)
    prof.pop("host_enqueue", None)
    prof.pop("host_launch_calls", None)
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
        "reps": {"n": reps["n"], "steps_per_rep": reps["steps_per_rep"],
                 "tok_s_mean": round(reps["steps_per_s_mean"] * n, 1), "tok_s_stddev": round(reps["steps_per_s_stddev"] * n, 1)},
        "higher_is_better": True, "data": f"synthetic (seeded random-init weights quantized to {wname.upper()})",
        "config": {"workload": f"{args.config}: prefill of {n} tokens at position 0", "n_tokens": n},
        "kernel_ms_per_step": {k: v["ms"] for k, v in breakdown.items()},
    }), flush=True)


def gemv_bench(gl, args):
    """--gemv: BASELINE.json configs[0], one quantized GEMV y = W x (ggml_mul_mat) with W 4096 x 4096
    drawn from N(0, 0.02) and quantized to Q4_0, x f32 N(0, 1). One graph holds --gemv-copies
    independent GEMVs, each with its own copy of W and its own x, so that consecutive launches read
    weights that are not in the 256 MB Infinity Cache (the copies together are larger). A step is one
    GEMV; its algorithmic bytes are W + x + y."""
    import numpy as np
    K = N = 4096
    R = args.gemv_copies
    core, hipl, loader = gl.libs()["core"], gl.libs()["hip"], gl.libs()["loader"]
    vp = lambda a: a.ctypes.data_as(C.c_void_p)
    w = np.empty(K * N, dtype=np.float32)
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    loader.gl_fill_normal(fp(w), w.size, args.seed, 0, 0.0, 0.02)
    wq = np.empty(core.ggml_row_size(gl.Q4_0, K) * N, dtype=np.uint8)
    core.ggml_quantize_chunk(gl.Q4_0, vp(w), vp(wq), 0, N, K, None)
    xs = np.empty((R, K), dtype=np.float32)
    loader.gl_fill_normal(fp(xs), xs.size, args.seed + 1, 0, 0.0, 1.0)

    def graph(backend, copies):
        ctx = core.ggml_init(gl.ggml_init_params(copies * 4 * core.ggml_tensor_overhead() + core.ggml_graph_overhead()
                                                 + (1 << 20), None, True))
        ws = [core.ggml_new_tensor_2d(ctx, gl.Q4_0, K, N) for _ in range(copies)]
        xt = [core.ggml_new_tensor_2d(ctx, gl.F32, K, 1) for _ in range(copies)]
        ys = [core.ggml_mul_mat(ctx, ws[r], xt[r]) for r in range(copies)]
        gf = core.ggml_new_graph(ctx)
        for y in ys:
            core.ggml_set_output(y)
            core.ggml_build_forward_expand(gf, y)
        buf = core.ggml_backend_alloc_ctx_tensors(ctx, backend)
        for r in range(copies):
            core.ggml_backend_tensor_set(ws[r], vp(wq), 0, wq.nbytes)
            core.ggml_backend_tensor_set(xt[r], vp(xs[r]), 0, K * 4)
        return ctx, gf, buf, ys

    be = gl.hip_backend(0)
    ctx, gf, buf, ys = graph(be, R)
    for _ in range(args.warmup):
        assert core.ggml_backend_graph_compute(be, gf) == 0
    t = time.perf_counter()
    for _ in range(args.steps):
        assert core.ggml_backend_graph_compute(be, gf) == 0
    secs = time.perf_counter() - t
    hipl.ggml_backend_hip_set_profile_filter(be, b"")
    hipl.ggml_backend_hip_reset_profile(be)
    hipl.ggml_backend_hip_set_profiling(be, True)
    for _ in range(args.breakdown_steps):
        assert core.ggml_backend_graph_compute(be, gf) == 0
    hipl.ggml_backend_hip_set_profiling(be, False)
    prof = gl.profile(be)
    prof.pop("host_enqueue", None)
    prof.pop("host_launch_calls", None)
    y0 = np.empty(N, dtype=np.float32)
    core.ggml_backend_tensor_get(ys[0], vp(y0), 0, N * 4)
    core.ggml_backend_buffer_free(buf)
    core.ggml_free(ctx)
    core.ggml_backend_free(be)

    n_gemv = args.steps * R
    us_gemv = 1e6 * secs / n_gemv
    alg = wq.nbytes + K * 4 + N * 4
    for k, (cnt, ms, by) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        log(f"[bench]   {k:22s} {cnt / (args.breakdown_steps * R):5.2f}/GEMV {ms / cnt * 1e3:8.2f} us/launch")
    g = prof.get("gemv_q4_0")
    k_us = g[1] / g[0] * 1e3 if g else None
    log(f"[bench] gemv 4096x4096 Q4_0: {us_gemv:.2f} us per GEMV (wall, {R} copies), kernel {k_us:.2f} us "
        f"-> {alg / (k_us * 1e-6) / 1e9:.1f} GB/s")

    cpu = None
    if not args.no_cpu_baseline:
        oracle_helpers()
        cb = core.ggml_backend_init_by_name(b"CPU", str(min(16, os.cpu_count() or 1)).encode())
        cctx, cgf, cbuf, cys = graph(cb, 1)
        assert core.ggml_backend_graph_compute(cb, cgf) == 0
        yc = np.empty(N, dtype=np.float32)
        core.ggml_backend_tensor_get(cys[0], vp(yc), 0, N * 4)
        n = 0
        t = time.perf_counter()
        while time.perf_counter() - t < min(args.cpu_seconds, 10.0):
            assert core.ggml_backend_graph_compute(cb, cgf) == 0
            n += 1
        ct = time.perf_counter() - t
        core.ggml_backend_buffer_free(cbuf)
        core.ggml_free(cctx)
        core.ggml_backend_free(cb)
        err = float(np.max(np.abs(y0 - yc) / np.maximum(np.abs(yc), 1e-3)))
        log(f"[bench] cpu baseline: {n} GEMVs in {ct:.2f}s; max rel err of the GPU result {err:.2e}")
        cpu = {"value": round(alg * n / ct / 1e9, 3), "unit": "GB/s", "cores": min(16, os.cpu_count() or 1),
               "kind": "port", "us_per_gemv": round(1e6 * ct / n, 1),
               "sample": f"{n} GEMVs ({ct:.1f}s) of the same W and x on the oracle/ CPU restatement of ggml-cpu",
               "gpu_max_rel_err": err}
    print(json.dumps({
        "metric": "quant-GEMV HBM GB/s (4096x4096 Q4_0 ggml_mul_mat)", "value": round(alg / (k_us * 1e-6) / 1e9, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "us_per_gemv_wall": round(us_gemv, 3), "higher_is_better": True, "dtype": "int8",
        "data": "synthetic (W ~ N(0,0.02) quantized to Q4_0, x ~ N(0,1), seeded)",
        "config": {"workload": f"C1: y = W x, W 4096x4096 Q4_0, x f32; {R} weight copies in rotation",
                   "bytes_per_gemv": alg},
        "roofline": {"bound": "hbm", "achieved": round(alg / (k_us * 1e-6) / 1e9, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(alg / (k_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4), "traffic": None,
                     "us_per_launch": round(k_us, 3)},
        "cpu_baseline": cpu,
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # a decode step is ~2 ms: 300 steps keep the timed region well above the run-to-run noise of a
    # 0.2 s region (GPU clock ramp, host scheduling), and 50 warmup steps bring the clocks up first
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--reps", type=int, default=3, help="timed loops of --steps steps: the first gives the value, all give mean +- sd")
    ap.add_argument("--config", default="llama3b")
    ap.add_argument("--n-past", type=int, default=None, help="KV positions before the step (default: per config)")
    ap.add_argument("--batch", type=int, default=1, help="new tokens per decode step")
    ap.add_argument("--prefill", type=int, default=0, help="time forward_step over this many prompt tokens instead")
    ap.add_argument("--gemv", action="store_true", help="time the single 4096x4096 Q4_0 GEMV instead")
    ap.add_argument("--gemv-copies", type=int, default=40, help="weight copies the --gemv graph rotates over")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--model-dir", default=os.environ.get("GL_BENCH_DIR", "/tmp/gl_bench"))
    ap.add_argument("--breakdown-steps", type=int, default=10, help="untimed steps with every kernel timed")
    ap.add_argument("--cpu-seconds", type=float, default=24.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-mb", type=int, default=0, help="only run the copy kernel of this size (counter calibration)")
    ap.add_argument("--summarize-pmc", nargs=4, metavar=("FETCH_DIR", "WRITE_DIR", "COPY_FETCH_DIR", "COPY_WRITE_DIR"),
                    help="print the HBM bytes per launch of the dominant kernel from rocprofv3 --pmc runs")
    ap.add_argument("--copy-mb-of-pmc", type=int, default=256, help="size of the copy kernel of the calibration runs")
    ap.add_argument("--pmc-prefix", default="void gemv_q_kernel<2,", help="kernel name prefix of --summarize-pmc")
    ap.add_argument("--pmc-all", action="store_true", help="--summarize-pmc: every kernel's bytes per dispatch")
    ap.add_argument("--summarize-activity", metavar="PMC_DIR",
                    help="print per-kernel wave activity from a rocprofv3 --pmc run of the SQ counters and exit")
    args = ap.parse_args()

    if args.summarize_activity:
        print(json.dumps(summarize_activity(args.summarize_activity), indent=1), flush=True)
        return
    if args.summarize_pmc:
        if args.pmc_all:
            print(json.dumps(summarize_pmc_all(*args.summarize_pmc, args.copy_mb_of_pmc), indent=1), flush=True)
        else:
            print(json.dumps(summarize_pmc(*args.summarize_pmc, args.copy_mb_of_pmc, args.pmc_prefix)), flush=True)
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
    if args.gemv:
        gemv_bench(gl, args)
        return
    decode_bench(gl, args)


def decode_bench(gl, args):
    """A step is one forward_step of --batch new tokens at position n_past (the same position every
    step) followed, at batch 1, by the greedy argmax: the reference's cmd_bench tg loop body."""
    import numpy as np
    cfg = gl.CONFIGS[args.config]
    wname = WNAME[cfg["wtype"]]
    model_path = model_path_of(gl, args)
    ensure_model(gl, model_path, args.config, args.seed)

    n_past = args.n_past if args.n_past is not None else DEFAULT_N_PAST.get(args.config, 2048)
    batch = args.batch
    token = 12345 % cfg["n_vocab"]
    tokens = np.random.default_rng(args.seed).integers(0, cfg["n_vocab"], batch).astype(np.int32)
    tokens[0] = token
    hipl = gl.libs()["hip"]
    dominant = "gemv_" + wname
    with gl.Session(model_path, "hip", n_ctx=n_past + batch + 1) as s:
        s.kv_fill_random(n_past, seed=3)

        def steps(k):
            if batch == 1:
                return s.decode_loop(n_past, token, k, fixed_pos=True)[1]
            t = time.perf_counter()
            for _ in range(k):
                s.forward(n_past, tokens)
            return time.perf_counter() - t

        steps(args.warmup)

        # timed region: K steps with no events in them. Once a launch carries dispatch-stamped HIP
        # events, the runtime timestamps every later dispatch of the process too (measured: 1.97 ->
        # 2.40 ms per Llama-3B step), so no event is used before this region ends.
        secs, reps = timed_reps(steps, args.steps, args.reps)
        value = args.steps * batch / secs
        tok_mean, tok_sd = reps["steps_per_s_mean"] * batch, reps["steps_per_s_stddev"] * batch
        log(f"[bench] {args.steps} steps in {secs:.4f}s -> {value:.1f} tok/s ({1000 * secs / args.steps:.3f} ms/step); "
            f"over {reps['n']} reps {tok_mean:.1f} +- {tok_sd:.1f} tok/s")

        # the dominant kernel's launch durations: the same K steps again, where in every 10th step
        # its launches (and only those) carry HIP events stamped by their own dispatches on the
        # backend's stream (the events add time between kernels, not to them)
        hipl.ggml_backend_hip_set_profile_filter(s.backend, dominant.encode())
        hipl.ggml_backend_hip_set_profile_sampling(s.backend, PROFILE_EVERY)
        hipl.ggml_backend_hip_reset_profile(s.backend)
        hipl.ggml_backend_hip_set_profiling(s.backend, True)
        secs_ev = steps(args.steps)
        hipl.ggml_backend_hip_set_profiling(s.backend, False)
        hipl.ggml_backend_hip_set_profile_sampling(s.backend, 1)
        timed = gl.profile(s.backend)
        log(f"[bench] kernel-timing pass: {args.steps} steps in {secs_ev:.4f}s ({1000 * secs_ev / args.steps:.3f} ms/step with events)")

        # untimed breakdown: every kernel bracketed
        hipl.ggml_backend_hip_set_profile_filter(s.backend, b"")
        hipl.ggml_backend_hip_reset_profile(s.backend)
        hipl.ggml_backend_hip_set_profiling(s.backend, True)
        steps(args.breakdown_steps)
        hipl.ggml_backend_hip_set_profiling(s.backend, False)
        prof = gl.profile(s.backend)
        weights_bytes = s.get("weights_bytes")

    host = timed.pop("host_enqueue", None)
    host_calls = timed.pop("host_launch_calls", None)
    prof.pop("host_enqueue", None)
    prof.pop("host_launch_calls", None)
    # host time per op handler of the executor (profiled steps), the largest first
    host_ops = sorted(((k[8:], v) for k, v in timed.items() if k.startswith("host_op:")), key=lambda kv: -kv[1][1])
    for k in [k for k in timed if k.startswith("host_op:")]: timed.pop(k)
    for k in [k for k in prof if k.startswith("host_op:")]: prof.pop(k)
    n_steps_timed = host[0] if host else 1
    for name, (n, ms, _) in host_ops[:12]:
        log(f"[bench]   host {name:<20} {n / n_steps_timed:7.1f} nodes/step {1e3 * ms / n_steps_timed:8.1f} us/step")
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
    tj = traffic_json(wname, args.config)
    if batch == 1 and os.path.exists(tj):
        traffic = json.load(open(tj))["traffic_bytes_per_launch"]
    gemv = [v for k, v in timed.items() if k.startswith(dominant)]
    g_launch = sum(v[0] for v in gemv)
    g_ms = sum(v[1] for v in gemv)
    g_bytes = sum(v[2] for v in gemv)
    achieved = g_bytes / (g_ms * 1e-3) / 1e9 if g_ms > 0 else 0.0
    moe = bool(cfg.get("n_expert"))
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBS, 4),
        "traffic": traffic,
        "kernel": f"{dominant}* (every quantized-GEMV launch of a step: QKV, O+residual, "
                  + ("routed-expert gate/up+SwiGLU and down (mul_mat_id)" if moe else "gate/up+SwiGLU, down+residual")
                  + ", LM head)",
        "launches_per_step": round(g_launch / timed_steps, 2),
        "bytes_per_launch": round(g_bytes / g_launch) if g_launch else None,
        "us_per_launch": round(g_ms / g_launch * 1e3, 3) if g_launch else None,
        "share_of_step": round((g_ms / timed_steps) / (secs * 1e3 / args.steps), 4),
        "timing": f"HIP events stamped by the kernel's own dispatches on the backend's stream, in every "
                  f"{PROFILE_EVERY}th of {args.steps} steps run again right after the timed region "
                  f"({1000 * secs_ev / args.steps:.3f} ms/step with the events)",
    }
    att = [prof[k] for k in ("attn_decode", "attn_decode_acc") if k in prof]
    if att:
        # the layer's decode attention (scores, [statistics,] PV[, combination] launches together),
        # from the breakdown steps; algorithmic bytes: the K and V rows read, Q in, the output out, the
        # mask. attn_decode_acc: one query whose PV launch accumulates the output for the O projection
        n_a, ms_a, by_a = (sum(e[i] for e in att) for i in range(3))
        a_ach = by_a / (ms_a * 1e-3) / 1e9 if ms_a > 0 else 0.0
        aj = os.path.join(ROOT, "profiles", f"attn_{wname}_{args.config}_decode_traffic.json")
        roofline["attention"] = {
            "bound": "hbm", "achieved": round(a_ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(a_ach / PEAK_HBM_GBS, 4),
            "traffic": json.load(open(aj))["traffic_bytes_per_layer"] if batch == 1 and os.path.exists(aj) else None,
            "kernel": "decode attention of one layer (attn_scores, attn_pv; attn_stats too past 2304 positions; attn_combine "
                      "unless the PV launch accumulates the one-query output for the O projection's prologue)",
            "us_per_layer": round(ms_a / n_a * 1e3, 2), "bytes_per_layer": round(by_a / n_a),
            "timing": f"HIP events around each layer's attention launches in {args.breakdown_steps} untimed steps",
        }
    if moe:
        roofline["bytes_note"] = ("mul_mat_id launches count each distinct selected expert's bytes once, from the "
                                  "step's routing ids (read back in the profiled steps only)")

    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(gl, model_path, n_past, tokens, args.cpu_seconds, cpu_threads())
        except Exception as e:  # the baseline is reported, never required
            log(f"[bench] cpu baseline failed: {e}")

    dot = "Q8_K" if cfg["wtype"] == gl.Q4_K else "Q8_0"
    data = f"synthetic (seeded random-init weights N(0,0.02) quantized to {wname.upper()}; KV cache N(0,1) F16)"
    if moe:
        data = data[:-1] + "; every layer holds layer 0's expert weights, routers per layer)"
    out = {
        "metric": "batch-1 decode tokens/s; quant-GEMV HBM GB/s as % of MI355X peak" if batch == 1
                  else f"decode tokens/s at batch {batch}; quant-GEMV HBM GB/s as % of MI355X peak",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000 * secs / args.steps, 4),
        "reps": {"n": reps["n"], "steps_per_rep": reps["steps_per_rep"], "tok_s_mean": round(tok_mean, 2),
                 "tok_s_stddev": round(tok_sd, 2)},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": data,
        "config": {"workload": f"{args.config}: " + describe(cfg, n_past, batch),
                   "global_batch": batch, "seq_len": n_past + batch, "parallelism": "single GPU",
                   "weights_bytes": weights_bytes,
                   "arithmetic": f"{wname.upper()} weights x {dot} activations by int8 dot products, f32 block sums; "
                                 "F16 KV with f64 dot accumulation"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernel_breakdown_us_per_step": {k: round(v["launches_per_step"] * v["us_per_launch"], 1) for k, v in breakdown.items()},
        "host_enqueue_us_per_step": round(host[1] / host[0] * 1e3, 1) if host else None,
        "host_launch_calls_us_per_step": round(host_calls[1] / host_calls[0] * 1e3, 1) if host_calls else None,
    }
    if host:
        log(f"[bench] host enqueue {host[1] / host[0] * 1e3:.1f} us/step (graph walk + kernel submission; "
            f"{host_calls[1] / host_calls[0] * 1e3 if host_calls else 0:.1f} us of it inside the launch calls)")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
