"""Exactness-contract experiment (CPU only; not collected by pytest): how far a different order of
the quantized GEMVs' block-term sums moves the C2 decode (Llama-3B shape, Q4_0, position 2048).

The HIP kernels reproduce ggml-cpu's generic order exactly (sumf += term, block by block), which
costs a serial chain per output row. A GPU wave reduction adds the same block terms in another
order: lane l sums blocks l, l + 32, ... then the 32 lanes pairwise. The oracle's hook
oracle_set_block_sum_order(1) computes the Q4_0 / Q8_0 dots in that order (the terms themselves
unchanged), and this script compares it with the default order on the same synthetic model:

  * per layer at one decode step: the residual stream after attention and after the FFN
    (per-element relative error with the reference's floor convention, test_vulkan.c:103-109);
  * teacher-forced: --steps steps fed the default order's greedy tokens, the logits' worst
    per-element relative error and argmax agreement;
  * free-running: each order's own greedy chain, the agreement of the two token sequences.

Prints one JSON object. Usage: python tests/exactness_experiment.py [--steps 256] [--threads 8]
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from gl import capture, cpu_backend, gl, oracle, rel_err_floor  # noqa: E402


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--threads", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--n-past", type=int, default=2048)
    ap.add_argument("--model-dir", default=os.environ.get("GL_BENCH_DIR", "/tmp/gl_bench"))
    args = ap.parse_args()

    o = oracle()
    o.oracle_set_block_sum_order.restype = None
    o.oracle_set_block_sum_order.argtypes = [C.c_int]
    gl.libs()["core"].ggml_backend_free(cpu_backend(1))
    cfg = dict(gl.CONFIGS["llama3b"])
    path = os.path.join(args.model_dir, "llama3b_q4_0_seed1.gguf")
    if not os.path.exists(path):
        os.makedirs(args.model_dir, exist_ok=True)
        gl.synth_model(path + ".tmp", seed=1, n_threads=args.threads, **cfg)
        os.replace(path + ".tmp", path)
    n_embd, n_past, first, n = cfg["n_embd"], args.n_past, 12345, args.steps
    core = gl.libs()["core"]
    t0 = time.time()

    def session():
        s = gl.Session(path, "cpu", n_ctx=n_past + n + 1, n_threads=args.threads)
        s.kv_fill_random(n_past, seed=3)
        return s

    # per-layer residual streams at the first step
    layers = {}
    for mode in (0, 1):
        o.oracle_set_block_sum_order(mode)
        with session() as s:
            store = []
            cb = capture(s.backend, store)
            s.forward(n_past, [first])
            core.ggml_backend_set_eval_callback(s.backend, None, None)
            del cb
        layers[mode] = [a for op, shape, a in store if op == "ADD" and shape == (n_embd, 1, 1, 1)]
    per_layer = [rel_err_floor(b, a) for a, b in zip(layers[0], layers[1])]

    # the default order's greedy chain, then the other order teacher-forced on its tokens
    o.oracle_set_block_sum_order(0)
    toks0, logits0 = [], []
    with session() as s:
        tok = first
        for i in range(n):
            lg = s.forward(n_past + i, [tok])
            logits0.append(lg)
            tok = int(np.argmax(lg))
            toks0.append(tok)
    o.oracle_set_block_sum_order(1)
    errs, agree_tf = [], 0
    with session() as s:
        tok = first
        for i in range(n):
            lg = s.forward(n_past + i, [tok])
            errs.append(rel_err_floor(lg, logits0[i]))
            agree_tf += int(np.argmax(lg)) == int(np.argmax(logits0[i]))
            tok = toks0[i]
    # the other order free-running
    with session() as s:
        toks1, _ = s.decode_loop(n_past, first, n)
    o.oracle_set_block_sum_order(0)
    toks1 = [int(t) for t in toks1]
    diverge = next((i for i, (a, b) in enumerate(zip(toks0, toks1)) if a != b), None)
    out = {
        "model": "llama3b Q4_0 (synthetic, seed 1), decode from position %d" % n_past,
        "orders": ["ggml-cpu block order (default)", "32-lane wave reduction"],
        "per_layer_rel_err_floor": [round(float(e), 9) for e in per_layer],
        "per_layer_rel_err_floor_max": float(max(per_layer)),
        "steps": n,
        "teacher_forced_logits_rel_err_floor_max": float(max(errs)),
        "teacher_forced_logits_rel_err_floor_median": float(np.median(errs)),
        "teacher_forced_argmax_agreement": agree_tf / n,
        "free_running_token_agreement": sum(int(a == b) for a, b in zip(toks0, toks1)) / n,
        "free_running_first_divergence": diverge,
        "seconds": round(time.time() - t0, 1),
    }
    print(json.dumps(out, indent=1), flush=True)


if __name__ == "__main__":
    main()
