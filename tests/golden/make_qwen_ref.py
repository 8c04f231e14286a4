"""Writes tests/golden/qwen_model_ref.npz: logits of the reference MoE engine's own qwen3moe forward.

The reference's scalar qwen3moe engine (GGML-Loader src/moe_stream/qwen_model.c with the GGUF index,
expert loader and scalar backend it calls) is built from its sources in place by oracle/Makefile.ref
into oracle/_ref/libqwen_ref.so. This script writes seeded synthetic qwen3moe GGUFs with the
product's writer (gl_synth_model), runs qwen_load + qwen_forward token by token from position 0
(qwen_model.c:972-1016: attention_block :456-531 with per-head q/k rmsnorm, NEOX rope from tables
computed in double :346-355, f32 KV, GQA head h -> KV head h / (n_head / n_head_kv), softmax
compute_backend.c:68-86; moe_block :608-730 with moe_route :551-606) and stores the logits after
every token, with the model's parameters and the sha256 of the GGUF it read.

    make -C oracle -f Makefile.ref && python tests/golden/make_qwen_ref.py

Models: the C5 attention layout (32 query heads, 4 KV heads, head_dim 128), 2 layers, 16 experts
with 4 used, n_embd 512, vocab 512; one with every matrix F32 (the reference and ggml then differ
only in summation order and the F16 KV cache) and one with Q4_K matrices (the MoE configuration's
weight type; ggml additionally quantizes activations to Q8_K). 32 tokens each.
Q8_0 is left out: the reference's vec_dot walks Q8_0 rows in 256-element super-blocks of 34-byte
blocks (dequant.c:255-297), so its qwen_forward returns garbage on Q8_0 matrices.
"""
import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

from gl import gl, ref_qwen, ref_qwen_logits  # noqa: E402

OUT = os.path.join(HERE, "qwen_model_ref.npz")
N_TOKENS = 32
MAX_SEQ = 64

BASE = dict(arch="qwen3moe", n_embd=512, n_layer=2, n_head=32, n_head_kv=4, head_dim=128, n_ff=256, n_vocab=512,
            rope_theta=1000000.0, rms_eps=1e-6, n_expert=16, n_expert_used=4, n_ff_exp=256, seed=7)
MODELS = {"f32": dict(BASE, wtype=gl.F32), "q4_K": dict(BASE, wtype=gl.Q4_K)}


def sha256(path):
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def tokens_of(cfg):
    return np.random.default_rng(cfg["seed"] + 1).integers(0, cfg["n_vocab"], N_TOKENS).astype(np.int32)


def main():
    lib = ref_qwen()
    if lib is None:
        raise SystemExit("oracle/_ref/libqwen_ref.so missing: run `make -C oracle -f Makefile.ref`")
    out = {}
    with tempfile.TemporaryDirectory() as tmp:
        for name, cfg in MODELS.items():
            path = os.path.join(tmp, f"{name}.gguf")
            gl.synth_model(path, **cfg)
            toks = tokens_of(cfg)
            logits = ref_qwen_logits(lib, path, toks, MAX_SEQ)
            assert np.isfinite(logits).all(), name
            out[f"{name}_config"] = np.array(json.dumps(cfg))
            out[f"{name}_sha256"] = np.array(sha256(path))
            out[f"{name}_tokens"] = toks
            out[f"{name}_logits"] = logits
            print(f"{name}: {len(toks)} tokens, logits {logits.shape}, std {logits.std():.4f}")
    np.savez(OUT, **out)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
