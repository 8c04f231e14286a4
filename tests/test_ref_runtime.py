"""The reference's own model runtime on this build's backends.

src/model.cpp and src/dory.c are compiled unchanged against include/ into
oracle/_ref/libref_runtime.so (oracle/Makefile.ref). oracle/ref_runtime.cpp drives them in
cmd_bench's sequence (load_weights, load_hparams, load_model, init_kv_cache, init_decode_session,
then prefill / forward_step) on a backend handle that the test passes in.

CPU tier:
* On the oracle's CPU backend, the reference's prefill and forward_step give the same logits, bit
  for bit, as this package's runtime (gl_session) on that backend. This holds for llama, qwen2,
  qwen3 and phi3, so the product's graph builder builds the reference's graphs.
* dory: the reference's dory graph on the oracle backend reproduces an independent float64
  statement of the architecture (tests/dory_model.py).
  - Model: F32 matrices; 10 blocks ("S-*-S-S-S-": 2 input, 6 recurrent run twice, 2 output);
    window 8, so the sliding rings wrap.
  - Rings: K/V filled with NaN bytes first, since init_kv_cache leaves them uninitialized and dory
    masks never-written cells.
  - Workload: 20 prompt tokens in the reference's 8-token prefill chunks, then 10 decode steps.
  - Bar: relative L2 at most 1e-3 per call (measured max 2.0e-4) and the same top token.
  - Each mistake planted in the float64 statement fails that check: rope pairing, no window,
    unsquared q scale, no loop reinjection, KV head h % n_head_kv.
GPU tier:
* The same reference runtime on ggml_backend_hip_init(0) is bit-identical to itself on the oracle
  backend for the four architectures, and to the product session on hip.
* dory on hip, NaN-filled rings, against the float64 statement (its top token within 0.1 logit
  standard deviation of the statement's best). hip's flash_attn_ext forms the softmax in one
  pass with float probabilities, not by ggml-cpu's online rescaling.
  - F32 matrices: within relative L2 1e-3 of the statement and of the oracle backend (measured
    4.8e-4 and 4.9e-4).
  - Q8_0 and Q4_K matrices: every matrix requantizes its input to 8 bits, which amplifies any
    rounding difference. Both backends then sit at about 2-4e-2 from the statement, and from each
    other. hip must be no further from the statement than 1.25x the oracle backend's own distance,
    in median and in max.
"""
import os

import numpy as np
import pytest

import dory_model as D
from gl import REF_RUNTIME_SO, RefRuntime, cpu_backend, gl

pytestmark = pytest.mark.skipif(not os.path.exists(REF_RUNTIME_SO),
                                reason="oracle/_ref/libref_runtime.so not built (no /root/reference)")

# the reference's model.cpp knows no qwen3moe (its MoE engine is qwen_model.c, checked in test_ref_qwen.py)
ARCHS = [("llama", gl.Q4_0, {}), ("qwen2", gl.Q8_0, {}), ("qwen3", gl.Q4_K, {}), ("phi3", gl.Q8_0, {}),
         # phi3 with LongRoPE keys: the reference reads rope_factors_short and passes ext_factor 1
         ("phi3", gl.Q8_0, {"rope_scaling_orig_ctx": 4096, "rope_attn_factor": 1.1902})]
ARCH_IDS = [a[0] + ("-longrope" if a[2] else "") for a in ARCHS]
TOKENS = np.array([1, 5, 9, 100, 200, 300, 7, 8, 11, 2], np.int32)
N_PROMPT = 6
N_CTX = 64
DORY_TOKENS, DORY_PROMPT = 30, 20
DORY_REL = 1e-3
DORY_TOP_GAP = 0.1     # near ties: the chosen token's logit within 0.1 standard deviation of the best


def synth(tmp_path, arch, wtype, extra):
    path = str(tmp_path / f"{arch}.gguf")
    gl.synth_model(path, arch=arch, n_embd=256, n_layer=2, n_head=4, n_head_kv=2, head_dim=64, n_ff=512,
                   n_vocab=512, wtype=wtype, seed=3, **extra)
    return path


def ref_runtime_logits(path, backend, tokens=TOKENS, n_prompt=N_PROMPT, **kw):
    """prefill of the prompt, then one forward_step per remaining token: the logits of each call"""
    with RefRuntime(path, backend, N_CTX, **kw) as r:
        out = [r.prefill(0, tokens[:n_prompt])]
        for i in range(n_prompt, len(tokens)):
            out.append(r.forward(i, tokens[i:i + 1]))
    return np.array(out)


def session_logits(path, backend_name):
    with gl.Session(path, backend_name, n_ctx=N_CTX, n_threads=8) as s:
        out = [s.forward(0, TOKENS[:N_PROMPT].tolist())]
        for i in range(N_PROMPT, len(TOKENS)):
            out.append(s.forward(i, [int(TOKENS[i])]))
    return np.array(out)


@pytest.fixture(scope="module")
def oracle_backend():
    b = cpu_backend(8)
    yield b
    gl.libs()["core"].ggml_backend_free(b)


@pytest.mark.parametrize("arch,wtype,extra", ARCHS, ids=ARCH_IDS)
def test_reference_runtime_equals_product_runtime_on_the_oracle(oracle_backend, tmp_path, arch, wtype, extra):
    path = synth(tmp_path, arch, wtype, extra)
    ref = ref_runtime_logits(path, oracle_backend)
    assert np.isfinite(ref).all()
    assert np.array_equal(ref, session_logits(path, "cpu"))


# ---- dory ----

def dory_calls(model, tokens, chunk):
    """the float64 statement over the reference's call pattern: prefill chunks, then decode steps"""
    out = None
    for o in range(0, DORY_PROMPT, chunk):
        out = model.forward(o, tokens[o:min(DORY_PROMPT, o + chunk)])[-1]
    calls = [out]
    for i in range(DORY_PROMPT, len(tokens)):
        calls.append(model.forward(i, tokens[i:i + 1])[-1])
    return np.array(calls)


def rel_l2(got, ref):
    return np.linalg.norm(got - ref, axis=-1) / np.linalg.norm(ref - ref.mean(axis=-1, keepdims=True), axis=-1)


def dory_ok(got, ref):
    rel = rel_l2(np.asarray(got, np.float64), ref)
    return bool(rel.max() <= DORY_REL and np.array_equal(got.argmax(-1), ref.argmax(-1))), float(rel.max())


@pytest.fixture(scope="module")
def dory_f32(tmp_path_factory):
    cfg = dict(D.BASE)
    path = str(tmp_path_factory.mktemp("dory") / "dory_f32.gguf")
    w = D.write_dory_gguf(path, cfg, gl.F32)
    toks = np.random.default_rng(1).integers(0, cfg["n_vocab"], DORY_TOKENS).astype(np.int32)
    chunk = min(64, cfg["n_swa"])      # model.cpp prefill: min(kDoryChunk, n_cells_min)
    return cfg, w, path, toks, chunk


def test_reference_dory_graph_on_the_oracle_matches_float64(oracle_backend, dory_f32):
    cfg, w, path, toks, chunk = dory_f32
    got = ref_runtime_logits(path, oracle_backend, toks, DORY_PROMPT, kv_fill=0xFF)
    want = dory_calls(D.DoryRef(cfg, w, N_CTX), toks, chunk)
    ok, worst = dory_ok(got, want)
    print(f"dory on the oracle: worst relative L2 {worst:.2e} over {len(got)} calls", flush=True)
    assert ok, worst


@pytest.mark.parametrize("plant", ["rope_normal", "no_window", "qk_unsquared", "no_reinjection", "kv_head_mod"])
def test_dory_comparison_catches_planted_mistakes(oracle_backend, dory_f32, plant):
    cfg, w, path, toks, chunk = dory_f32
    got = ref_runtime_logits(path, oracle_backend, toks, DORY_PROMPT, kv_fill=0xFF)
    want = dory_calls(D.DoryRef(cfg, w, N_CTX, plant=[plant]), toks, chunk)
    ok, worst = dory_ok(got, want)
    print(f"planted {plant}: worst relative L2 {worst:.2e}", flush=True)
    assert not ok and worst > 10 * DORY_REL, worst


# ---- GPU ----

@pytest.fixture(scope="module")
def hip_backend():
    b = gl.hip_backend(0)
    yield b
    gl.libs()["core"].ggml_backend_free(b)


@pytest.mark.gpu
@pytest.mark.parametrize("arch,wtype,extra", ARCHS, ids=ARCH_IDS)
def test_reference_runtime_on_hip(oracle_backend, hip_backend, tmp_path, arch, wtype, extra):
    path = synth(tmp_path, arch, wtype, extra)
    on_hip = ref_runtime_logits(path, hip_backend)
    on_oracle = ref_runtime_logits(path, oracle_backend)
    print(f"{arch}: max |hip - oracle| {np.abs(on_hip - on_oracle).max():.3e}", flush=True)
    assert np.array_equal(on_hip, on_oracle)
    assert np.array_equal(on_hip, session_logits(path, "hip"))


def top_token_gap(got, ref):
    """per call: how far below the reference's best logit the got-top token's reference logit lies,
    in units of that row's logit standard deviation (0 when the top tokens agree)"""
    top = np.asarray(got).argmax(-1)
    return np.array([(r.max() - r[t]) / r.std() for r, t in zip(ref, top)])


@pytest.mark.gpu
@pytest.mark.parametrize("wtype", [gl.F32, gl.Q8_0, gl.Q4_K], ids=["f32", "q8_0", "q4_K"])
def test_reference_dory_graph_on_hip(oracle_backend, hip_backend, tmp_path, wtype):
    cfg = dict(D.BASE)
    path = str(tmp_path / "dory.gguf")
    w = D.write_dory_gguf(path, cfg, wtype)
    toks = np.random.default_rng(2).integers(0, cfg["n_vocab"], DORY_TOKENS).astype(np.int32)
    on_hip = ref_runtime_logits(path, hip_backend, toks, DORY_PROMPT, kv_fill=0xFF)
    on_oracle = ref_runtime_logits(path, oracle_backend, toks, DORY_PROMPT, kv_fill=0xFF)
    f64 = dory_calls(D.DoryRef(cfg, w, N_CTX), toks, min(64, cfg["n_swa"]))
    rh, ro, rho = rel_l2(on_hip, f64), rel_l2(on_oracle, f64), rel_l2(on_hip, on_oracle.astype(np.float64))
    gap = top_token_gap(on_hip, f64)
    print(f"dory on hip: relative L2 to float64 median {np.median(rh):.2e} max {rh.max():.2e} (oracle backend "
          f"{np.median(ro):.2e} / {ro.max():.2e}), to the oracle backend max {rho.max():.2e}; top-token gap "
          f"{gap.max():.3f} std", flush=True)
    assert np.isfinite(on_hip).all()
    assert gap.max() <= DORY_TOP_GAP
    if wtype == gl.F32:
        assert rh.max() <= DORY_REL and rho.max() <= DORY_REL
    else:
        # activations requantized for every matrix amplify any rounding difference alike in both
        # engines: the hip backend must stay as close to the float64 statement as the oracle does
        assert np.median(rh) <= 1.25 * np.median(ro) and rh.max() <= 1.25 * ro.max()
