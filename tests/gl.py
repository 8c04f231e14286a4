"""Test helpers: load the product package and the oracle, build small ggml graphs through the
C-ABI, and compare results.

The oracle (oracle/_build/libggml-cpu-oracle.so, the CPU restatement of ggml-cpu) is loaded only
here, in tests, as the checker.
"""
from __future__ import annotations

import ctypes as C
import importlib.util
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_INIT = os.path.join(ROOT, "ggml-loader_amd", "__init__.py")
# GGML_LOADER_ORACLE_SO: another build of the oracle (the sanitized one, oracle/_asan)
ORACLE_SO = os.environ.get("GGML_LOADER_ORACLE_SO") or os.path.join(ROOT, "oracle", "_build", "libggml-cpu-oracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libmoe_ref.so")
REF_SAMPLER_SO = os.path.join(ROOT, "oracle", "_ref", "libref_sampler.so")
REF_QWEN_SO = os.path.join(ROOT, "oracle", "_ref", "libqwen_ref.so")
REF_RUNTIME_SO = os.path.join(ROOT, "oracle", "_ref", "libref_runtime.so")
GOLDEN = os.path.join(ROOT, "tests", "golden")


def load_pkg():
    if "ggml_loader_amd" in sys.modules:
        return sys.modules["ggml_loader_amd"]
    spec = importlib.util.spec_from_file_location("ggml_loader_amd", PKG_INIT)
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ggml_loader_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


gl = load_pkg()
_oracle = None


def oracle():
    """The oracle library (also registers the "CPU" ggml backend)."""
    global _oracle
    if _oracle is None:
        gl.libs()
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle`")
        if not gl.libs()["core"].ggml_backend_load(ORACLE_SO.encode()):
            raise RuntimeError("loading the oracle backend failed")
        o = C.CDLL(ORACLE_SO, mode=C.RTLD_GLOBAL)
        vp, i64 = C.c_void_p, C.c_int64
        o.oracle_fp16_to_fp32.restype = C.c_float
        o.oracle_fp16_to_fp32.argtypes = [C.c_uint16]
        o.oracle_fp32_to_fp16.restype = C.c_uint16
        o.oracle_fp32_to_fp16.argtypes = [C.c_float]
        for n in ("oracle_quantize_q4_0", "oracle_quantize_q8_0", "oracle_quantize_q4_K", "oracle_quantize_q8_K",
                  "oracle_quantize_q5_K", "oracle_quantize_q6_K"):
            getattr(o, n).restype = None
            getattr(o, n).argtypes = [vp, vp, i64]
        o.oracle_dequantize.restype = C.c_int
        o.oracle_dequantize.argtypes = [C.c_int, vp, vp, i64]
        for n in ("oracle_vec_dot_q4_0_q8_0", "oracle_vec_dot_q8_0_q8_0", "oracle_vec_dot_q4_K_q8_K",
                  "oracle_vec_dot_q5_K_q8_K", "oracle_vec_dot_q6_K_q8_K"):
            getattr(o, n).restype = C.c_float
            getattr(o, n).argtypes = [i64, vp, vp]
        o.oracle_gemv.restype = None
        o.oracle_gemv.argtypes = [C.c_int, vp, i64, i64, vp, vp, C.c_int]
        o.oracle_rope.restype = None
        o.oracle_rope.argtypes = [vp, vp, i64, C.c_int, C.c_int, C.c_int32] + [C.c_float] * 6 + [C.c_int, vp]
        o.oracle_make_qx_quants.restype = C.c_float
        o.oracle_make_qx_quants.argtypes = [C.c_int, C.c_int, vp, vp]
        o.oracle_make_qkx2_quants.restype = C.c_float
        o.oracle_make_qkx2_quants.argtypes = [C.c_int, C.c_int, vp, vp, vp, vp, C.c_float, C.c_float, C.c_int]
        o.oracle_moe_route.restype = None
        o.oracle_moe_route.argtypes = [vp, C.c_int, C.c_int, vp, vp]
        o.oracle_sample.restype = C.c_int32
        o.oracle_sample.argtypes = [vp, i64, vp, i64, C.c_float, C.c_int32, C.c_float, C.c_float, C.c_int32,
                                    C.c_double, C.POINTER(C.c_int32)]
        _oracle = o
    return _oracle


# ---- sampling ----
class Draws:
    """The uniform variates libstdc++'s std::discrete_distribution takes from a std::mt19937 seeded
    with `seed` (the reference's init_sampler, model.cpp:1668-1673): generate_canonical<double, 53>
    of two 32-bit outputs, (a + b * 2^32) / 2^64, kept below 1 (GCC 11 bits/random.tcc). numpy's
    MT19937 with legacy seeding is std::mt19937's generator and seeding. A variate stays pending
    until a sampling call reports that it consumed it (the reference's generator only advances
    then)."""

    def __init__(self, seed: int):
        self.bg = np.random.MT19937()
        self.bg._legacy_seeding(seed)
        self.pending = None

    def peek(self) -> float:
        if self.pending is None:
            a, b = (float(v) for v in self.bg.random_raw(2))
            u = (a + b * 4294967296.0) / 18446744073709551616.0
            self.pending = u if u < 1.0 else float(np.nextafter(1.0, 0.0))
        return self.pending

    def consume(self) -> None:
        self.pending = None


SAMPLER_DEFAULTS = dict(temp=0.0, top_k=40, top_p=0.95, repeat_penalty=1.0, repeat_last_n=64)


def oracle_sample(logits, recent=(), u=0.5, **params):
    """oracle_sample on one row: (token id, whether u was used)."""
    p = dict(SAMPLER_DEFAULTS, **params)
    x = np.ascontiguousarray(logits, dtype=np.float32)
    r = np.ascontiguousarray(recent, dtype=np.int32)
    used = C.c_int32(0)
    tok = oracle().oracle_sample(ptr(x), x.size, ptr(r), r.size, p["temp"], p["top_k"], p["top_p"],
                                 p["repeat_penalty"], p["repeat_last_n"], u, C.byref(used))
    return int(tok), bool(used.value)


def oracle_sample_seq(logits, recent, seed, n_calls, **params):
    """n_calls samples of the same row with one generator running on, as the reference's
    decode loop calls sample()."""
    d, out = Draws(seed), []
    for _ in range(n_calls):
        tok, used = oracle_sample(logits, recent, d.peek(), **params)
        if used:
            d.consume()
        out.append(tok)
    return out


def ref_sampler():
    """The reference's own init_sampler/sample (oracle/_ref/libref_sampler.so), or None."""
    if not os.path.exists(REF_SAMPLER_SO):
        return None
    gl.libs()
    lib = C.CDLL(REF_SAMPLER_SO)
    lib.ref_sample_run.restype = C.c_int
    lib.ref_sample_run.argtypes = [C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.c_float, C.c_int32, C.c_float,
                                   C.c_float, C.c_int32, C.c_uint32, C.c_int, C.c_void_p]
    return lib


def ref_sample_seq(lib, logits, recent, seed, n_calls, **params):
    p = dict(SAMPLER_DEFAULTS, **params)
    x = np.ascontiguousarray(logits, dtype=np.float32)
    r = np.ascontiguousarray(recent, dtype=np.int32)
    out = np.zeros(n_calls, dtype=np.int32)
    lib.ref_sample_run(ptr(x), x.size, ptr(r), r.size, p["temp"], p["top_k"], p["top_p"], p["repeat_penalty"],
                       p["repeat_last_n"], seed, n_calls, ptr(out))
    return [int(v) for v in out]


def ref_qwen():
    """The reference MoE engine's scalar qwen3moe forward (oracle/_ref/libqwen_ref.so), or None."""
    if not os.path.exists(REF_QWEN_SO):
        return None
    lib = C.CDLL(REF_QWEN_SO)
    lib.qwen_load.restype = C.c_void_p
    lib.qwen_load.argtypes = [C.c_char_p, C.c_size_t, C.c_int, C.c_int, C.c_int]
    lib.qwen_forward.restype = C.c_int
    lib.qwen_forward.argtypes = [C.c_void_p, C.c_int]
    lib.qwen_logits.restype = C.POINTER(C.c_float)
    lib.qwen_logits.argtypes = [C.c_void_p]
    lib.qwen_vocab_size.restype = C.c_int
    lib.qwen_vocab_size.argtypes = [C.c_void_p]
    lib.qwen_free.restype = None
    lib.qwen_free.argtypes = [C.c_void_p]
    return lib


def ref_qwen_logits(lib, path, tokens, max_seq=64):
    """qwen_load, then qwen_forward token by token from position 0 (qwen_model.c:972-1016): the
    logits after each token, one row per token."""
    m = lib.qwen_load(path.encode(), 64 << 20, 1, max_seq, 0)
    if not m:
        raise RuntimeError(f"qwen_load failed on {path}")
    try:
        n_vocab = lib.qwen_vocab_size(m)
        out = np.zeros((len(tokens), n_vocab), np.float32)
        for i, t in enumerate(tokens):
            if lib.qwen_forward(m, int(t)) != 0:
                raise RuntimeError(f"qwen_forward failed at step {i}")
            out[i] = np.ctypeslib.as_array(lib.qwen_logits(m), (n_vocab,))
        return out
    finally:
        lib.qwen_free(m)


class RefRuntime:
    """The reference's own model runtime (model.cpp + dory.c via oracle/_ref/libref_runtime.so) on a
    backend handle: load_weights .. init_decode_session at open, forward_step / prefill per call."""
    _lib = None

    @classmethod
    def lib(cls):
        if cls._lib is None:
            gl.libs()
            lib = C.CDLL(REF_RUNTIME_SO)
            lib.ref_rt_open.restype = C.c_void_p
            lib.ref_rt_open.argtypes = [C.c_char_p, C.c_void_p, C.c_int64, C.c_int]
            lib.ref_rt_n_vocab.restype = C.c_int64
            lib.ref_rt_n_vocab.argtypes = [C.c_void_p]
            lib.ref_rt_kv_fill.restype = None
            lib.ref_rt_kv_fill.argtypes = [C.c_void_p, C.c_uint8]
            lib.ref_rt_forward.restype = C.c_int
            lib.ref_rt_forward.argtypes = [C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.c_void_p]
            lib.ref_rt_prefill.restype = C.c_int
            lib.ref_rt_prefill.argtypes = [C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.c_int, C.c_void_p]
            lib.ref_rt_close.restype = None
            lib.ref_rt_close.argtypes = [C.c_void_p]
            cls._lib = lib
        return cls._lib

    def __init__(self, path, backend, n_ctx=64, flash_attn=False, kv_fill=None):
        self.l = self.lib()
        self.h = self.l.ref_rt_open(path.encode(), backend, n_ctx, int(flash_attn))
        self.n_vocab = int(self.l.ref_rt_n_vocab(self.h))
        if kv_fill is not None:
            self.l.ref_rt_kv_fill(self.h, kv_fill)

    def _call(self, fn, n_past, tokens, *extra):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros(self.n_vocab, np.float32)
        if fn(self.h, n_past, ptr(t), t.size, *extra, ptr(out)) != 0:
            raise RuntimeError("reference runtime call failed")
        return out

    def forward(self, n_past, tokens):
        return self._call(self.l.ref_rt_forward, n_past, tokens)

    def prefill(self, n_past, tokens, use_chunking=False):
        return self._call(self.l.ref_rt_prefill, n_past, tokens, int(use_chunking))

    def close(self):
        if self.h:
            self.l.ref_rt_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


def cpu_backend(n_threads: int = 8):
    oracle()
    b = gl.libs()["core"].ggml_backend_init_by_name(b"CPU", str(n_threads).encode())
    if not b:
        raise RuntimeError("CPU backend not registered")
    return b


def ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


# ---- quantization helpers (through the oracle) ----
BLOCK = {gl.Q4_0: (32, 18), gl.Q8_0: (32, 34), gl.Q4_K: (256, 144), gl.Q5_K: (256, 176), gl.Q6_K: (256, 210),
         gl.Q8_K: (256, 292)}


def quantize(x: np.ndarray, qtype: int, impl: str = "oracle") -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    qk, bs = BLOCK[qtype]
    assert x.size % qk == 0
    out = np.zeros(x.size // qk * bs, dtype=np.uint8)
    if impl == "oracle":
        fn = {gl.Q4_0: "oracle_quantize_q4_0", gl.Q8_0: "oracle_quantize_q8_0", gl.Q4_K: "oracle_quantize_q4_K",
              gl.Q5_K: "oracle_quantize_q5_K", gl.Q6_K: "oracle_quantize_q6_K", gl.Q8_K: "oracle_quantize_q8_K"}[qtype]
        getattr(oracle(), fn)(ptr(x), ptr(out), x.size)
    else:
        n_per_row = x.shape[-1] if x.ndim > 1 else x.size
        gl.libs()["core"].ggml_quantize_chunk(qtype, ptr(x), ptr(out), 0, x.size // n_per_row, n_per_row, None)
    return out


def dequantize(q: np.ndarray, qtype: int, n: int, impl: str = "oracle") -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    q = np.ascontiguousarray(q)
    if impl == "oracle":
        assert oracle().oracle_dequantize(qtype, ptr(q), ptr(out), n)
    else:
        assert gl.libs()["core"].ggml_dequantize_row(qtype, ptr(q), ptr(out), n)
    return out


def randn(n, seed, std=1.0, mean=0.0):
    """The product's seeded normal generator (also used by the synthetic models)."""
    out = np.empty(n, dtype=np.float32)
    gl.libs()["loader"].gl_fill_normal(out.ctypes.data_as(C.POINTER(C.c_float)), n, seed, 0, mean, std)
    return out


# ---- error metrics ----
def rel_err(x, ref) -> float:
    """max |x - ref| / max |ref| (normwise, infinity norm)."""
    x = np.asarray(x, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(x - ref)) / (den if den > 0 else 1.0))


def rel_err_floor(x, ref) -> float:
    """The reference's per-element convention (test_vulkan.c:103-109): |x-ref| / (|ref| if |ref| > 1e-3 else 1)."""
    x = np.asarray(x, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    den = np.where(np.abs(ref) > 1e-3, np.abs(ref), 1.0)
    return float(np.max(np.abs(x - ref) / den))


# ---- graph builder over the C-ABI ----
class Graph:
    """One no_alloc ggml context; tensors are allocated on a backend by compute()."""

    def __init__(self, mem: int = 256 << 20):
        self.core = gl.libs()["core"]
        self.ctx = self.core.ggml_init(gl.ggml_init_params(mem, None, True))
        self.inputs = []
        self.buf = None

    def __getattr__(self, name):
        # g.mul_mat(a, b) -> ggml_mul_mat(ctx, a, b)
        fn = getattr(self.core, "ggml_" + name)
        return lambda *args: fn(self.ctx, *args)

    def tensor(self, ttype, *ne, data=None, name=None):
        f = {1: self.core.ggml_new_tensor_1d, 2: self.core.ggml_new_tensor_2d, 3: self.core.ggml_new_tensor_3d,
             4: self.core.ggml_new_tensor_4d}[len(ne)]
        t = f(self.ctx, ttype, *ne)
        if name:
            self.core.ggml_set_name(t, name.encode())
        if data is not None:
            self.inputs.append((t, np.ascontiguousarray(data)))
        return t

    def compute(self, backend, outs):
        if not isinstance(outs, (list, tuple)):
            outs = [outs]
        gf = self.core.ggml_new_graph(self.ctx)
        for o in outs:
            self.core.ggml_set_output(o)   # read back after compute: ggml's output contract
            self.core.ggml_build_forward_expand(gf, o)
        self.buf = self.core.ggml_backend_alloc_ctx_tensors(self.ctx, backend)
        for t, a in self.inputs:
            assert a.nbytes == self.core.ggml_nbytes(t), (a.nbytes, self.core.ggml_nbytes(t))
            self.core.ggml_backend_tensor_set(t, ptr(a), 0, a.nbytes)
        assert self.core.ggml_backend_graph_compute(backend, gf) == 0
        res = []
        for o in outs:
            res.append(self.read(o))
        if not res:
            return None
        return res if len(res) > 1 else res[0]

    def read(self, t, dtype=np.float32):
        nb = self.core.ggml_nbytes(t)
        out = np.empty(nb // np.dtype(dtype).itemsize, dtype=dtype)
        self.core.ggml_backend_tensor_get(t, ptr(out), 0, nb)
        return out

    def n_nodes(self, outs):
        gf = self.core.ggml_new_graph(self.ctx)
        for o in (outs if isinstance(outs, (list, tuple)) else [outs]):
            self.core.ggml_build_forward_expand(gf, o)
        return self.core.ggml_graph_n_nodes(gf)

    def close(self):
        if self.buf:
            self.core.ggml_backend_buffer_free(self.buf)
            self.buf = None
        if self.ctx:
            self.core.ggml_free(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def run_on(backend, build):
    """build(g) -> (outs, raw-dtype) ; returns the computed output(s) on `backend`."""
    with Graph() as g:
        outs = build(g)
        return g.compute(backend, outs)


def attention_graph(g, hd, n_head, n_head_kv, n_kv, n_new, n_ctx, kc, vc, q, mask, flash=False):
    """The attention block of build_graph (reference model.cpp:1416-1444)."""
    K_cache = g.tensor(gl.F16, hd, n_head_kv, n_ctx, data=kc)
    V_cache = g.tensor(gl.F16, hd, n_head_kv, n_ctx, data=vc)
    Qcur = g.tensor(gl.F32, hd, n_head, n_new, data=q)
    m = g.tensor(gl.F32, n_kv, n_new, data=mask)
    nb1, nb2 = hd * 2, hd * n_head_kv * 2
    K_full = g.view_3d(K_cache, hd, n_head_kv, n_kv, nb1, nb2, 0)
    V_full = g.view_3d(V_cache, hd, n_head_kv, n_kv, nb1, nb2, 0)
    Q = g.permute(Qcur, 0, 2, 1, 3)
    K = g.permute(K_full, 0, 2, 1, 3)
    scale = 1.0 / np.sqrt(hd)
    if flash:
        V = g.permute(V_full, 0, 2, 1, 3)
        out = g.flash_attn_ext(Q, K, V, g.cast(m, gl.F16), scale, 0.0, 0.0)
        return g.cont_2d(out, hd * n_head, n_new)
    KQ = g.soft_max_ext(g.mul_mat(K, Q), m, scale, 0.0)
    V_trans = g.cont_3d(g.permute(V_full, 1, 2, 0, 3), n_kv, hd, n_head_kv)
    KQV = g.mul_mat(V_trans, KQ)
    return g.cont_2d(g.permute(KQV, 0, 2, 1, 3), hd * n_head, n_new)


def moe_ffn_graph(g, y, router, gate_exps, up_exps, down_exps, k, residual=None):
    """The routed expert FFN of model.cpp's build_moe_ffn (softmax router, top-k, renormalized
    weights, mul_mat_id gate/up/down with SiLU, weighted sum over the slots in order)."""
    core = gl.libs()["core"]
    tt = lambda t: t.contents
    n_embd, n_tok = tt(y).ne[0], tt(y).ne[1]
    n_expert = tt(router).ne[1]
    probs = g.soft_max_ext(g.mul_mat(router, y), None, 1.0, 0.0)
    sel = g.top_k(probs, k)
    w = g.get_rows(g.reshape_3d(probs, 1, n_expert, n_tok), sel)
    w = g.reshape_2d(w, k, n_tok)
    w = g.div(w, g.sum_rows(w))
    w = g.reshape_3d(w, 1, k, n_tok)
    x = g.reshape_3d(y, n_embd, 1, n_tok)
    act = g.mul(g.silu(g.mul_mat_id(gate_exps, x, sel)), g.mul_mat_id(up_exps, x, sel))
    experts = g.mul(g.mul_mat_id(down_exps, act, sel), w)
    nb1, nb2 = tt(experts).nb[1], tt(experts).nb[2]
    out = g.view_2d(experts, n_embd, n_tok, nb2, 0)
    for i in range(1, k):
        out = g.add(out, g.view_2d(experts, n_embd, n_tok, nb2, i * nb1))
    return g.add(out, residual) if residual is not None else out


# ---- node-by-node capture (debugging / parity localization) ----
EVAL_CB = C.CFUNCTYPE(C.c_bool, gl.T, C.c_bool, C.c_void_p)
OP_NAMES = ["NONE", "DUP", "ADD", "MUL", "SCALE", "SQR", "RMS_NORM", "MUL_MAT", "MUL_MAT_ID", "CPY", "CONT", "RESHAPE",
            "VIEW", "PERMUTE", "TRANSPOSE", "GET_ROWS", "SOFT_MAX", "ROPE", "FLASH_ATTN_EXT", "ARGMAX", "UNARY",
            "DIV", "SUM_ROWS", "ARGSORT"]
NOOP = {"NONE", "RESHAPE", "VIEW", "PERMUTE", "TRANSPOSE"}


def capture(backend, store: list):
    """Record (op, shape, f32 data) of every node the backend reports; returns the callback object
    (keep it alive while the backend computes)."""
    core = gl.libs()["core"]

    def cb(t, ask, user):
        tt = t.contents
        op = OP_NAMES[tt.op] if tt.op < len(OP_NAMES) else str(tt.op)
        if op in NOOP:
            return True
        shape = tuple(tt.ne[i] for i in range(4))
        if tt.type == gl.F32 and core.ggml_is_contiguous(t):
            n = core.ggml_nbytes(t) // 4
            a = np.empty(n, dtype=np.float32)
            core.ggml_backend_tensor_get(t, ptr(a), 0, n * 4)
        else:
            a = None
        store.append((op, shape, a))
        return True

    f = EVAL_CB(cb)
    core.ggml_backend_set_eval_callback(backend, f, None)
    return f


def first_divergence(a: list, b: list, tol=1e-4):
    """Compare two captured sequences (same graph); returns list of (i, op, shape, err) above tol."""
    out = []
    for i, ((oa, sa, xa), (ob, sb, xb)) in enumerate(zip(a, b)):
        if oa != ob or sa != sb:
            out.append((i, f"{oa}/{ob}", sa, float("nan")))
            break
        if xa is not None and xb is not None and xa.size == xb.size:
            e = rel_err(xa, xb)
            if e > tol:
                out.append((i, oa, sa, e))
    return out
