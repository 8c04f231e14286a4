"""Python bindings (ctypes) of the MI355X-native GGML-Loader build.

The product is the set of C-ABI shared libraries built in-tree under ``lib/``:

* ``libggml.so``        ggml core (tensors, graphs, GGUF, graph allocator, backend plumbing)
* ``libggml-hip.so``    the gfx950 HIP backend (``ggml_backend_hip_*``)
* ``libggml-loader.so`` the forward-pass runtime and synthetic-model writer (``gl_*``)

This module only loads them and declares their signatures; every computation happens in the
native code. Loading fails loudly if a library is missing (run ``build()`` first).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
# GGML_LOADER_LIB_DIR: another build of the same libraries (the sanitized one, _asan/lib)
LIB_DIR = os.environ.get("GGML_LOADER_LIB_DIR") or os.path.join(PKG_DIR, "lib")
BIN_DIR = os.path.join(PKG_DIR, "bin")

# ggml type ids (GGUF on-disk ids)
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, I32, BF16 = 0, 1, 2, 8, 12, 13, 14, 15, 26, 30
ROPE_NORMAL, ROPE_NEOX = 0, 2
SORT_ASC, SORT_DESC = 0, 1
UNARY_SILU = 1

_libs: dict | None = None


def build(jobs: int = 8) -> None:
    """Compile the product libraries (hipcc for gfx950 + g++) in-tree."""
    subprocess.run(["make", "-C", PKG_DIR, f"-j{jobs}"], check=True)


class ggml_init_params(C.Structure):
    _fields_ = [("mem_size", C.c_size_t), ("mem_buffer", C.c_void_p), ("no_alloc", C.c_bool)]


GGML_MAX_NAME = 128


class ggml_tensor(C.Structure):
    pass


ggml_tensor._fields_ = [
    ("type", C.c_int),
    ("buffer", C.c_void_p),
    ("ne", C.c_int64 * 4),
    ("nb", C.c_size_t * 4),
    ("op", C.c_int),
    ("op_params", C.c_int32 * 16),
    ("flags", C.c_int32),
    ("src", C.POINTER(ggml_tensor) * 10),
    ("view_src", C.POINTER(ggml_tensor)),
    ("view_offs", C.c_size_t),
    ("data", C.c_void_p),
    ("name", C.c_char * GGML_MAX_NAME),
    ("extra", C.c_void_p),
    ("padding", C.c_char * 8),
]

T = C.POINTER(ggml_tensor)


class ggml_hip_sampler_params(C.Structure):
    _fields_ = [("temp", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float), ("repeat_penalty", C.c_float),
                ("repeat_last_n", C.c_int32)]


class gl_sampler_params(C.Structure):
    _fields_ = [("temp", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float), ("repeat_penalty", C.c_float),
                ("repeat_last_n", C.c_int32), ("seed", C.c_uint32)]


class gl_synth_params(C.Structure):
    _fields_ = [
        ("arch", C.c_char_p),
        ("n_embd", C.c_int64), ("n_layer", C.c_int64), ("n_head", C.c_int64), ("n_head_kv", C.c_int64),
        ("head_dim", C.c_int64), ("n_ff", C.c_int64), ("n_vocab", C.c_int64), ("n_ctx_train", C.c_int64),
        ("n_expert", C.c_int64), ("n_expert_used", C.c_int64), ("n_ff_exp", C.c_int64),
        ("rope_theta", C.c_float), ("rms_eps", C.c_float),
        ("wtype", C.c_int32), ("embd_type", C.c_int32), ("output_type", C.c_int32), ("tied_output", C.c_int32),
        ("w_std", C.c_float), ("norm_std", C.c_float),
        ("seed", C.c_uint64), ("n_threads", C.c_int32), ("share_experts", C.c_int32),
        ("rope_scaling_orig_ctx", C.c_int32), ("rope_attn_factor", C.c_float), ("kquant_mix", C.c_int32),
    ]


def _sig(lib, name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)
    return f


def _declare(core, hip, loader):
    vp, sz, i64, i32, f32 = C.c_void_p, C.c_size_t, C.c_int64, C.c_int, C.c_float
    _sig(core, "ggml_init", vp, ggml_init_params)
    _sig(core, "ggml_free", None, vp)
    _sig(core, "ggml_tensor_overhead", sz)
    _sig(core, "ggml_graph_overhead", sz)
    _sig(core, "ggml_type_size", sz, i32)
    _sig(core, "ggml_blck_size", i64, i32)
    _sig(core, "ggml_row_size", sz, i32, i64)
    _sig(core, "ggml_type_name", C.c_char_p, i32)
    _sig(core, "ggml_nbytes", sz, T)
    _sig(core, "ggml_nelements", i64, T)
    _sig(core, "ggml_is_contiguous", C.c_bool, T)
    _sig(core, "ggml_new_tensor_1d", T, vp, i32, i64)
    _sig(core, "ggml_new_tensor_2d", T, vp, i32, i64, i64)
    _sig(core, "ggml_new_tensor_3d", T, vp, i32, i64, i64, i64)
    _sig(core, "ggml_new_tensor_4d", T, vp, i32, i64, i64, i64, i64)
    _sig(core, "ggml_set_name", T, T, C.c_char_p)
    _sig(core, "ggml_set_input", None, T)
    _sig(core, "ggml_set_output", None, T)
    _sig(core, "ggml_get_tensor", T, vp, C.c_char_p)
    _sig(core, "ggml_get_rows", T, vp, T, T)
    _sig(core, "ggml_rms_norm", T, vp, T, f32)
    _sig(core, "ggml_mul", T, vp, T, T)
    _sig(core, "ggml_add", T, vp, T, T)
    _sig(core, "ggml_scale", T, vp, T, f32)
    _sig(core, "ggml_mul_mat", T, vp, T, T)
    _sig(core, "ggml_mul_mat_id", T, vp, T, T, T)
    _sig(core, "ggml_reshape_2d", T, vp, T, i64, i64)
    _sig(core, "ggml_reshape_3d", T, vp, T, i64, i64, i64)
    _sig(core, "ggml_view_1d", T, vp, T, i64, sz)
    _sig(core, "ggml_view_2d", T, vp, T, i64, i64, sz, sz)
    _sig(core, "ggml_view_3d", T, vp, T, i64, i64, i64, sz, sz, sz)
    _sig(core, "ggml_permute", T, vp, T, i32, i32, i32, i32)
    _sig(core, "ggml_transpose", T, vp, T)
    _sig(core, "ggml_cont", T, vp, T)
    _sig(core, "ggml_cont_2d", T, vp, T, i64, i64)
    _sig(core, "ggml_cont_3d", T, vp, T, i64, i64, i64)
    _sig(core, "ggml_cpy", T, vp, T, T)
    _sig(core, "ggml_cast", T, vp, T, i32)
    _sig(core, "ggml_rope_ext", T, vp, T, T, T, i32, i32, i32, f32, f32, f32, f32, f32, f32)
    _sig(core, "ggml_soft_max_ext", T, vp, T, T, f32, f32)
    _sig(core, "ggml_silu", T, vp, T)
    _sig(core, "ggml_unary", T, vp, T, i32)
    _sig(core, "ggml_flash_attn_ext", T, vp, T, T, T, T, f32, f32, f32)
    _sig(core, "ggml_argmax", T, vp, T)
    _sig(core, "ggml_div", T, vp, T, T)
    _sig(core, "ggml_sub", T, vp, T, T)
    _sig(core, "ggml_abs", T, vp, T)
    _sig(core, "ggml_softplus", T, vp, T)
    _sig(core, "ggml_l2_norm", T, vp, T, f32)
    _sig(core, "ggml_concat", T, vp, T, T, i32)
    _sig(core, "ggml_swiglu_split", T, vp, T, T)
    _sig(core, "ggml_ssm_conv", T, vp, T, T)
    _sig(core, "ggml_ssm_scan", T, vp, T, T, T, T, T, T, T, i32)
    _sig(core, "ggml_gated_delta_net", T, vp, T, T, T, T, T, T, i32)
    _sig(core, "ggml_sum_rows", T, vp, T)
    _sig(core, "ggml_argsort", T, vp, T, i32)
    _sig(core, "ggml_top_k", T, vp, T, i32)
    _sig(core, "ggml_new_graph", vp, vp)
    _sig(core, "ggml_build_forward_expand", None, vp, T)
    _sig(core, "ggml_graph_n_nodes", i32, vp)
    _sig(core, "ggml_graph_node", T, vp, i32)
    _sig(core, "ggml_fp16_to_fp32", f32, C.c_uint16)
    _sig(core, "ggml_fp32_to_fp16", C.c_uint16, f32)
    _sig(core, "ggml_quantize_chunk", sz, i32, vp, vp, i64, i64, i64, vp)
    _sig(core, "ggml_dequantize_row", C.c_bool, i32, vp, vp, i64)
    _sig(core, "ggml_backend_alloc_ctx_tensors", vp, vp, vp)
    _sig(core, "ggml_backend_buffer_free", None, vp)
    _sig(core, "ggml_backend_buffer_get_size", sz, vp)
    _sig(core, "ggml_backend_buffer_clear", None, vp, C.c_uint8)
    _sig(core, "ggml_backend_tensor_set", None, T, vp, sz, sz)
    _sig(core, "ggml_backend_tensor_get", None, T, vp, sz, sz)
    _sig(core, "ggml_backend_graph_compute", i32, vp, vp)
    _sig(core, "ggml_backend_free", None, vp)
    _sig(core, "ggml_backend_name", C.c_char_p, vp)
    _sig(core, "ggml_backend_get_default_buffer_type", vp, vp)
    _sig(core, "ggml_backend_init_by_name", vp, C.c_char_p, C.c_char_p)
    _sig(core, "ggml_backend_load", C.c_bool, C.c_char_p)
    _sig(core, "ggml_backend_set_eval_callback", None, vp, vp, vp)
    _sig(core, "ggml_gallocr_new", vp, vp)
    _sig(core, "ggml_gallocr_free", None, vp)
    _sig(core, "ggml_gallocr_alloc_graph", C.c_bool, vp, vp)
    _sig(core, "gguf_init_empty", vp)
    _sig(core, "gguf_free", None, vp)
    _sig(core, "gguf_set_val_u32", None, vp, C.c_char_p, C.c_uint32)
    _sig(core, "gguf_set_val_f32", None, vp, C.c_char_p, f32)
    _sig(core, "gguf_set_val_str", None, vp, C.c_char_p, C.c_char_p)
    _sig(core, "gguf_set_arr_data", None, vp, C.c_char_p, i32, vp, sz)
    _sig(core, "gguf_set_arr_str", None, vp, C.c_char_p, C.POINTER(C.c_char_p), sz)
    _sig(core, "gguf_add_tensor", None, vp, T)
    _sig(core, "gguf_write_to_file", C.c_bool, vp, C.c_char_p, C.c_bool)

    class gguf_init_params(C.Structure):
        _fields_ = [("no_alloc", C.c_bool), ("ctx", C.POINTER(C.c_void_p))]

    core.gguf_init_params = gguf_init_params
    _sig(core, "gguf_init_from_file", vp, C.c_char_p, gguf_init_params)
    _sig(core, "gguf_get_version", C.c_uint32, vp)
    _sig(core, "gguf_get_alignment", sz, vp)
    _sig(core, "gguf_get_data_offset", sz, vp)
    _sig(core, "gguf_get_n_kv", i64, vp)
    _sig(core, "gguf_find_key", i64, vp, C.c_char_p)
    _sig(core, "gguf_get_key", C.c_char_p, vp, i64)
    _sig(core, "gguf_get_kv_type", i32, vp, i64)
    _sig(core, "gguf_get_arr_type", i32, vp, i64)
    _sig(core, "gguf_get_val_u32", C.c_uint32, vp, i64)
    _sig(core, "gguf_get_val_f32", f32, vp, i64)
    _sig(core, "gguf_get_val_str", C.c_char_p, vp, i64)
    _sig(core, "gguf_get_arr_n", sz, vp, i64)
    _sig(core, "gguf_get_arr_data", vp, vp, i64)
    _sig(core, "gguf_get_arr_str", C.c_char_p, vp, i64, sz)
    _sig(core, "gguf_get_n_tensors", i64, vp)
    _sig(core, "gguf_get_tensor_name", C.c_char_p, vp, i64)
    _sig(core, "gguf_get_tensor_type", i32, vp, i64)
    _sig(core, "gguf_get_tensor_offset", sz, vp, i64)
    _sig(core, "gguf_get_tensor_size", sz, vp, i64)
    _sig(core, "gguf_get_tensor_n_dims", i32, vp, i64)
    _sig(core, "gguf_get_tensor_ne", C.POINTER(C.c_int64), vp, i64)

    _sig(hip, "ggml_backend_hip_get_device_count", i32)
    _sig(hip, "ggml_backend_hip_get_device_description", None, i32, C.c_char_p, sz)
    _sig(hip, "ggml_backend_hip_init", vp, i32)
    _sig(hip, "ggml_backend_is_hip", C.c_bool, vp)
    _sig(hip, "ggml_backend_hip_graph_compute_static", i32, vp, vp)
    _sig(hip, "ggml_backend_hip_sample", i32, vp, vp, i64, C.POINTER(ggml_hip_sampler_params), vp, sz,
         C.c_double, C.POINTER(C.c_int32), C.POINTER(C.c_bool))
    _sig(hip, "ggml_backend_hip_set_fusion", None, vp, C.c_bool)
    _sig(hip, "ggml_backend_hip_set_profiling", None, vp, C.c_bool)
    _sig(hip, "ggml_backend_hip_set_profile_filter", None, vp, C.c_char_p)
    _sig(hip, "ggml_backend_hip_set_profile_sampling", None, vp, i32)
    _sig(hip, "ggml_backend_hip_reset_profile", None, vp)
    _sig(hip, "ggml_backend_hip_profile_count", i32, vp)
    _sig(hip, "ggml_backend_hip_profile_entry", C.c_bool, vp, i32, C.c_char_p, sz, C.POINTER(i64),
         C.POINTER(C.c_double), C.POINTER(C.c_double))

    eb = C.c_char_p
    _sig(loader, "gl_session_open", vp, C.c_char_p, C.c_char_p, i32, i64, i32, eb, sz)
    _sig(loader, "gl_session_free", None, vp)
    _sig(loader, "gl_session_backend", vp, vp)
    _sig(loader, "gl_session_get", i64, vp, C.c_char_p)
    _sig(loader, "gl_forward_step", i32, vp, i64, C.POINTER(C.c_int32), i64, C.POINTER(C.c_float), eb, sz)
    _sig(loader, "gl_decode_loop", i32, vp, i64, C.c_int32, i32, i32, C.POINTER(C.c_int32), C.POINTER(C.c_double), eb, sz)
    _sig(loader, "gl_generate", i32, vp, i64, C.POINTER(C.c_int32), i64, i32, C.POINTER(gl_sampler_params),
         C.POINTER(C.c_int32), C.POINTER(C.c_double), eb, sz)
    _sig(loader, "gl_kv_fill_random", i32, vp, i64, C.c_uint64, eb, sz)
    _sig(loader, "gl_kv_read", i32, vp, i32, i32, vp, sz, sz)
    _sig(loader, "gl_synth_model", i32, C.c_char_p, C.POINTER(gl_synth_params), eb, sz)
    _sig(loader, "gl_fill_normal", None, C.POINTER(C.c_float), i64, C.c_uint64, i64, f32, f32)


def libs() -> dict:
    """Load (once) and return {'core', 'hip', 'loader'} CDLL handles."""
    global _libs
    if _libs is None:
        paths = {k: os.path.join(LIB_DIR, f) for k, f in
                 (("core", "libggml.so"), ("hip", "libggml-hip.so"), ("loader", "libggml-loader.so"))}
        for k, p in paths.items():
            if not os.path.exists(p):
                raise RuntimeError(f"{p} is missing: build the native libraries first (ggml-loader_amd build())")
        mode = C.RTLD_GLOBAL
        core = C.CDLL(paths["core"], mode=mode)
        hip = C.CDLL(paths["hip"], mode=mode)
        loader = C.CDLL(paths["loader"], mode=mode)
        _declare(core, hip, loader)
        _libs = {"core": core, "hip": hip, "loader": loader}
    return _libs


def hip_device_count() -> int:
    return int(libs()["hip"].ggml_backend_hip_get_device_count())


def hip_sample(backend, logits_tensor, row: int, recent, u: float, *, temp: float, top_k: int = 40,
               top_p: float = 0.95, repeat_penalty: float = 1.0, repeat_last_n: int = 64):
    """ggml_backend_hip_sample on one row of an F32 tensor in the backend's buffer:
    (token id, whether u was used)."""
    import numpy as np
    r = np.ascontiguousarray(np.asarray(recent, dtype=np.int32))
    sp = ggml_hip_sampler_params(temp, top_k, top_p, repeat_penalty, repeat_last_n)
    tok, used = C.c_int32(-1), C.c_bool(False)
    st = libs()["hip"].ggml_backend_hip_sample(backend, logits_tensor, row, C.byref(sp), r.ctypes.data_as(C.c_void_p),
                                               r.size, u, C.byref(tok), C.byref(used))
    if st != 0:
        raise RuntimeError(f"ggml_backend_hip_sample failed ({st})")
    return int(tok.value), bool(used.value)


def hip_backend(device: int = 0):
    b = libs()["hip"].ggml_backend_hip_init(device)
    if not b:
        raise RuntimeError(f"ggml_backend_hip_init({device}) failed (no HIP device?)")
    return b


def profile(backend) -> dict:
    """Per-kernel stats accumulated while profiling was on: name -> (launches, ms, bytes)."""
    h = libs()["hip"]
    out = {}
    name = C.create_string_buffer(128)
    for i in range(h.ggml_backend_hip_profile_count(backend)):
        n, ms, by = C.c_int64(), C.c_double(), C.c_double()
        if h.ggml_backend_hip_profile_entry(backend, i, name, 128, C.byref(n), C.byref(ms), C.byref(by)):
            out[name.value.decode()] = (n.value, ms.value, by.value)
    return out


# synthetic model shapes of the benchmark configurations (BASELINE.json configs[1..4])
CONFIGS = {
    "llama3b": dict(arch="llama", n_embd=3072, n_layer=28, n_head=24, n_head_kv=8, head_dim=128, n_ff=8192,
                    n_vocab=128256, n_ctx_train=131072, rope_theta=500000.0, rms_eps=1e-5, wtype=Q4_0),
    "qwen3": dict(arch="qwen3", n_embd=2560, n_layer=36, n_head=32, n_head_kv=8, head_dim=128, n_ff=9728,
                  n_vocab=151936, n_ctx_train=40960, rope_theta=1e6, rms_eps=1e-6, wtype=Q4_K),
    "phi3mini": dict(arch="phi3", n_embd=3072, n_layer=32, n_head=32, n_head_kv=32, head_dim=96, n_ff=8192,
                     n_vocab=32064, n_ctx_train=4096, rope_theta=10000.0, rms_eps=1e-5, wtype=Q8_0),
    "qwen3moe": dict(arch="qwen3moe", n_embd=2048, n_layer=48, n_head=32, n_head_kv=4, head_dim=128, n_ff=6144,
                     n_vocab=151936, n_ctx_train=40960, rope_theta=1e6, rms_eps=1e-6, wtype=Q4_K,
                     n_expert=128, n_expert_used=8, n_ff_exp=768),
}


def synth_model(path: str, *, arch: str, n_embd: int, n_layer: int, n_head: int, n_head_kv: int, head_dim: int,
                n_ff: int, n_vocab: int, n_ctx_train: int = 4096, rope_theta: float = 10000.0, rms_eps: float = 1e-5,
                wtype: int = Q4_0, embd_type: int | None = None, output_type: int | None = None, tied: bool = False,
                w_std: float = 0.02, norm_std: float = 0.01, seed: int = 1, n_threads: int = 0, n_expert: int = 0,
                n_expert_used: int = 0, n_ff_exp: int = 0, share_experts: bool = False,
                rope_scaling_orig_ctx: int = 0, rope_attn_factor: float = 1.0, kquant_mix: int = 0) -> None:
    """Write a seeded synthetic GGUF model (weights ~ N(0, w_std), quantized by the ggml reference quantizers)."""
    p = gl_synth_params()
    p.arch = arch.encode()
    p.n_embd, p.n_layer, p.n_head, p.n_head_kv = n_embd, n_layer, n_head, n_head_kv
    p.head_dim, p.n_ff, p.n_vocab, p.n_ctx_train = head_dim, n_ff, n_vocab, n_ctx_train
    p.n_expert, p.n_expert_used, p.n_ff_exp = n_expert, n_expert_used, n_ff_exp
    p.rope_theta, p.rms_eps = rope_theta, rms_eps
    p.wtype = wtype
    p.embd_type = wtype if embd_type is None else embd_type
    p.output_type = wtype if output_type is None else output_type
    p.tied_output = 1 if tied else 0
    p.w_std, p.norm_std, p.seed, p.n_threads = w_std, norm_std, seed, n_threads
    p.share_experts = 1 if share_experts else 0
    p.rope_scaling_orig_ctx, p.rope_attn_factor = rope_scaling_orig_ctx, rope_attn_factor
    p.kquant_mix = kquant_mix
    err = C.create_string_buffer(512)
    if libs()["loader"].gl_synth_model(path.encode(), C.byref(p), err, 512) != 0:
        raise RuntimeError(err.value.decode())


class Session:
    """A loaded model + KV cache + decode session on one backend (the cmd_bench/cmd_run setup)."""

    def __init__(self, model_path: str, backend: str = "hip", n_ctx: int = 512, n_threads: int = 8,
                 flash_attn: bool = False):
        err = C.create_string_buffer(512)
        self._l = libs()["loader"]
        self.h = self._l.gl_session_open(model_path.encode(), backend.encode(), n_threads, n_ctx, int(flash_attn), err, 512)
        if not self.h:
            raise RuntimeError(err.value.decode())
        self.n_vocab = self.get("n_vocab")

    def get(self, name: str) -> int:
        return int(self._l.gl_session_get(self.h, name.encode()))

    @property
    def backend(self):
        return self._l.gl_session_backend(self.h)

    def forward(self, n_past: int, tokens):
        import numpy as np
        toks = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        out = np.empty(self.n_vocab, dtype=np.float32)
        err = C.create_string_buffer(512)
        rc = self._l.gl_forward_step(self.h, n_past, toks.ctypes.data_as(C.POINTER(C.c_int32)), len(toks),
                                     out.ctypes.data_as(C.POINTER(C.c_float)), err, 512)
        if rc != 0:
            raise RuntimeError(err.value.decode())
        return out

    def decode_loop(self, n_past: int, first_token: int, n_steps: int, fixed_pos: bool = False):
        import numpy as np
        toks = np.zeros(max(n_steps, 1), dtype=np.int32)
        secs = C.c_double()
        err = C.create_string_buffer(512)
        rc = self._l.gl_decode_loop(self.h, n_past, first_token, n_steps, int(fixed_pos),
                                    toks.ctypes.data_as(C.POINTER(C.c_int32)), C.byref(secs), err, 512)
        if rc != 0:
            raise RuntimeError(err.value.decode())
        return toks[:n_steps], secs.value

    def generate(self, n_past: int, prompt, n_steps: int, *, temp: float, top_k: int = 40, top_p: float = 0.95,
                 repeat_penalty: float = 1.0, repeat_last_n: int = 64, seed: int = 1):
        """gl_generate: the prompt at n_past, then n_steps sampled tokens (the first from the prompt's
        logits); returns (tokens, seconds)."""
        import numpy as np
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        toks = np.zeros(max(n_steps, 1), dtype=np.int32)
        sp = gl_sampler_params(temp, top_k, top_p, repeat_penalty, repeat_last_n, seed)
        secs = C.c_double()
        err = C.create_string_buffer(512)
        rc = self._l.gl_generate(self.h, n_past, p.ctypes.data_as(C.POINTER(C.c_int32)), len(p), n_steps, C.byref(sp),
                                 toks.ctypes.data_as(C.POINTER(C.c_int32)), C.byref(secs), err, 512)
        if rc != 0:
            raise RuntimeError(err.value.decode())
        return toks[:n_steps], secs.value

    def kv_fill_random(self, n_pos: int, seed: int = 7) -> None:
        err = C.create_string_buffer(512)
        if self._l.gl_kv_fill_random(self.h, n_pos, seed, err, 512) != 0:
            raise RuntimeError(err.value.decode())

    def close(self) -> None:
        if self.h:
            self._l.gl_session_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
