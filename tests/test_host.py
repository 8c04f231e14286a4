"""Host-side tests that run without a GPU: the C-ABI libraries load and export every declared
symbol, the GGUF reader/writer and synthetic models, the graph allocator, graph-op semantics, the
runtime's error paths, and whole forward_steps of the oracle against an independent float64 model.
"""
import ctypes as C
import hashlib
import os
import re
import subprocess

import numpy as np
import pytest

from gguf_py import GGUFFile
from gl import ORACLE_SO, ROOT, Graph, cpu_backend, gl, ptr, rel_err
from ref_model import RefModel

INCLUDE = os.path.join(ROOT, "include")
LIB_DIR = os.path.join(ROOT, "ggml-loader_amd", "lib")

# which library implements each public header
HEADER_LIB = {
    "ggml.h": "libggml.so", "gguf.h": "libggml.so", "ggml-alloc.h": "libggml.so", "ggml-backend.h": "libggml.so",
    "ggml-hip.h": "libggml-hip.so", "ggml-loader.h": "libggml-loader.so", "ggml-cpu.h": ORACLE_SO,
    "ggml-vulkan.h": "libggml.so",
}

TINY = {
    "llama": dict(arch="llama", n_embd=256, n_layer=2, n_head=8, n_head_kv=2, head_dim=64, n_ff=512,
                  n_vocab=600, rope_theta=500000.0, wtype=gl.Q4_0),
    "qwen3": dict(arch="qwen3", n_embd=512, n_layer=2, n_head=8, n_head_kv=2, head_dim=128, n_ff=768,
                  n_vocab=700, rope_theta=1e6, rms_eps=1e-6, wtype=gl.Q4_K),
    "qwen2": dict(arch="qwen2", n_embd=256, n_layer=2, n_head=4, n_head_kv=2, head_dim=64, n_ff=512,
                  n_vocab=500, rope_theta=1e6, wtype=gl.Q8_0),
    "phi3": dict(arch="phi3", n_embd=384, n_layer=2, n_head=4, n_head_kv=4, head_dim=96, n_ff=512,
                 n_vocab=400, wtype=gl.Q8_0),
    "qwen3moe": dict(arch="qwen3moe", n_embd=256, n_layer=2, n_head=8, n_head_kv=2, head_dim=64, n_ff=512,
                     n_vocab=500, n_expert=16, n_expert_used=4, n_ff_exp=256, rope_theta=1e6, rms_eps=1e-6,
                     wtype=gl.Q4_K),
}


@pytest.fixture(scope="module", autouse=True)
def oracle_loaded():
    gl.libs()["core"].ggml_backend_free(cpu_backend(1))


def declared_functions(header):
    text = open(os.path.join(INCLUDE, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"^\s*#[^\n]*", "", text, flags=re.M)
    names = []
    for decl in re.findall(r"GGML_API\s+([^;{]*?)\(", text, flags=re.S):
        m = re.search(r"(\w+)\s*$", decl)
        if m:
            names.append(m.group(1))
    return names


def exported(lib_path):
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


@pytest.mark.parametrize("header", sorted(HEADER_LIB))
def test_library_exports_every_declared_symbol(header):
    gl.libs()
    lib = HEADER_LIB[header]
    path = lib if os.path.isabs(lib) else os.path.join(LIB_DIR, lib)
    names = declared_functions(header)
    assert names, header
    missing = sorted(set(names) - exported(path))
    assert not missing, (header, missing)


def test_hip_backend_entry_points_without_gpu():
    """On a machine without a GPU the hip entry points report zero devices and the runtime refuses
    the hip backend with an error instead of falling back to any CPU path."""
    hip = gl.libs()["hip"]
    if hip.ggml_backend_hip_get_device_count() > 0:
        pytest.skip("a GPU is present")
    assert not hip.ggml_backend_hip_init(0)
    with pytest.raises(RuntimeError, match="no HIP device"):
        gl.Session("/nonexistent.gguf", "hip")


# ---- GGUF ------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("host_models")
    out = {}
    for name, cfg in TINY.items():
        p = str(d / f"{name}.gguf")
        gl.synth_model(p, seed=5, w_std=0.06, **cfg)
        out[name] = p
    return out


def read_with_c(path):
    core = gl.libs()["core"]
    ctx = core.gguf_init_from_file(path.encode(), core.gguf_init_params(True, None))
    assert ctx
    try:
        info = {"version": core.gguf_get_version(ctx), "alignment": core.gguf_get_alignment(ctx),
                "data_offset": core.gguf_get_data_offset(ctx), "keys": [], "tensors": {}}
        for i in range(core.gguf_get_n_kv(ctx)):
            info["keys"].append(core.gguf_get_key(ctx, i).decode())
        for i in range(core.gguf_get_n_tensors(ctx)):
            name = core.gguf_get_tensor_name(ctx, i).decode()
            nd = core.gguf_get_tensor_n_dims(ctx, i)
            info["tensors"][name] = (core.gguf_get_tensor_type(ctx, i), list(core.gguf_get_tensor_ne(ctx, i)[:nd]),
                                     core.gguf_get_tensor_offset(ctx, i), core.gguf_get_tensor_size(ctx, i))
        return info
    finally:
        core.gguf_free(ctx)


@pytest.mark.parametrize("arch", list(TINY))
def test_gguf_reader_agrees_with_independent_parser(models, arch):
    path = models[arch]
    py = GGUFFile(path)
    c = read_with_c(path)
    assert c["version"] == py.version == 3
    assert c["alignment"] == 32 and c["data_offset"] == py.data_offset
    assert c["keys"] == list(py.kv)
    assert list(c["tensors"]) == list(py.tensors)
    for name, (ttype, ne, off) in py.tensors.items():
        ct, cne, coff, csize = c["tensors"][name]
        assert (ct, cne, coff) == (ttype, ne, off), name
        assert off % 32 == 0
        assert csize == py.raw(name)[0].size
    assert py.data_offset + max(o + c["tensors"][n][3] for n, (_, _, o) in py.tensors.items()) <= os.path.getsize(path)


def test_gguf_writer_all_value_types(tmp_path):
    core = gl.libs()["core"]
    ctx = core.gguf_init_empty()
    core.gguf_set_val_u32(ctx, b"a.u32", 4000000000)
    core.gguf_set_val_f32(ctx, b"a.f32", C.c_float(-1.25))
    core.gguf_set_val_str(ctx, b"a.str", "ünïcode".encode())
    arr = np.array([1, -2, 3], dtype=np.int32)
    core.gguf_set_arr_data(ctx, b"a.arr_i32", 5, ptr(arr), 3)
    strs = (C.c_char_p * 2)(b"x", b"yz")
    core.gguf_set_arr_str(ctx, b"a.arr_str", strs, 2)
    path = str(tmp_path / "kv.gguf")
    assert core.gguf_write_to_file(ctx, path.encode(), False)
    core.gguf_free(ctx)
    py = GGUFFile(path)
    assert py.kv == {"a.u32": 4000000000, "a.f32": -1.25, "a.str": "ünïcode", "a.arr_i32": [1, -2, 3],
                     "a.arr_str": ["x", "yz"]}
    assert py.kv_types == {"a.u32": 4, "a.f32": 6, "a.str": 8, "a.arr_i32": 9, "a.arr_str": 9}


def test_synthetic_model_is_deterministic(tmp_path):
    cfg = dict(TINY["llama"], n_layer=1)
    paths = [str(tmp_path / f"m{i}.gguf") for i in range(3)]
    for p, seed in zip(paths, (11, 11, 12)):
        gl.synth_model(p, seed=seed, **cfg)
    digest = [hashlib.sha256(open(p, "rb").read()).hexdigest() for p in paths]
    assert digest[0] == digest[1] != digest[2]
    # norm weights are 1 + N(0, 0.01); linear weights N(0, w_std) before quantization
    m = RefModel(paths[0])
    nw = m.w["blk.0.attn_norm.weight"]
    assert abs(nw.mean() - 1) < 3e-3 and 0.007 < nw.std() < 0.013
    wq = m.w["blk.0.attn_q.weight"]
    assert abs(wq.std() - 0.02) < 2e-3


def test_synthetic_shared_experts(tmp_path):
    """share_experts writes layer 0's expert tensors into every layer and changes nothing else."""
    cfg = dict(TINY["qwen3moe"], n_layer=3)
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    gl.synth_model(a, seed=3, **cfg)
    gl.synth_model(b, seed=3, share_experts=True, **cfg)
    fa, fb = GGUFFile(a), GGUFFile(b)
    assert fa.tensors == fb.tensors
    n_exp = 0
    for name in fa.tensors:
        ra, rb = fa.raw(name)[0], fb.raw(name)[0]
        if "_exps." in name:
            r0 = fb.raw("blk.0." + name.split(".", 2)[2])[0]
            assert np.array_equal(rb, r0), name
            assert np.array_equal(ra, rb) == name.startswith("blk.0."), name
            n_exp += 1
        else:
            assert np.array_equal(ra, rb), name
    assert n_exp == 9


def test_moe_graph_capacity(tmp_path):
    """A 48-layer qwen3moe graph (about 60 tensors per layer more than a dense layer) fits the decode
    session's graph, at one token and at a 16-token step."""
    p = str(tmp_path / "moe48.gguf")
    gl.synth_model(p, seed=2, **dict(TINY["qwen3moe"], n_layer=48, n_embd=64, n_head=2, n_head_kv=1, head_dim=32,
                                     n_expert=8, n_expert_used=2, n_ff_exp=64, n_vocab=64, wtype=gl.Q8_0))
    with gl.Session(p, "cpu", n_ctx=32, n_threads=4) as s:
        one = s.forward(0, [5])
        many = s.forward(1, list(range(16)))
    assert np.all(np.isfinite(one)) and np.all(np.isfinite(many))


def test_seeded_normal_generator():
    from gl import randn
    a = randn(200000, 7)
    assert np.array_equal(a, randn(200000, 7))
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    out = np.empty(100, dtype=np.float32)
    gl.libs()["loader"].gl_fill_normal(out.ctypes.data_as(C.POINTER(C.c_float)), 100, 7, 1000, 0.0, 1.0)
    assert np.array_equal(out, a[1000:1100])    # counter-based: any window can be generated alone


# ---- graph allocator and op semantics --------------------------------------------------------

def test_gallocr_reuses_memory_and_keeps_results():
    core = gl.libs()["core"]
    cpu = cpu_backend(2)
    n = 4096
    x = np.random.default_rng(1).standard_normal(n).astype(np.float32)

    def chain(g, xt):
        y = xt
        for i in range(12):
            y = g.add(g.scale(y, 1.01), xt) if i % 2 else g.mul(y, xt)
        return y

    with Graph() as g:
        xt = g.tensor(gl.F32, n, data=x)
        expect = g.compute(cpu, chain(g, xt))
    with Graph() as g:
        xt = g.tensor(gl.F32, n)
        core.ggml_set_input(xt)
        out = chain(g, xt)
        gf = core.ggml_new_graph(g.ctx)
        core.ggml_build_forward_expand(gf, out)
        alloc = core.ggml_gallocr_new(core.ggml_backend_get_default_buffer_type(cpu))
        try:
            assert core.ggml_gallocr_alloc_graph(alloc, gf)
            core.ggml_gallocr_get_buffer_size.restype = C.c_size_t
            core.ggml_gallocr_get_buffer_size.argtypes = [C.c_void_p, C.c_int]
            size = core.ggml_gallocr_get_buffer_size(alloc, 0)
            # 25 tensors of 16 KiB would need 400 KiB without reuse; the chain needs a few live at once
            assert size <= 6 * n * 4, size
            core.ggml_backend_tensor_set(xt, ptr(x), 0, n * 4)
            assert core.ggml_backend_graph_compute(cpu, gf) == 0
            got = np.empty(n, dtype=np.float32)
            core.ggml_backend_tensor_get(out, ptr(got), 0, n * 4)
        finally:
            core.ggml_gallocr_free(alloc)
            core.ggml_backend_free(cpu)
    assert np.array_equal(got, expect)


def test_views_permute_cont_get_rows():
    cpu = cpu_backend(2)
    r = np.random.default_rng(2)
    a = r.standard_normal((5, 4, 6)).astype(np.float32)          # ggml ne = [6, 4, 5]
    ids = np.array([4, 0, 2, 2], dtype=np.int32)
    try:
        with Graph() as g:
            t = g.tensor(gl.F32, 6, 4, 5, data=a)
            p = g.cont(g.permute(t, 1, 2, 0, 3))                   # ne0 -> axis 1 etc.
            v = g.cont(g.view_2d(t, 3, 4, 6 * 4, 2 * 4))              # [3 elements from 2, 4 rows]
            rows = g.get_rows(g.reshape_2d(t, 6, 20), g.tensor(gl.I32, 4, data=ids))
            tr = g.cont(g.transpose(g.reshape_2d(t, 6, 20)))
            pr, vr, rr, trr = g.compute(cpu, [p, v, rows, tr])
    finally:
        gl.libs()["core"].ggml_backend_free(cpu)
    # permute(1,2,0): source axis 0 (ne0) goes to destination axis 1, ne1 -> 2, ne2 -> 0
    assert np.array_equal(pr.reshape(4, 6, 5), np.transpose(a, (1, 2, 0)))
    assert np.array_equal(vr.reshape(4, 3), a.reshape(20, 6)[:4, 2:5])
    assert np.array_equal(rr.reshape(4, 6), a.reshape(20, 6)[ids])
    assert np.array_equal(trr.reshape(6, 20), a.reshape(20, 6).T)


def test_broadcast_binary_ops():
    cpu = cpu_backend(2)
    r = np.random.default_rng(3)
    a = r.standard_normal((3, 2, 8)).astype(np.float32)
    b = r.standard_normal(8).astype(np.float32)
    c = r.standard_normal((1, 2, 8)).astype(np.float32)
    try:
        with Graph() as g:
            ta = g.tensor(gl.F32, 8, 2, 3, data=a)
            m, s = g.compute(cpu, [g.mul(ta, g.tensor(gl.F32, 8, data=b)), g.add(ta, g.tensor(gl.F32, 8, 2, 1, data=c))])
    finally:
        gl.libs()["core"].ggml_backend_free(cpu)
    assert np.array_equal(m.reshape(a.shape), a * b)
    assert np.array_equal(s.reshape(a.shape), a + c)


# ---- runtime ---------------------------------------------------------------------------------

def test_session_hparams_and_errors(models):
    with gl.Session(models["qwen3"], "cpu", n_ctx=16, n_threads=2) as s:
        assert [s.get(k) for k in ("n_embd", "n_layer", "n_head", "n_head_kv", "head_dim", "n_ff", "n_vocab", "n_ctx")] == \
               [512, 2, 8, 2, 128, 768, 700, 16]
        assert s.get("no_such_key") == -1
        with pytest.raises(RuntimeError, match="exceeds the KV cache"):
            s.forward(15, [1, 2])
        with pytest.raises(RuntimeError, match="no tokens"):
            s.forward(0, [])
    with pytest.raises(RuntimeError, match="unknown backend"):
        gl.Session(models["qwen3"], "vulkan")
    with pytest.raises(RuntimeError, match="failed to load"):
        gl.Session("/nonexistent/model.gguf", "cpu")


def test_decode_loop_matches_forward_steps(models):
    with gl.Session(models["llama"], "cpu", n_ctx=32, n_threads=4) as s:
        toks, secs = s.decode_loop(0, 1, 6)
    with gl.Session(models["llama"], "cpu", n_ctx=32, n_threads=4) as s:
        tok, seq = 1, []
        for i in range(6):
            tok = int(np.argmax(s.forward(i, [tok])))
            seq.append(tok)
    assert toks.tolist() == seq and secs > 0


@pytest.mark.parametrize("arch", list(TINY))
def test_oracle_forward_against_float64_model(models, arch):
    """Prefill of 7 tokens then 3 decode steps. ggml's roundings (Q8 activations, F16 KV and
    attention operands) keep the oracle within 6e-2 of the float64 model; the same model with the
    other RoPE pair layout is more than 0.2 away, so a layout or mapping mistake cannot pass."""
    prompt = [1, 17, 250, 3, 99, 4, 300]
    ref = RefModel(models[arch])
    other = RefModel(models[arch], rope_mode="normal" if arch != "llama" else "neox")
    checked = 0
    with gl.Session(models[arch], "cpu", n_ctx=32, n_threads=8) as s:
        lc = s.forward(0, prompt)
        lr, lo = ref.forward(0, prompt), other.forward(0, prompt)
        assert rel_err(lc, lr) < 6e-2 or ref.route_margin < 0.05
        assert rel_err(lc, lo) > 0.2
        tok = int(np.argmax(lc))
        for step in range(3):
            n_past = len(prompt) + step
            lc, lr = s.forward(n_past, [tok]), ref.forward(n_past, [tok])
            # an expert whose probability sits within rounding of the k-th one may route either way;
            # such steps only need to stay finite
            if ref.route_margin >= 0.05:
                assert rel_err(lc, lr) < 6e-2, (step, rel_err(lc, lr))
                checked += 1
            assert np.all(np.isfinite(lc))
            tok = int(np.argmax(lc))
    assert checked >= 1


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 exits with a message instead of a number."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""


def test_bench_pmc_summary_scales_by_the_copy_kernel(tmp_path):
    """The HBM traffic per launch: each counter (KiB per dispatch) scaled by what it reads for the
    copy kernel of known size, averaged over the matching dispatches."""
    import csv
    import importlib.util
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)

    def write(d, rows):
        os.makedirs(d / "run", exist_ok=True)
        with open(d / "run" / "x_counter_collection.csv", "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Counter_Value"])
            w.writeheader()
            for name, v in rows:
                w.writerow({"Kernel_Name": name, "Counter_Value": v})

    mb = 256
    write(tmp_path / "cf", [("cpy_kernel(tview)", mb * 1024 / 2)])        # FETCH_SIZE reads half the bytes
    write(tmp_path / "cw", [("cpy_kernel(tview)", mb * 1024)])
    write(tmp_path / "f", [("void gemv_kernel<2, 16>", 100.0), ("void gemv_kernel<2, 32>", 300.0), ("other", 1e6)])
    write(tmp_path / "w", [("void gemv_kernel<2, 16>", 2.0), ("void gemv_kernel<2, 32>", 4.0)])
    out = bench.summarize_pmc(str(tmp_path / "f"), str(tmp_path / "w"), str(tmp_path / "cf"), str(tmp_path / "cw"), mb,
                              "void gemv_kernel<2,")
    assert out["dispatches"] == 2
    assert out["fetch_scale"] == 2.0 and out["write_scale"] == 1.0
    assert out["traffic_bytes_per_launch"] == round(200.0 * 1024 * 2 + 3.0 * 1024)


def test_bench_activity_summary(tmp_path):
    """Wave activity per kernel: counters summed over a kernel's dispatches, divided by its waves
    (instructions per wave) or by its waves' cycles (issue and wait shares)."""
    import csv
    import importlib.util
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    os.makedirs(tmp_path / "run")
    rows = []
    for disp, (waves, valu, lds, act_valu, act_any, wait) in ((1, (100, 6000, 500, 200, 300, 700)),
                                                              (2, (100, 4000, 300, 100, 200, 800))):
        for name, v in (("SQ_WAVES", waves), ("SQ_INSTS_VALU", valu), ("SQ_INSTS_LDS", lds),
                        ("SQ_ACTIVE_INST_VALU", act_valu), ("SQ_ACTIVE_INST_ANY", act_any), ("SQ_WAIT_ANY", wait)):
            rows.append({"Dispatch_Id": disp, "Kernel_Name": "(anonymous namespace)::k<1>(args)", "Counter_Name": name,
                         "Counter_Value": v})
    with open(tmp_path / "run" / "p_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        w.writerows(rows)
    out = bench.summarize_activity(str(tmp_path))
    k = out["k<1>"]
    assert k["dispatches"] == 2 and k["waves_per_dispatch"] == 100
    assert k["valu_per_wave"] == 50.0 and k["lds_per_wave"] == 4.0
    assert k["valu_issue_share"] == 0.15 and k["wait_share"] == 0.75
