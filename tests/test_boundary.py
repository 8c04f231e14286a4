"""The drop-in boundary: the reference's own callers compile unchanged against include/.

GGML-Loader's model.cpp / model.h / cmd_*.cpp and dory.c are written against the ggml backend API
(reference model.h:380 names ggml_gallocr_t through ggml-backend.h; model.cpp:1156-1295 and
dory.c:722-724 build the other architectures' ops; model.cpp:5 includes ggml-vulkan.h;
cmd_inspect.cpp:76 reads a tensor's extents as an array). Each file is checked with
-fsyntax-only against this build's headers (the reference's own headers from its src/), so any
declaration the reference needs and include/ lacks fails here. Skipped where the reference
sources are absent (the GPU box).

The ops those other graphs add run on the CPU oracle (checked against closed forms here) and on
the HIP backend (tests/test_gpu_ops.py checks them bit-exact against the oracle).
"""
import os
import subprocess

import numpy as np
import pytest

from gl import Graph, cpu_backend, gl, run_on

REF_SRC = "/root/reference/src"
INCLUDE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
CALLERS = ["model.cpp", "cmd_bench.cpp", "cmd_run.cpp", "cmd_chat.cpp", "cmd_inspect.cpp", "dory.c"]


@pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="reference sources absent (only the build container has them)")
@pytest.mark.parametrize("name", CALLERS)
def test_reference_caller_compiles_against_include(name):
    if name.endswith(".c"):
        cmd = ["gcc", "-std=c11", "-Werror=implicit-function-declaration"]
    else:
        cmd = ["g++", "-std=c++17"]
    cmd += ["-fsyntax-only", "-I", INCLUDE, "-I", REF_SRC, os.path.join(REF_SRC, name)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]


@pytest.fixture(scope="module")
def cpu():
    b = cpu_backend(4)
    yield b
    gl.libs()["core"].ggml_backend_free(b)


def test_other_arch_ops_on_the_oracle(cpu):
    r = np.random.default_rng(7)
    a = (r.standard_normal((3, 5, 40)) * 4).astype(np.float32)
    b = r.standard_normal((3, 5, 40)).astype(np.float32)
    c = r.standard_normal((3, 2, 40)).astype(np.float32)
    row = r.standard_normal(40).astype(np.float32)

    def build(g):
        ta = g.tensor(gl.F32, 40, 5, 3, data=a)
        tb = g.tensor(gl.F32, 40, 5, 3, data=b)
        tc = g.tensor(gl.F32, 40, 2, 3, data=c)
        tr = g.tensor(gl.F32, 40, data=row)
        return [g.sub(ta, tr), g.abs(ta), g.softplus(ta), g.l2_norm(ta, 1e-6), g.concat(ta, tc, 1),
                g.swiglu_split(ta, tb)]

    sub, ab, sp, l2, cat, glu = run_on(cpu, build)
    assert np.array_equal(sub.reshape(a.shape), a - row)
    assert np.array_equal(ab.reshape(a.shape), np.abs(a))
    # softplus: log1p(exp(x)) rounded once from double, x itself above 20
    a64 = a.astype(np.float64)
    expect = np.where(a > 20, a, np.log1p(np.exp(a64)).astype(np.float32))
    assert np.array_equal(sp.reshape(a.shape), expect)
    # l2_norm: rows over ne0 scaled by 1 / max(sqrt(sum of f32 squares, in double), eps)
    sq = (a * a).astype(np.float64).sum(axis=-1, keepdims=True)
    scale = (np.float32(1.0) / np.maximum(np.sqrt(sq.astype(np.float32)), np.float32(1e-6))).astype(np.float32)
    assert np.array_equal(l2.reshape(a.shape), (a * scale).astype(np.float32))
    assert np.array_equal(cat.reshape(3, 7, 40), np.concatenate([a, c], axis=1))
    sl = (a / (np.float32(1.0) + np.exp(-a64).astype(np.float32))).astype(np.float32)
    assert np.array_equal(glu.reshape(a.shape), (sl * b).astype(np.float32))


def test_ssm_ops_build_nodes_with_the_reference_shapes():
    with Graph() as g:
        d_conv, n_t, d_inner, d_state, head_dim, n_head = 4, 3, 16, 8, 4, 4
        sx = g.tensor(gl.F32, d_conv - 1 + n_t, d_inner, 1)
        cw = g.tensor(gl.F32, d_conv, d_inner)
        conv = g.ssm_conv(sx, cw)
        assert [conv.contents.ne[i] for i in range(3)] == [d_inner, n_t, 1]
        s = g.tensor(gl.F32, d_state, head_dim, n_head, 1)
        x = g.tensor(gl.F32, head_dim, n_head, n_t, 1)
        scan = g.ssm_scan(s, x, x, x, x, x, g.tensor(gl.I32, 1), 1)
        assert scan.contents.ne[0] == head_dim * n_head * n_t + d_state * head_dim * n_head
        st = g.tensor(gl.F32, head_dim, head_dim, n_head, 1)
        gdn = g.gated_delta_net(x, x, x, x, x, st, 1)
        assert gdn.contents.ne[0] == head_dim * n_head * n_t + head_dim * head_dim * n_head
