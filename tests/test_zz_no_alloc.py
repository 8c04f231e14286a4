"""ggml_backend_hip_graph_compute_static (the allocation-free graph compute: kernel scratch in a
static device array) against ggml_backend_graph_compute on the same graphs, through the C-ABI.

Bar: bit-identical outputs (both run the same kernels; only where their scratch lives differs).
Two calls in a row with the second graph smaller, so the second static call runs over the first
one's leftovers in the shared array; and a graph needing more scratch than the array holds is
rejected with GGML_STATUS_ALLOC_FAILED before its attention is launched, after which both entry
points still work.
"""
import numpy as np
import pytest

from gl import Graph, attention_graph, gl, quantize

pytestmark = pytest.mark.gpu

GGML_STATUS_ALLOC_FAILED = -2


@pytest.fixture(scope="module")
def hip():
    b = gl.hip_backend(0)
    yield b
    gl.libs()["core"].ggml_backend_free(b)


def rng(seed):
    return np.random.default_rng(seed)


def layer_inputs(n_kv, n_new, hd=128, n_head=24, n_head_kv=8, seed=0):
    r = rng(seed + n_kv)
    E = n_head * hd
    n_ctx = n_kv + 2
    d = {
        "kc": r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16),
        "vc": r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16),
        "q": r.standard_normal((n_new, n_head, hd)).astype(np.float32),
        "x": r.standard_normal((n_new, E)).astype(np.float32),
        "nw": (1 + 0.01 * r.standard_normal(E)).astype(np.float32),
        "wo": quantize((r.standard_normal((E, E)) * 0.02).astype(np.float32), gl.Q4_0, impl="product"),
        "wu": quantize((r.standard_normal((256, E)) * 0.02).astype(np.float32), gl.Q4_0, impl="product"),
    }
    mask = np.zeros((n_new, n_kv), dtype=np.float32)
    for i in range(n_new):
        mask[i, n_kv - n_new + i + 1:] = -np.inf
    d["mask"] = mask
    d["shape"] = (hd, n_head, n_head_kv, n_kv, n_new, n_ctx)
    return d


def build_layer(g, d):
    """Attention over the F16 cache, its output through a Q4_0 projection plus residual (the
    quantized activation the attention writes), and rms_norm * w into a second Q4_0 GEMV."""
    hd, n_head, n_head_kv, n_kv, n_new, n_ctx = d["shape"]
    E = n_head * hd
    attn = attention_graph(g, hd, n_head, n_head_kv, n_kv, n_new, n_ctx, d["kc"], d["vc"], d["q"], d["mask"])
    x = g.tensor(gl.F32, E, n_new, data=d["x"])
    o = g.add(g.mul_mat(g.tensor(gl.Q4_0, E, E, data=d["wo"]), attn), x)
    nrm = g.mul(g.rms_norm(o, 1e-5), g.tensor(gl.F32, E, data=d["nw"]))
    u = g.mul_mat(g.tensor(gl.Q4_0, E, 256, data=d["wu"]), nrm)
    return [o, u]


def compute(backend, d, static):
    """(status, outputs) of one graph compute through either entry point."""
    core, hip = gl.libs()["core"], gl.libs()["hip"]
    with Graph() as g:
        outs = build_layer(g, d)
        gf = core.ggml_new_graph(g.ctx)
        for t in outs:
            core.ggml_set_output(t)
            core.ggml_build_forward_expand(gf, t)
        g.buf = core.ggml_backend_alloc_ctx_tensors(g.ctx, backend)
        for t, a in g.inputs:
            core.ggml_backend_tensor_set(t, a.ctypes.data, 0, a.nbytes)
        if static:
            st = hip.ggml_backend_hip_graph_compute_static(backend, gf)
        else:
            st = core.ggml_backend_graph_compute(backend, gf)
        return st, ([g.read(t) for t in outs] if st == 0 else None)


@pytest.mark.parametrize("n_new", [1, 3])
def test_static_compute_matches_graph_compute(hip, n_new):
    # two calls in a row, the second with the smaller graph
    for n_kv in (700, 150):
        d = layer_inputs(n_kv, n_new)
        st_a, ref = compute(hip, d, static=False)
        st_b, got = compute(hip, d, static=True)
        assert st_a == 0 and st_b == 0
        for a, b in zip(ref, got):
            assert np.array_equal(a, b), (n_kv, n_new)


def test_static_compute_rejects_oversized_scratch(hip):
    # 64 queries x 32 heads x 8192 positions of f32 scores alone exceed the static array
    big = layer_inputs(8192, 64, hd=128, n_head=32, n_head_kv=8, seed=3)
    st, _ = compute(hip, big, static=True)
    assert st == GGML_STATUS_ALLOC_FAILED
    # both entry points still work afterwards, and agree
    d = layer_inputs(300, 1, seed=4)
    st_a, ref = compute(hip, d, static=False)
    st_b, got = compute(hip, d, static=True)
    assert st_a == 0 and st_b == 0
    for a, b in zip(ref, got):
        assert np.array_equal(a, b)
