"""ggml_backend_hip_graph_compute_static (the allocation-free graph compute: kernel scratch in a
static device array) against ggml_backend_graph_compute on the same graphs, through the C-ABI.

Bar: bit-identical outputs (both run the same kernels; only where their scratch lives differs).
Two calls in a row with the second graph smaller, so the second static call runs over the first
one's leftovers in the shared array; and a graph needing more scratch than the array holds is
rejected with GGML_STATUS_ALLOC_FAILED (kernels queued before the arena ran out have run), after
which both entry points still work. The device's free memory (hipMemGetInfo) is the same just
before and just after each static call, so the call allocated nothing.
"""
import ctypes as C

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


_hip_rt = None


def free_device_bytes():
    """hipMemGetInfo's free bytes of the current device (the HIP runtime the backend loaded)."""
    global _hip_rt
    if _hip_rt is None:
        _hip_rt = C.CDLL("libamdhip64.so")
        _hip_rt.hipMemGetInfo.restype = C.c_int
        _hip_rt.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    free, total = C.c_size_t(0), C.c_size_t(0)
    assert _hip_rt.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def compute(backend, d, static, probe=None):
    """(status, outputs) of one graph compute through either entry point; with probe (a list), the
    device's free bytes just before and just after the compute call are appended to it."""
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
        if probe is not None:
            probe.append(free_device_bytes())
        if static:
            st = hip.ggml_backend_hip_graph_compute_static(backend, gf)
        else:
            st = core.ggml_backend_graph_compute(backend, gf)
        if probe is not None:
            probe.append(free_device_bytes())
        return st, ([g.read(t) for t in outs] if st == 0 else None)


@pytest.mark.parametrize("n_new", [1, 3])
def test_static_compute_matches_graph_compute(hip, n_new):
    # two calls in a row, the second with the smaller graph
    for n_kv in (700, 150):
        d = layer_inputs(n_kv, n_new)
        st_a, ref = compute(hip, d, static=False)
        probe = []
        st_b, got = compute(hip, d, static=True, probe=probe)
        assert st_a == 0 and st_b == 0
        for a, b in zip(ref, got):
            assert np.array_equal(a, b), (n_kv, n_new)
        # the static call itself takes no device memory (the runtime's own first-use allocations
        # aside: checked on a repeat of the same call)
        probe = []
        st_c, again = compute(hip, d, static=True, probe=probe)
        assert st_c == 0 and all(np.array_equal(a, b) for a, b in zip(ref, again))
        assert probe[0] == probe[1], (n_kv, n_new, probe)


def test_static_compute_rejects_oversized_scratch(hip):
    # 64 queries x 32 heads x 8192 positions of f32 scores alone exceed the static array
    big = layer_inputs(8192, 64, hd=128, n_head=32, n_head_kv=8, seed=3)
    st, _ = compute(hip, big, static=True)
    assert st == GGML_STATUS_ALLOC_FAILED
    # both entry points still work afterwards, and agree
    d = layer_inputs(300, 1, seed=4)
    st_a, ref = compute(hip, d, static=False)
    probe = []
    st_b, got = compute(hip, d, static=True, probe=probe)
    assert st_a == 0 and st_b == 0
    for a, b in zip(ref, got):
        assert np.array_equal(a, b)
    assert probe[0] == probe[1], probe
