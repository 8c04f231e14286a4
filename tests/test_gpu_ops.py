"""Op-level parity of the HIP backend against the oracle (CPU restatement of ggml-cpu), through the
ggml C-ABI: each test builds the same small ggml graph twice and runs it on both backends.

Bars: bit-exact for everything the decode path runs. The HIP kernels reproduce the oracle's
chain of float roundings (same block-sum order in the quantized dots, double accumulation where
ggml-cpu accumulates in double, correctly rounded transcendentals), so GEMV, RMSNorm, RoPE,
softmax, SwiGLU and the attention chain are compared with array_equal. The fused flash-attention
node, whose CPU semantics use an online softmax, is held to max relative error 2e-3 (normwise,
rel_err in gl.py), the ggml test-backend-ops bar for that op.
"""
import numpy as np
import pytest

from gl import Graph, attention_graph, cpu_backend, gl, moe_ffn_graph, quantize, rel_err, rel_err_floor, run_on

pytestmark = pytest.mark.gpu

TOL = 2e-3


@pytest.fixture(scope="module")
def hip():
    b = gl.hip_backend(0)
    yield b
    gl.libs()["core"].ggml_backend_free(b)


@pytest.fixture(scope="module")
def cpu():
    b = cpu_backend(16)
    yield b
    gl.libs()["core"].ggml_backend_free(b)


def rng(seed):
    return np.random.default_rng(seed)


def both(hip, cpu, build, fusion=True):
    gl.libs()["hip"].ggml_backend_hip_set_fusion(hip, fusion)
    try:
        return run_on(hip, build), run_on(cpu, build)
    finally:
        gl.libs()["hip"].ggml_backend_hip_set_fusion(hip, True)


def qweight(qtype, K, N, seed, std=0.02):
    w = (rng(seed).standard_normal((N, K)) * std).astype(np.float32)
    return quantize(w, qtype, impl="product")


# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("qtype", [gl.Q4_0, gl.Q8_0, gl.Q4_K, gl.Q5_K, gl.Q6_K])
def test_weight_repack_roundtrip(hip, qtype):
    K, N = 512, 96
    q = qweight(qtype, K, N, 1)
    with Graph() as g:
        w = g.tensor(qtype, K, N, data=q)
        g.compute(hip, [])
        back = g.read(w, np.uint8)
    assert np.array_equal(back, q)


def bf16_bits(x):
    """float32 -> bfloat16 bit patterns, rounded to nearest even (ggml's fp32_to_bf16 on finite values)"""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("qtype", [gl.Q4_0, gl.Q8_0, gl.Q4_K, gl.Q5_K, gl.Q6_K, gl.F16, gl.F32, gl.BF16])
def test_get_rows(hip, cpu, qtype):
    K, N = 512, 40
    if qtype in (gl.F16, gl.F32):
        w = (rng(2).standard_normal((N, K)) * 0.1).astype(np.float16 if qtype == gl.F16 else np.float32)
    elif qtype == gl.BF16:
        w = bf16_bits(rng(2).standard_normal((N, K)) * 0.1)
    else:
        w = qweight(qtype, K, N, 2, std=0.1)
    ids = np.array([3, 0, 39, 3, 17], dtype=np.int32)

    def build(g):
        wt = g.tensor(qtype, K, N, data=w)
        it = g.tensor(gl.I32, len(ids), data=ids)
        return g.get_rows(wt, it)

    a, b = both(hip, cpu, build)
    assert np.array_equal(a, b)  # dequantization is exact on both sides


@pytest.mark.parametrize("qtype,K,N", [
    (gl.Q4_0, 4096, 4096),
    (gl.Q4_0, 3072, 1024),
    (gl.Q4_0, 8192, 3072),
    (gl.Q4_0, 96, 7),
    (gl.Q8_0, 3072, 640),
    (gl.Q8_0, 8192, 300),
    (gl.Q4_K, 2560, 1024),
    (gl.Q4_K, 9728, 512),
    (gl.Q4_K, 768, 200),
    (gl.Q4_K, 4096, 2048),
    (gl.Q5_K, 2560, 1024),
    (gl.Q5_K, 9728, 512),
    (gl.Q5_K, 768, 200),
    (gl.Q6_K, 2560, 1024),
    (gl.Q6_K, 9728, 512),
    (gl.Q6_K, 4096, 300),
    (gl.Q6_K, 256, 70),
])
@pytest.mark.parametrize("ncols", [1, 3, 8, 13, 17, 40])
def test_gemv(hip, cpu, qtype, K, N, ncols):
    w = qweight(qtype, K, N, K + N)
    x = rng(7).standard_normal((ncols, K)).astype(np.float32)

    def build(g):
        wt = g.tensor(qtype, K, N, data=w)
        xt = g.tensor(gl.F32, K, ncols, data=x)
        return g.mul_mat(wt, xt)

    a, b = both(hip, cpu, build)
    assert np.array_equal(a, b), rel_err(a, b)


@pytest.mark.parametrize("qtype", [gl.Q5_K, gl.Q6_K])
@pytest.mark.parametrize("ncols", [1, 2])
def test_gemv_kquant_lm_head_width(hip, cpu, qtype, ncols):
    """A Q6_K (or Q5_K) output matrix wider than 32768 rows, as a Q4_K_M checkpoint's LM head: its
    activation is quantized once (act_quant) rather than in every workgroup; a view of the upper
    rows checks the planes' block offsets."""
    K, N = 2560, 40000
    w = qweight(qtype, K, N, 31)
    x = rng(32).standard_normal((ncols, K)).astype(np.float32)
    rb = {gl.Q5_K: 176, gl.Q6_K: 210}[qtype] * K // 256

    def build(g):
        wt = g.tensor(qtype, K, N, data=w)
        xt = g.tensor(gl.F32, K, ncols, data=x)
        top = g.view_2d(wt, K, 1000, rb, rb * (N - 1000))
        return [g.mul_mat(wt, xt), g.mul_mat(top, xt)]

    hs, cs = both(hip, cpu, build)
    for a, b in zip(hs, cs):
        assert np.array_equal(a, b), rel_err(a, b)


@pytest.mark.parametrize("wtype", [gl.F32, gl.F16, gl.BF16])
@pytest.mark.parametrize("K,N,ncols,n2", [
    (2048, 128, 1, 1),     # the MoE router
    (2048, 128, 16, 1),
    (4104, 33, 3, 1),      # more than one batch of chunks, a partial one
    (64, 17, 5, 4),        # batched over dim 2
    (12, 9, 2, 1),         # rows too short for the vector path
])
def test_mul_mat_float_weights(hip, cpu, wtype, K, N, ncols, n2):
    """F32 / F16 / BF16 weights (no quantization): float products summed in double, as ggml-cpu's
    vec_dot_f32 / vec_dot_f16 / vec_dot_bf16 (with the activation rounded to the weight's type)."""
    r = rng(K + N + ncols)
    w = r.standard_normal((n2, N, K)).astype(np.float16 if wtype == gl.F16 else np.float32)
    if wtype == gl.BF16:
        w = bf16_bits(w)
    x = r.standard_normal((n2, ncols, K)).astype(np.float32)

    def build(g):
        return g.mul_mat(g.tensor(wtype, K, N, n2, data=w), g.tensor(gl.F32, K, ncols, n2, data=x))

    a, b = both(hip, cpu, build)
    assert np.array_equal(a, b), rel_err(a, b)


def profiled(hip, fn):
    """Runs fn with every kernel timed; returns (fn's result, kernel names launched)."""
    h = gl.libs()["hip"]
    h.ggml_backend_hip_set_profile_filter(hip, b"")
    h.ggml_backend_hip_reset_profile(hip)
    h.ggml_backend_hip_set_profiling(hip, True)
    try:
        out = fn()
    finally:
        h.ggml_backend_hip_set_profiling(hip, False)
    return out, set(gl.profile(hip))


@pytest.mark.parametrize("qtype,K,N", [
    (gl.Q8_0, 3072, 1152),   # phi3 QKV shape, a slice of its rows
    (gl.Q8_0, 8192, 768),    # the down projection's row length
    (gl.Q4_0, 3072, 1024),
    (gl.Q4_0, 256, 100),     # rows end inside a 16-row tile
    (gl.Q8_0, 128, 4),       # one row group, one 4-block step
    (gl.Q8_0, 384, 36),
    (gl.Q4_K, 2560, 1024),   # Qwen3-shape rows (32 x 64 tiles: at most 128 of 64 x 64)
    (gl.Q4_K, 4096, 72),     # 32 x 64 tiles, rows end inside a 16-row tile
    (gl.Q4_K, 256, 100),     # one super-block per row
    (gl.Q5_K, 2560, 1024),
    (gl.Q5_K, 256, 100),
    (gl.Q6_K, 2560, 1024),
    (gl.Q6_K, 4096, 72),
    (gl.Q6_K, 256, 100),
])
@pytest.mark.parametrize("ncols", [64, 100, 512])
def test_gemm_prefill(hip, cpu, qtype, K, N, ncols):
    """Prefill-width mul_mat on the int8-MFMA GEMM: the same floats as the oracle's block-ordered
    sums, including partial row and column tiles."""
    w = qweight(qtype, K, N, K + 3 * N)
    x = rng(K + ncols).standard_normal((ncols, K)).astype(np.float32)

    def build(g):
        wt = g.tensor(qtype, K, N, data=w)
        xt = g.tensor(gl.F32, K, ncols, data=x)
        return g.mul_mat(wt, xt)

    a, names = profiled(hip, lambda: run_on(hip, build))
    b = run_on(cpu, build)
    assert any(n.startswith("gemm_") for n in names), names
    assert np.array_equal(a, b), rel_err(a, b)


@pytest.mark.parametrize("qtype", [gl.Q8_0, gl.Q4_0])
def test_gemm_subnormal_scales(hip, cpu, qtype):
    """Blocks whose F16 scales are subnormal (d below 2^-14) in the weights, the activations and
    both, among normal blocks: the block terms formed exactly, whichever unit forms the scale
    products."""
    K, N, ncols = 512, 256, 64
    w = rng(91).standard_normal((N, K)).astype(np.float32) * 0.02
    w[:, :256] *= 1e-2 if qtype == gl.Q8_0 else 1e-3      # Q4_0's d is amax / 8
    x = rng(92).standard_normal((ncols, K)).astype(np.float32)
    x[:, 128:384] *= 2e-4
    wq = quantize(w, qtype, impl="product")
    d16 = np.frombuffer(wq, np.uint8).reshape(N, -1)[:, :2].copy().view(np.float16)   # first block's d
    assert (np.abs(d16.astype(np.float32)) < 2.0 ** -14).all()

    def build(g):
        return g.mul_mat(g.tensor(qtype, K, N, data=wq), g.tensor(gl.F32, K, ncols, data=x))

    a, names = profiled(hip, lambda: run_on(hip, build))
    b = run_on(cpu, build)
    assert any(n.startswith("gemm_") for n in names), names
    assert np.array_equal(a, b), rel_err(a, b)


@pytest.mark.parametrize("qtype,K,N,ncols,tile", [
    (gl.Q4_0, 128, 16384, 512, "4x4x2"),     # 128 x 128 tiles: 512 of them
    (gl.Q4_0, 128, 16424, 529, "4x4x2"),     # partial row and column tiles of the largest shape
    (gl.Q4_0, 128, 8192, 512, "2x4x2"),      # 64 x 128 tiles: 512
    (gl.Q8_0, 128, 16384, 512, "2x4x2"),     # Q8_0 wants 1024 tiles: 64 x 128 ones
    (gl.Q8_0, 128, 16400, 520, "2x4x2"),
    (gl.Q8_0, 128, 32768, 512, "4x4x2"),     # 1024 tiles of 128 x 128
    (gl.Q8_0, 256, 4096, 512, "1x2x4"),      # below both thresholds
    (gl.Q4_K, 256, 4096, 512, "2x2"),        # 64 x 64 tiles: 512 (>= 256)
    (gl.Q4_K, 512, 4120, 515, "2x2"),        # partial tiles, two super-blocks per row
    (gl.Q4_K, 256, 1024, 512, "1x2"),        # 128 tiles of 64 x 64: 32 x 64 instead
    (gl.Q5_K, 256, 4096, 512, "2x2"),
    (gl.Q5_K, 512, 1000, 70, "1x2"),
    (gl.Q6_K, 512, 4120, 515, "2x2"),
    (gl.Q6_K, 256, 1024, 512, "1x2"),
])
def test_gemm_tile_variants(hip, cpu, qtype, K, N, ncols, tile):
    """Each workgroup tile of the prefill GEMM (the launch picks it from the tile count), pinned by
    the profile name and bit-exact against the oracle; small K keeps the oracle cheap."""
    w = qweight(qtype, K, N, K + 7 * N + ncols)
    x = rng(K + ncols + 5).standard_normal((ncols, K)).astype(np.float32)

    def build(g):
        return g.mul_mat(g.tensor(qtype, K, N, data=w), g.tensor(gl.F32, K, ncols, data=x))

    a, names = profiled(hip, lambda: run_on(hip, build))
    b = run_on(cpu, build)
    gemm = [n for n in names if n.startswith("gemm_")]
    assert gemm and all(n.endswith("_" + tile) for n in gemm), (gemm, tile)
    assert np.array_equal(a, b), rel_err(a, b)


@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_gemm_q4k_extreme_blocks(hip, cpu, sign):
    """The Q4_K GEMM's exactness bounds at their extremes: every 6-bit scale and min 63, every nibble
    15 (all quant bytes 0xFF, so sc * q4 = 945 in f16) against activations that quantize to -127 or
    +127 everywhere (|aux32| = 32 * 945 * 127 and |bsum| = 2032, the largest the MFMA sums see), on
    odd rows; even rows are ordinary quantized weights."""
    K, N, ncols = 1024, 96, 64
    w = qweight(gl.Q4_K, K, N, 77).reshape(N, -1).copy()
    nb = K // 256
    r = rng(78)
    for row in range(1, N, 2):
        blocks = w[row].reshape(nb, 144)
        blocks[:] = 0xFF
        for b in range(nb):
            blocks[b, 0:2] = np.frombuffer(np.float16(0.001 * (1 + r.random())).tobytes(), dtype=np.uint8)
            blocks[b, 2:4] = np.frombuffer(np.float16(0.0005 * (1 + r.random())).tobytes(), dtype=np.uint8)
    # a column of equal values quantizes to -127 everywhere; with the first value of each
    # super-block negated (it sets the scale: the first of the largest magnitudes) the rest is +127
    x = np.full((ncols, K), 3.0, dtype=np.float32)
    if sign < 0:
        x[:, ::256] = -3.0
    x[::3] *= 0.5
    x[1::3] = rng(79).standard_normal((len(x[1::3]), K)).astype(np.float32)   # ordinary columns

    def build(g):
        return g.mul_mat(g.tensor(gl.Q4_K, K, N, data=w.reshape(-1)), g.tensor(gl.F32, K, ncols, data=x))

    a, names = profiled(hip, lambda: run_on(hip, build))
    b = run_on(cpu, build)
    assert any(n.startswith("gemm_q4_K") for n in names), names
    assert np.array_equal(a, b), rel_err(a, b)


@pytest.mark.parametrize("qtype", [gl.Q5_K, gl.Q6_K])
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_gemm_kquant_extreme_blocks(hip, cpu, qtype, sign):
    """The Q5_K / Q6_K GEMM's exactness bounds at their extremes, on odd rows against activations
    that quantize to -127 or +127 everywhere. Q5_K: every scale and min 63 and every quant 31
    (sc * q5 = 1953). Q6_K: in the first super-block of a row every scale -128 and every quant 0
    (sc * (q - 32) = 4096, |aux32| = 32 * 4096 * 127); in the others random scales and quants, so
    that most products are odd integers above 2048, which f16 cannot hold (the kernel's hi / lo
    split). Even rows are ordinary quantized weights."""
    K, N, ncols = 1024, 96, 64
    bs = {gl.Q5_K: 176, gl.Q6_K: 210}[qtype]
    w = qweight(qtype, K, N, 87).reshape(N, -1).copy()
    nb = K // 256
    r = rng(88)
    for row in range(1, N, 2):
        blocks = w[row].reshape(nb, bs)
        for b in range(nb):
            if qtype == gl.Q5_K:
                blocks[b, :] = 0xFF
                blocks[b, 0:2] = np.frombuffer(np.float16(0.001 * (1 + r.random())).tobytes(), dtype=np.uint8)
                blocks[b, 2:4] = np.frombuffer(np.float16(0.0005 * (1 + r.random())).tobytes(), dtype=np.uint8)
            else:
                # ql[128] qh[64] scales[16] d
                if b == 0:
                    blocks[b, :208] = 0
                    blocks[b, 192:208] = 0x80
                else:
                    blocks[b, :208] = r.integers(0, 256, 208, dtype=np.uint8)
                blocks[b, 208:210] = np.frombuffer(np.float16(0.0001 * (1 + r.random())).tobytes(), dtype=np.uint8)
    x = np.full((ncols, K), 3.0, dtype=np.float32)
    if sign < 0:
        x[:, ::256] = -3.0
    x[::3] *= 0.5
    x[1::3] = rng(89).standard_normal((len(x[1::3]), K)).astype(np.float32)

    def build(g):
        return g.mul_mat(g.tensor(qtype, K, N, data=w.reshape(-1)), g.tensor(gl.F32, K, ncols, data=x))

    a, names = profiled(hip, lambda: run_on(hip, build))
    b = run_on(cpu, build)
    assert any(n.startswith("gemm_" + {gl.Q5_K: "q5_K", gl.Q6_K: "q6_K"}[qtype]) for n in names), names
    assert np.array_equal(a, b), rel_err(a, b)


def test_gemm_q6k_lm_head_width(hip, cpu):
    """A Q6_K LM head (at least 65536 rows) takes the GEMM from 16 columns; a view of its upper
    rows checks the planes' block offsets on that path."""
    K, N, ncols = 256, 66600, 16
    w = qweight(gl.Q6_K, K, N, 41)
    x = rng(42).standard_normal((ncols, K)).astype(np.float32)
    rb = 210 * K // 256

    def build(g):
        wt = g.tensor(gl.Q6_K, K, N, data=w)
        xt = g.tensor(gl.F32, K, ncols, data=x)
        top = g.view_2d(wt, K, N - 1000, rb, rb * 1000)
        return [g.mul_mat(wt, xt), g.mul_mat(top, xt)]

    (hs, names) = profiled(hip, lambda: run_on(hip, build))
    cs = run_on(cpu, build)
    assert any(n.startswith("gemm_q6_K") for n in names) and not any(n.startswith("gemv") for n in names), names
    for a, b in zip(hs, cs):
        assert np.array_equal(a, b), rel_err(a, b)


@pytest.mark.parametrize("qtype", [gl.Q4_0, gl.Q8_0, gl.Q4_K, gl.Q5_K, gl.Q6_K])
def test_gemm_norm_qkv_residual(hip, cpu, qtype):
    """rms_norm * w feeding three prefill-width GEMMs (normalized and quantized once), and a GEMM
    whose residual add is fused into its store."""
    K, ncols = 512, 96
    x = rng(30).standard_normal((ncols, K)).astype(np.float32) * 2
    nw = (1 + 0.01 * rng(31).standard_normal(K)).astype(np.float32)
    r = rng(32).standard_normal((ncols, K)).astype(np.float32)
    Wq, Wk, Wv, Wo = (qweight(qtype, K, n, s) for n, s in ((512, 33), (128, 34), (128, 35), (512, 36)))

    def build(g):
        xt = g.tensor(gl.F32, K, ncols, data=x)
        y = g.mul(g.rms_norm(xt, 1e-5), g.tensor(gl.F32, K, data=nw))
        q = g.mul_mat(g.tensor(qtype, K, 512, data=Wq), y)
        k = g.mul_mat(g.tensor(qtype, K, 128, data=Wk), y)
        v = g.mul_mat(g.tensor(qtype, K, 128, data=Wv), y)
        o = g.add(g.mul_mat(g.tensor(qtype, K, K, data=Wo), q), g.tensor(gl.F32, K, ncols, data=r))
        return [q, k, v, o]

    for fusion in (True, False):
        hs, cs = both(hip, cpu, build, fusion)
        for a, b in zip(hs, cs):
            assert np.array_equal(a, b), (fusion, rel_err(a, b))


@pytest.mark.parametrize("qtype", [gl.Q4_0, gl.Q4_K, gl.Q5_K, gl.Q6_K])
@pytest.mark.parametrize("ncols", [1, 16, 19])
def test_gemv_residual_and_qkv_group(hip, cpu, qtype, ncols):
    """Q, K and V in one launch (matrices starting on workgroup boundaries) and the O projection
    with its residual add; several columns take the multi-column kernels (Q4_K: the matrix cores)."""
    K = 1024
    Nq, Nk = 1024, 200
    wq, wk, wv, wo = (qweight(qtype, K, n, s) for n, s in ((Nq, 11), (Nk, 12), (Nk, 13), (K, 14)))
    x = rng(3).standard_normal((ncols, K)).astype(np.float32)
    r = rng(4).standard_normal((ncols, K)).astype(np.float32)

    def build(g):
        xt = g.tensor(gl.F32, K, ncols, data=x)
        rt = g.tensor(gl.F32, K, ncols, data=r)
        q = g.mul_mat(g.tensor(qtype, K, Nq, data=wq), xt)
        k = g.mul_mat(g.tensor(qtype, K, Nk, data=wk), xt)
        v = g.mul_mat(g.tensor(qtype, K, Nk, data=wv), xt)
        o = g.add(g.mul_mat(g.tensor(qtype, K, K, data=wo), q), rt)
        return [q, k, v, o]

    for fusion in (True, False):
        hs, cs = both(hip, cpu, build, fusion)
        for a, b in zip(hs, cs):
            assert np.array_equal(a, b), (fusion, rel_err(a, b))


@pytest.mark.parametrize("qtype", [gl.Q4_0, gl.Q8_0, gl.Q4_K, gl.Q5_K, gl.Q6_K])
@pytest.mark.parametrize("ncols", [1, 2, 16, 21])
def test_swiglu_ffn(hip, cpu, qtype, ncols):
    E, F = 512, 1536
    wg, wu, wd = qweight(qtype, E, F, 21), qweight(qtype, E, F, 22), qweight(qtype, F, E, 23)
    x = rng(5).standard_normal((ncols, E)).astype(np.float32)
    r = rng(6).standard_normal((ncols, E)).astype(np.float32)

    def build(g):
        xt = g.tensor(gl.F32, E, ncols, data=x)
        gate = g.mul_mat(g.tensor(qtype, E, F, data=wg), xt)
        up = g.mul_mat(g.tensor(qtype, E, F, data=wu), xt)
        act = g.mul(g.silu(gate), up)
        down = g.mul_mat(g.tensor(qtype, F, E, data=wd), act)
        return g.add(down, g.tensor(gl.F32, E, ncols, data=r))

    for fusion in (True, False):
        a, b = both(hip, cpu, build, fusion)
        assert np.array_equal(a, b), (fusion, rel_err(a, b))


@pytest.mark.parametrize("n,rows", [(3072, 1), (2560, 3), (128, 40), (96, 7)])
def test_rms_norm_mul_then_gemv(hip, cpu, n, rows):
    x = rng(8).standard_normal((rows, n)).astype(np.float32) * 3
    w = (1 + 0.01 * rng(9).standard_normal(n)).astype(np.float32)
    qtype = gl.Q4_K if n % 256 == 0 else gl.Q4_0
    W = qweight(qtype, n, 64, 10)

    def build(g):
        xt = g.tensor(gl.F32, n, rows, data=x)
        y = g.mul(g.rms_norm(xt, 1e-5), g.tensor(gl.F32, n, data=w))
        return [y, g.mul_mat(g.tensor(qtype, n, 64, data=W), y)]

    for fusion in (True, False):
        (y1, z1), (y2, z2) = both(hip, cpu, build, fusion)
        assert np.array_equal(y1, y2), (fusion, rel_err(y1, y2))
        assert np.array_equal(z1, z2), (fusion, rel_err(z1, z2))


@pytest.mark.parametrize("qtype,n", [(gl.Q4_0, 3072), (gl.Q8_0, 4096), (gl.Q4_K, 2560), (gl.Q4_K, 4096),
                                     (gl.Q4_0, 96), (gl.Q4_0, 9216), (gl.Q5_K, 2560), (gl.Q6_K, 3072)])
@pytest.mark.parametrize("ncols", [1, 3])
def test_rms_norm_folded_into_gemv(hip, cpu, qtype, n, ncols):
    """rms_norm * w read only by GEMVs (Q, K and V; a gate/up pair with SwiGLU): the GEMVs compute
    and quantize the normalization in their prologue and it is never materialized (K = 9216 is
    beyond the prologue and takes the materialized path)."""
    x = rng(20).standard_normal((ncols, n)).astype(np.float32) * 2
    w1 = (1 + 0.01 * rng(21).standard_normal(n)).astype(np.float32)
    w2 = (1 + 0.01 * rng(27).standard_normal(n)).astype(np.float32)
    Wq, Wk, Wv = (qweight(qtype, n, r, s) for r, s in ((256, 22), (64, 23), (64, 24)))
    Wg, Wu = qweight(qtype, n, 512, 25), qweight(qtype, n, 512, 26)

    def build(g):
        xt = g.tensor(gl.F32, n, ncols, data=x)
        y = g.mul(g.rms_norm(xt, 1e-5), g.tensor(gl.F32, n, data=w1))
        q = g.mul_mat(g.tensor(qtype, n, 256, data=Wq), y)
        k = g.mul_mat(g.tensor(qtype, n, 64, data=Wk), y)
        v = g.mul_mat(g.tensor(qtype, n, 64, data=Wv), y)
        y2 = g.mul(g.rms_norm(xt, 1e-6), g.tensor(gl.F32, n, data=w2))
        act = g.mul(g.silu(g.mul_mat(g.tensor(qtype, n, 512, data=Wg), y2)), g.mul_mat(g.tensor(qtype, n, 512, data=Wu), y2))
        return [q, k, v, act]

    for fusion in (True, False):
        hs, cs = both(hip, cpu, build, fusion)
        for a, b in zip(hs, cs):
            assert np.array_equal(a, b), (fusion, rel_err(a, b))


@pytest.mark.parametrize("mode", [gl.ROPE_NORMAL, gl.ROPE_NEOX])
@pytest.mark.parametrize("hd,n_head,theta", [(128, 8, 500000.0), (128, 4, 1e6), (96, 4, 10000.0)])
def test_rope(hip, cpu, mode, hd, n_head, theta):
    pos = np.array([0, 1, 7, 2048, 8191], dtype=np.int32)
    x = rng(11).standard_normal((len(pos), n_head, hd)).astype(np.float32)

    def build(g):
        xt = g.tensor(gl.F32, hd, n_head, len(pos), data=x)
        pt = g.tensor(gl.I32, len(pos), data=pos)
        return g.rope_ext(xt, pt, None, hd, mode, 4096, theta, 1.0, 0.0, 1.0, 0.0, 0.0)

    a, b = both(hip, cpu, build)
    assert np.array_equal(a, b), rel_err(a, b)


@pytest.mark.parametrize("mode,hd,n_new", [(gl.ROPE_NORMAL, 128, 1), (gl.ROPE_NEOX, 128, 3), (gl.ROPE_NEOX, 96, 1)])
def test_rope_and_kv_append_batched(hip, cpu, mode, hd, n_new):
    """The decode step's RoPE(Q), RoPE(K) -> F16 cache and V -> F16 cache (reference
    model.cpp:1389-1414): one launch on the fused path, the K rotation stored straight into the cache."""
    n_head, n_head_kv, n_ctx, n_past = 24, 8, 40, 17
    r = rng(40 + hd)
    q = r.standard_normal((n_new, n_head, hd)).astype(np.float32)
    k = r.standard_normal((n_new, n_head_kv, hd)).astype(np.float32) * 3
    v = r.standard_normal((n_new, n_head_kv, hd)).astype(np.float32) * 3
    pos = np.arange(n_past, n_past + n_new, dtype=np.int32) + 2000
    cache0 = r.standard_normal((2, n_ctx, n_head_kv, hd)).astype(np.float16)

    def run(backend, fusion):
        with Graph() as g:
            kc = g.tensor(gl.F16, hd, n_head_kv, n_ctx, data=cache0[0])
            vc = g.tensor(gl.F16, hd, n_head_kv, n_ctx, data=cache0[1])
            pt = g.tensor(gl.I32, n_new, data=pos)
            qr = g.rope_ext(g.tensor(gl.F32, hd, n_head, n_new, data=q), pt, None, hd, mode, 4096, 500000.0, 1.0, 0.0, 1.0, 0.0, 0.0)
            kr = g.rope_ext(g.tensor(gl.F32, hd, n_head_kv, n_new, data=k), pt, None, hd, mode, 4096, 500000.0, 1.0, 0.0, 1.0, 0.0, 0.0)
            nb1, nb2 = hd * 2, hd * n_head_kv * 2
            ck = g.cpy(kr, g.view_3d(kc, hd, n_head_kv, n_new, nb1, nb2, n_past * nb2))
            cv = g.cpy(g.tensor(gl.F32, hd, n_head_kv, n_new, data=v), g.view_3d(vc, hd, n_head_kv, n_new, nb1, nb2, n_past * nb2))
            gl.libs()["hip"].ggml_backend_hip_set_fusion(hip, fusion)
            try:
                qo = g.compute(backend, [qr, ck, cv])[0]
            finally:
                gl.libs()["hip"].ggml_backend_hip_set_fusion(hip, True)
            return qo, g.read(kc, np.float16), g.read(vc, np.float16)

    ref = run(cpu, True)
    for fusion in (True, False):
        got = run(hip, fusion)
        assert np.array_equal(got[0], ref[0]), fusion
        assert np.array_equal(got[1].view(np.uint16), ref[1].view(np.uint16)), fusion
        assert np.array_equal(got[2].view(np.uint16), ref[2].view(np.uint16)), fusion
    # untouched cache rows keep their contents; the new V rows are the f16 rounding of v
    kcache = ref[1].reshape(n_ctx, n_head_kv, hd)
    assert np.array_equal(kcache[:n_past].view(np.uint16), cache0[0][:n_past].view(np.uint16))
    assert np.array_equal(ref[2].reshape(n_ctx, n_head_kv, hd)[n_past:n_past + n_new], v.astype(np.float16))


@pytest.mark.parametrize("mode,hd,n_dims,n_new", [
    (gl.ROPE_NEOX, 128, 128, 16),    # the MoE 16-token step (Q: 32 heads x 16 tokens = 512 rows)
    (gl.ROPE_NORMAL, 128, 128, 5),
    (gl.ROPE_NEOX, 64, 32, 33),      # a partial rotation: dims past n_dims are copied
    (gl.ROPE_NORMAL, 96, 64, 20),    # and across the (cos, sin) table's threshold of 16 tokens
])
def test_rope_with_qk_norm_batched(hip, cpu, mode, hd, n_dims, n_new):
    """QK-Norm (rms_norm(x) * w over the head dimension, model.cpp:1382-1387) in front of RoPE for
    more tokens than the attention folds in: the norm runs inside the RoPE launch, one wave per
    (head, token) row, with the rms_norm and mul ops' roundings, K stored straight into the F16
    cache; bit-identical to the op chain, and no separate norm launch."""
    n_head, n_head_kv, n_past = 32, 4, 9
    n_ctx = n_past + n_new + 3
    r = rng(90 + hd + n_new)
    q = r.standard_normal((n_new, n_head, hd)).astype(np.float32) * 2
    k = r.standard_normal((n_new, n_head_kv, hd)).astype(np.float32) * 2
    qw = (1 + 0.1 * r.standard_normal(hd)).astype(np.float32)
    kw = (1 + 0.1 * r.standard_normal(hd)).astype(np.float32)
    pos = np.arange(n_past, n_past + n_new, dtype=np.int32) + 4000
    cache0 = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)

    def run(backend, fusion):
        with Graph() as g:
            kc = g.tensor(gl.F16, hd, n_head_kv, n_ctx, data=cache0)
            pt = g.tensor(gl.I32, n_new, data=pos)
            qs = g.mul(g.rms_norm(g.tensor(gl.F32, hd, n_head, n_new, data=q), 1e-6), g.tensor(gl.F32, hd, data=qw))
            ks = g.mul(g.rms_norm(g.tensor(gl.F32, hd, n_head_kv, n_new, data=k), 1e-6), g.tensor(gl.F32, hd, data=kw))
            qr = g.rope_ext(qs, pt, None, n_dims, mode, 4096, 1e6, 1.0, 0.0, 1.0, 0.0, 0.0)
            kr = g.rope_ext(ks, pt, None, n_dims, mode, 4096, 1e6, 1.0, 0.0, 1.0, 0.0, 0.0)
            nb1, nb2 = hd * 2, hd * n_head_kv * 2
            ck = g.cpy(kr, g.view_3d(kc, hd, n_head_kv, n_new, nb1, nb2, n_past * nb2))
            gl.libs()["hip"].ggml_backend_hip_set_fusion(hip, fusion)
            try:
                if backend is hip:
                    qo, names = profiled(hip, lambda: g.compute(backend, [qr, ck])[0])
                else:
                    qo, names = g.compute(backend, [qr, ck])[0], set()
            finally:
                gl.libs()["hip"].ggml_backend_hip_set_fusion(hip, True)
            return qo, g.read(kc, np.float16), names

    ref = run(cpu, True)
    for fusion in (True, False):
        got = run(hip, fusion)
        assert np.array_equal(got[0], ref[0]), (fusion, rel_err(got[0], ref[0]))
        assert np.array_equal(got[1].view(np.uint16), ref[1].view(np.uint16)), fusion
        if fusion:
            assert "rope" in got[2] and "rms_norm_mul" not in got[2], got[2]
    kcache = ref[1].reshape(n_ctx, n_head_kv, hd)
    assert np.array_equal(kcache[:n_past].view(np.uint16), cache0[:n_past].view(np.uint16))


@pytest.mark.parametrize("mode,hd,n_head,n_head_kv,qk_norm", [
    (gl.ROPE_NORMAL, 128, 24, 8, False), (gl.ROPE_NEOX, 96, 8, 8, False), (gl.ROPE_NEOX, 64, 8, 2, False),
    (gl.ROPE_NEOX, 128, 32, 8, True),    # Qwen3: QK-Norm before the rotations
    (gl.ROPE_NEOX, 64, 8, 2, True),
])
@pytest.mark.parametrize("n_new", [1, 3])
def test_attention_with_rope_and_kv_append(hip, cpu, mode, hd, n_head, n_head_kv, qk_norm, n_new):
    """[QK-Norm (rms_norm * w per head, model.cpp:1382-1387),] RoPE(Q), RoPE(K) -> F16 cache, V -> F16
    cache, then decode attention over the caches (the reference's per-layer order, model.cpp:1389-1444):
    on the fused path the norms, rotations and cache writes happen inside the attention's scores
    kernel, with the same floats and cache rows."""
    n_ctx, n_past = 140, 129          # the new rows straddle a 64-position chunk boundary for n_new = 3
    n_kv = n_past + n_new
    r = rng(60 + hd + n_new)
    q = r.standard_normal((n_new, n_head, hd)).astype(np.float32)
    k = r.standard_normal((n_new, n_head_kv, hd)).astype(np.float32) * 2
    v = r.standard_normal((n_new, n_head_kv, hd)).astype(np.float32) * 2
    qw = (1 + 0.1 * r.standard_normal(hd)).astype(np.float32)
    kw = (1 + 0.1 * r.standard_normal(hd)).astype(np.float32)
    pos = np.arange(n_past, n_kv, dtype=np.int32)
    cache0 = r.standard_normal((2, n_ctx, n_head_kv, hd)).astype(np.float16)
    mask = np.zeros((n_new, n_kv), dtype=np.float32)
    for i in range(n_new):
        mask[i, n_past + i + 1:] = -np.inf

    def run(backend, fusion):
        with Graph() as g:
            kc = g.tensor(gl.F16, hd, n_head_kv, n_ctx, data=cache0[0])
            vc = g.tensor(gl.F16, hd, n_head_kv, n_ctx, data=cache0[1])
            pt = g.tensor(gl.I32, n_new, data=pos)
            m = g.tensor(gl.F32, n_kv, n_new, data=mask)
            qs, ks = g.tensor(gl.F32, hd, n_head, n_new, data=q), g.tensor(gl.F32, hd, n_head_kv, n_new, data=k)
            if qk_norm:
                qs = g.mul(g.rms_norm(qs, 1e-6), g.tensor(gl.F32, hd, data=qw))
                ks = g.mul(g.rms_norm(ks, 1e-6), g.tensor(gl.F32, hd, data=kw))
            qr = g.rope_ext(qs, pt, None, hd, mode, 4096, 10000.0, 1.0, 0.0, 1.0, 0.0, 0.0)
            kr = g.rope_ext(ks, pt, None, hd, mode, 4096, 10000.0, 1.0, 0.0, 1.0, 0.0, 0.0)
            nb1, nb2 = hd * 2, hd * n_head_kv * 2
            ck = g.cpy(kr, g.view_3d(kc, hd, n_head_kv, n_new, nb1, nb2, n_past * nb2))
            cv = g.cpy(g.tensor(gl.F32, hd, n_head_kv, n_new, data=v), g.view_3d(vc, hd, n_head_kv, n_new, nb1, nb2, n_past * nb2))
            K = g.permute(g.view_3d(kc, hd, n_head_kv, n_kv, nb1, nb2, 0), 0, 2, 1, 3)
            V_full = g.view_3d(vc, hd, n_head_kv, n_kv, nb1, nb2, 0)
            KQ = g.soft_max_ext(g.mul_mat(K, g.permute(qr, 0, 2, 1, 3)), m, 1.0 / np.sqrt(hd), 0.0)
            KQV = g.mul_mat(g.cont_3d(g.permute(V_full, 1, 2, 0, 3), n_kv, hd, n_head_kv), KQ)
            out = g.cont_2d(g.permute(KQV, 0, 2, 1, 3), hd * n_head, n_new)
            gl.libs()["hip"].ggml_backend_hip_set_fusion(hip, fusion)
            try:
                if backend is hip:
                    o, names = profiled(hip, lambda: g.compute(backend, [ck, cv, out])[2])
                else:
                    o, names = g.compute(backend, [ck, cv, out])[2], set()
            finally:
                gl.libs()["hip"].ggml_backend_hip_set_fusion(hip, True)
            return o, g.read(kc, np.float16), g.read(vc, np.float16), names

    ref = run(cpu, True)
    for fusion in (True, False):
        got = run(hip, fusion)
        assert np.array_equal(got[0], ref[0]), (fusion, rel_err(got[0], ref[0]))
        assert np.array_equal(got[1].view(np.uint16), ref[1].view(np.uint16)), fusion
        assert np.array_equal(got[2].view(np.uint16), ref[2].view(np.uint16)), fusion
        if fusion:
            assert "rope" not in got[3] and "rms_norm_mul" not in got[3] and "attn_decode" in got[3], got[3]


def test_soft_max_masked(hip, cpu):
    n_kv, n_q, n_head = 300, 3, 5
    x = rng(12).standard_normal((n_head, n_q, n_kv)).astype(np.float32) * 4
    mask = np.zeros((n_q, n_kv), dtype=np.float32)
    for q in range(n_q):
        mask[q, n_kv - n_q + q + 1:] = -np.inf

    def build(g):
        xt = g.tensor(gl.F32, n_kv, n_q, n_head, data=x)
        mt = g.tensor(gl.F32, n_kv, n_q, data=mask)
        return g.soft_max_ext(xt, mt, 0.125, 0.0)

    a, b = both(hip, cpu, build)
    assert np.array_equal(a, b), rel_err(a, b)


def test_kv_append_f16_exact(hip, cpu):
    hd, nkv, n_ctx, n_past, n_new = 128, 8, 64, 17, 3
    cache = np.zeros((n_ctx, nkv, hd), dtype=np.float16)
    src = rng(13).standard_normal((n_new, nkv, hd)).astype(np.float32) * 10

    def build(g):
        c = g.tensor(gl.F16, hd, nkv, n_ctx, data=cache)
        s = g.tensor(gl.F32, hd, nkv, n_new, data=src)
        nb1, nb2 = hd * 2, hd * nkv * 2
        dst = g.view_3d(c, hd, nkv, n_new, nb1, nb2, n_past * nb2)
        cp = g.cpy(s, dst)
        return cp

    a, b = both(hip, cpu, build)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    expect = src.astype(np.float16)  # numpy rounds to nearest even
    assert np.array_equal(a.view(np.uint16).reshape(n_new, nkv, hd), expect.view(np.uint16))


def test_argmax(hip, cpu):
    x = rng(14).standard_normal((3, 5000)).astype(np.float32)
    x[1, 4000] = x[1, 123] = 50.0  # tie: the first index wins

    def build(g):
        return g.argmax(g.tensor(gl.F32, 5000, 3, data=x))

    a, b = both(hip, cpu, build)
    assert np.array_equal(a.view(np.int32), b.view(np.int32))
    assert a.view(np.int32)[1] == 123


@pytest.mark.parametrize("n,ties", [(16384, (9000, 16383)), (128256, (70000, 130)), (151936, (151935, 151934)), (200003, (1, 0))])
def test_argmax_wide_row(hip, cpu, n, ties):
    """One logits row (the greedy pick of forward_step_greedy) in two launches over 128 chunk
    maxima: the first index of the maximum, also when the tied indices sit in different chunks."""
    x = rng(15).standard_normal(n).astype(np.float32)
    for i in ties:
        x[i] = 40.0

    def build(g):
        return g.argmax(g.tensor(gl.F32, n, 1, data=x))

    a, b = both(hip, cpu, build)
    assert a.view(np.int32)[0] == b.view(np.int32)[0] == min(ties)


@pytest.mark.parametrize("hd,n_head,n_head_kv,n_kv,n_new", [
    (128, 24, 8, 2049, 1),    # Llama-3B shape at position 2048
    (128, 24, 8, 2304, 1),    # the longest row whose PV workgroups form the softmax statistics
    (128, 24, 8, 2305, 1),    # the shortest row with the statistics launch
    (128, 32, 8, 8193, 1),    # Qwen3 shape at position 8192
    (128, 32, 4, 4097, 1),    # MoE config attention
    (96, 32, 32, 130, 1),     # Phi-3 head dim
    (64, 8, 8, 1, 1),         # first token: output = V
    (128, 24, 8, 64, 1),
    (128, 24, 8, 65, 2),
    (128, 16, 8, 200, 4),
    (128, 32, 4, 2400, 16),   # a 16-token MoE step past the prefill kernel's rows: 8 tiles of 16 (query, head) rows per KV head
    (128, 16, 8, 2400, 13),   # a partial last row tile (13 queries x 2 heads)
])
@pytest.mark.parametrize("flash", [False, True])
def test_attention_decode(hip, cpu, hd, n_head, n_head_kv, n_kv, n_new, flash):
    r = rng(n_kv + hd)
    n_ctx = n_kv + 3
    kc = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)
    vc = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)
    q = r.standard_normal((n_new, n_head, hd)).astype(np.float32)
    mask = np.zeros((n_new, n_kv), dtype=np.float32)
    n_past = n_kv - n_new
    for i in range(n_new):
        mask[i, n_past + i + 1:] = -np.inf

    def build(g):
        return attention_graph(g, hd, n_head, n_head_kv, n_kv, n_new, n_ctx, kc, vc, q, mask, flash)

    for fusion in (True, False):
        if flash and not fusion:
            continue
        a, b = both(hip, cpu, build, fusion)
        if flash:
            # ggml-cpu's online softmax against one pass with float p: per element within 2e-3
            assert rel_err_floor(a, b) < TOL, (fusion, rel_err_floor(a, b))
        else:
            # the graph's chain of float roundings is reproduced exactly, fused or not
            assert np.array_equal(a, b), (fusion, rel_err(a, b))
    if n_kv == 1:
        # a single key: the output is that key's V row for every head of the group
        grp = n_head // n_head_kv
        expect = np.repeat(vc[0].astype(np.float32), grp, axis=0).reshape(-1)
        assert rel_err(a, expect) < 1e-6


@pytest.mark.parametrize("qtype,hd,n_head,n_head_kv,n_kv", [
    (gl.Q4_0, 128, 24, 8, 2049),   # Llama-3B shape: PV forms its rows' statistics, two launches
    (gl.Q8_0, 96, 32, 32, 130),    # Phi-3 head dim
    (gl.Q4_K, 128, 32, 8, 8193),   # Qwen3 shape: the statistics launch
    (gl.Q4_K, 128, 32, 4, 4097),   # MoE config attention
    (gl.Q6_K, 128, 16, 8, 300),
    (gl.Q5_K, 64, 8, 8, 1),        # first token: the output is V's row
])
def test_attention_output_accumulated_into_o_projection(hip, cpu, qtype, hd, n_head, n_head_kv, n_kv):
    """One query's attention read only by its O projection: the PV workgroups add their chunk
    partials into one double accumulator (FP64 atomics: the sums are exact, so their order does not
    change them), no combination launch runs and the output is never written; the projection's
    prologue rounds the doubles to float and quantizes them as the combination's output would have
    been. Bit-exact against the oracle, fused or not."""
    r = rng(n_kv + n_head + hd)
    n_ctx = n_kv + 3
    kc = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)
    vc = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)
    q = r.standard_normal((1, n_head, hd)).astype(np.float32)
    mask = np.zeros((1, n_kv), dtype=np.float32)
    K, rows = n_head * hd, 640
    wo = qweight(qtype, K, rows, 95, std=0.05)

    def build(g):
        att = attention_graph(g, hd, n_head, n_head_kv, n_kv, 1, n_ctx, kc, vc, q, mask)
        return g.mul_mat(g.tensor(qtype, K, rows, data=wo), att)

    for fusion in (True, False):
        a, b = both(hip, cpu, build, fusion)
        assert np.array_equal(a, b), (fusion, rel_err(a, b))
    _, names = profiled(hip, lambda: run_on(hip, build))
    assert "attn_decode_acc" in names and "attn_decode" not in names, names


@pytest.mark.parametrize("qtype,hd,n_head,n_head_kv,n_kv,n_new", [
    (gl.Q4_K, 128, 32, 4, 2400, 16),   # the MoE 16-token step: the multi-query matrix-core kernels
    (gl.Q4_K, 128, 16, 8, 300, 3),     # the four-query decode kernels
    (gl.Q6_K, 64, 8, 8, 90, 3),        # head dim 64: four heads per super-block
])
def test_attention_combination_writes_q8k(hip, cpu, qtype, hd, n_head, n_head_kv, n_kv, n_new):
    """Several queries' attention read by a K-quant O projection: the combination launch writes the
    output's Q8_K copy itself (quantize_row_q8_K's arithmetic over each 256-dim super-block), so no
    separate quantization launch runs; bit-exact against the oracle, fused or not."""
    r = rng(n_kv + n_new + hd)
    n_ctx = n_kv + 3
    kc = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)
    vc = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)
    q = r.standard_normal((n_new, n_head, hd)).astype(np.float32)
    mask = np.zeros((n_new, n_kv), dtype=np.float32)
    n_past = n_kv - n_new
    for i in range(n_new):
        mask[i, n_past + i + 1:] = -np.inf
    K, rows = n_head * hd, 640
    wo = qweight(qtype, K, rows, 97, std=0.05)

    def build(g):
        att = attention_graph(g, hd, n_head, n_head_kv, n_kv, n_new, n_ctx, kc, vc, q, mask)
        return g.mul_mat(g.tensor(qtype, K, rows, data=wo), att)

    for fusion in (True, False):
        a, b = both(hip, cpu, build, fusion)
        assert np.array_equal(a, b), (fusion, rel_err(a, b))
    _, names = profiled(hip, lambda: run_on(hip, build))
    assert "attn_decode" in names and "quantize_q8K" not in names, names


@pytest.mark.parametrize("n_new,n_kv", [
    (2, 70),       # the decode kernels
    (20, 70),      # the prefill kernel
    (20, 2400),    # the multi-query decode kernels (past the prefill kernel's rows)
])
def test_attention_masked_nonfinite_k_row(hip, cpu, n_new, n_kv):
    """The fused attention gives a position masked for a query the score -inf without reading its
    dot, on every path. ggml-cpu's manual chain forms NaN * scale + (-inf) = NaN there and spreads
    it over the row: a documented deviation. In forward_step the manual chain masks only the step's
    own later tokens, whose K rows come from the same activations, so it shows only when those are
    already non-finite. Queries that cannot see the row equal the chain over a finite row; the
    query that attends it is NaN on both."""
    hd, n_head, n_head_kv = 128, 8, 2
    G = n_head // n_head_kv
    r = rng(n_kv + n_new)
    n_ctx = n_kv + 3
    kc = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)
    vc = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)
    q = r.standard_normal((n_new, n_head, hd)).astype(np.float32)
    mask = np.zeros((n_new, n_kv), dtype=np.float32)
    for i in range(n_new):
        mask[i, n_kv - n_new + i + 1:] = -np.inf
    bad, finite = kc.copy(), kc.copy()
    bad[n_kv - 1, 0, :] = np.nan                  # the last new token's K row of KV head 0
    finite[n_kv - 1, 0, :] = 0.5

    def build(k):
        return lambda g: attention_graph(g, hd, n_head, n_head_kv, n_kv, n_new, n_ctx, k, vc, q, mask, False)

    a = run_on(hip, build(bad)).reshape(n_new, n_head, hd)
    b = run_on(cpu, build(finite)).reshape(n_new, n_head, hd)
    c = run_on(cpu, build(bad)).reshape(n_new, n_head, hd)
    assert np.array_equal(a[:-1], b[:-1])
    assert np.array_equal(a[-1, G:], b[-1, G:])
    assert np.isnan(a[-1, :G]).all() and np.isnan(c[-1, :G]).all()
    assert np.isnan(c[0, :G]).all()               # the chain itself spreads the masked NaN


@pytest.mark.parametrize("hd,n_head,n_head_kv,n_kv,n_new", [
    (96, 32, 32, 512, 512),   # Phi-3 prefill of 512 tokens, one layer
    (128, 8, 2, 100, 100),    # GQA, partial last query tile and position chunk
    (64, 4, 4, 77, 37),       # after 40 cached positions
    (128, 24, 8, 300, 20),
    (96, 6, 2, 1000, 5),      # the smallest batch past the decode kernels
])
@pytest.mark.parametrize("flash", [False, True])
def test_attention_prefill(hip, cpu, hd, n_head, n_head_kv, n_kv, n_new, flash):
    """Attention over a prefill-width query batch (causal mask): the chain's float roundings
    exactly (its fully masked position chunks are skipped), flash_attn_ext within tolerance."""
    r = rng(n_kv + hd + n_new)
    n_ctx = n_kv + 3
    kc = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)
    vc = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)
    q = r.standard_normal((n_new, n_head, hd)).astype(np.float32)
    mask = np.zeros((n_new, n_kv), dtype=np.float32)
    n_past = n_kv - n_new
    for i in range(n_new):
        mask[i, n_past + i + 1:] = -np.inf

    def build(g):
        return attention_graph(g, hd, n_head, n_head_kv, n_kv, n_new, n_ctx, kc, vc, q, mask, flash)

    a, names = profiled(hip, lambda: run_on(hip, build))
    b = run_on(cpu, build)
    assert "attn_prefill" in names, names
    if flash:
        assert rel_err_floor(a, b) < TOL, rel_err_floor(a, b)
    else:
        assert np.array_equal(a, b), rel_err(a, b)


@pytest.mark.parametrize("hd,n_head,n_head_kv,n_kv,n_new", [
    (128, 32, 4, 4112, 16),   # the MoE config's 16-token step at position 4096
    (128, 8, 8, 3000, 7),     # a partial last group of queries
    (64, 4, 2, 9000, 5),
    (96, 8, 8, 2500, 20),     # Phi-3 head dim
    (128, 24, 8, 2300, 70),   # Llama GQA group of 3, two launches of up to 64 queries
])
@pytest.mark.parametrize("flash", [False, True])
def test_attention_long_context_query_groups(hip, cpu, hd, n_head, n_head_kv, n_kv, n_new, flash):
    """A multi-token step over more positions than the prefill kernel holds in LDS: the multi-query
    decode kernels (scores and P V on the f64 matrix cores over tiles of 16 (query, head) rows,
    launches of up to 64 queries), the chain's float roundings exactly."""
    r = rng(n_kv + 7 * n_new)
    n_ctx = n_kv + 3
    kc = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)
    vc = r.standard_normal((n_ctx, n_head_kv, hd)).astype(np.float16)
    q = r.standard_normal((n_new, n_head, hd)).astype(np.float32)
    mask = np.zeros((n_new, n_kv), dtype=np.float32)
    n_past = n_kv - n_new
    for i in range(n_new):
        mask[i, n_past + i + 1:] = -np.inf

    def build(g):
        return attention_graph(g, hd, n_head, n_head_kv, n_kv, n_new, n_ctx, kc, vc, q, mask, flash)

    a, names = profiled(hip, lambda: run_on(hip, build))
    b = run_on(cpu, build)
    assert "attn_decode" in names and "attn_prefill" not in names, names
    if flash:
        assert rel_err_floor(a, b) < TOL, rel_err_floor(a, b)
    else:
        assert np.array_equal(a, b), rel_err(a, b)


@pytest.mark.parametrize("qtype,ncols", [(gl.Q8_0, 1), (gl.Q8_0, 77), (gl.Q4_0, 100), (gl.Q4_K, 5)])
def test_swiglu_fused_halves(hip, cpu, qtype, ncols):
    """The fused gate/up projection's halves (phi3, model.cpp:1119-1121): silu(gate) * up as one
    kernel that also writes the down projection's Q8_0 input; the same floats as the op chain."""
    E, F = 256, 512
    x = rng(80 + ncols).standard_normal((ncols, E)).astype(np.float32)
    wgu = qweight(qtype, E, 2 * F, 81, std=0.05)
    wd = qweight(qtype, F, E, 82, std=0.05)

    def build(g):
        gu = g.mul_mat(g.tensor(qtype, E, 2 * F, data=wgu), g.tensor(gl.F32, E, ncols, data=x))
        nb1 = 2 * F * 4
        gate, up = g.view_2d(gu, F, ncols, nb1, 0), g.view_2d(gu, F, ncols, nb1, F * 4)
        act = g.mul(g.silu(gate), up)
        return [act, g.mul_mat(g.tensor(qtype, F, E, data=wd), act)]

    (a_act, a_out), names = profiled(hip, lambda: run_on(hip, build))
    b_act, b_out = run_on(cpu, build)
    assert "swiglu" in names, names
    assert np.array_equal(a_act, b_act) and np.array_equal(a_out, b_out), (rel_err(a_act, b_act), rel_err(a_out, b_out))


@pytest.mark.parametrize("qtype", [gl.Q4_0, gl.Q8_0, gl.Q4_K])
def test_swiglu_separate_projections(hip, cpu, qtype):
    """Separate gate and up projections at prefill width (llama/qwen FFN, model.cpp:1122-1126): the
    silu comes before the up projection in node order; it is held back and runs with the mul as one
    kernel writing the down projection's Q8_0 / Q8_K input. The same floats as the op chain."""
    E, F, ncols = 256, 512, 96
    x = rng(90).standard_normal((ncols, E)).astype(np.float32)
    wg, wu = qweight(qtype, E, F, 91, std=0.05), qweight(qtype, E, F, 92, std=0.05)
    wd = qweight(qtype, F, E, 93, std=0.05)

    def build(g):
        xt = g.tensor(gl.F32, E, ncols, data=x)
        gate = g.silu(g.mul_mat(g.tensor(qtype, E, F, data=wg), xt))
        act = g.mul(gate, g.mul_mat(g.tensor(qtype, E, F, data=wu), xt))
        return [act, g.mul_mat(g.tensor(qtype, F, E, data=wd), act)]

    (a_act, a_out), names = profiled(hip, lambda: run_on(hip, build))
    b_act, b_out = run_on(cpu, build)
    assert "swiglu" in names and "unary" not in names, names
    assert np.array_equal(a_act, b_act) and np.array_equal(a_out, b_out), (rel_err(a_act, b_act), rel_err(a_out, b_out))


def f16_tie_scores(n_kv, seed):
    """Scores (F16, one head, scale 1/8) whose softmax holds a probability p = e * (1/S) that is an
    exact F16 rounding tie as a float, while the exact product e * (1/S) lies on the side whose
    rounding disagrees with round-half-to-even: converting the product to F16 in one rounding
    (instead of rounding it to float first, as the graph does) gives the other neighbour."""
    r = rng(seed)
    for _ in range(100000):
        s = (r.standard_normal(n_kv) * 2).astype(np.float16)
        w = s.astype(np.float32) * np.float32(0.125)
        e = np.exp((w - w.max()).astype(np.float64)).astype(np.float32)
        inv = np.float32(1.0 / e.astype(np.float64).sum())
        p = e * inv
        exact = e.astype(np.float64) * np.float64(inv)
        bits = p.view(np.uint32)
        tie = ((bits & 0x1FFF) == 0x1000) & (p >= 2.0 ** -14)
        odd = (bits >> 13) & 1
        flips = tie & (((exact > p) & (odd == 0)) | ((exact < p) & (odd == 1)))
        if flips.any():
            return s, int(np.argmax(flips))
    raise AssertionError("no tie found")


def test_attention_f16_probability_ties(hip, cpu):
    """Regression: a probability on an F16 tie must round like the graph's float -> F16 operand
    conversion (first to float, then half to even)."""
    hd, n_kv = 64, 64
    s, t = f16_tie_scores(n_kv, 3)
    kc = np.zeros((n_kv, 1, hd), dtype=np.float16)
    kc[:, 0, 0] = s
    vc = rng(4).standard_normal((n_kv, 1, hd)).astype(np.float16)
    q = np.zeros((1, 1, hd), dtype=np.float32)
    q[0, 0, 0] = 1.0
    mask = np.zeros((1, n_kv), dtype=np.float32)

    def build(g):
        return attention_graph(g, hd, 1, 1, n_kv, 1, n_kv, kc, vc, q, mask)

    for fusion in (True, False):
        a, b = both(hip, cpu, build, fusion)
        assert np.array_equal(a, b), (fusion, t, rel_err(a, b))


# ---- MoE --------------------------------------------------------------------------------------

@pytest.mark.parametrize("n", [8, 128, 1000])
def test_argsort_sum_rows_div(hip, cpu, n):
    x = rng(60 + n).integers(-4, 5, (3, n)).astype(np.float32) * 0.5     # ties
    x[1] = rng(61).standard_normal(n).astype(np.float32)

    def build(g):
        xt = g.tensor(gl.F32, n, 3, data=x)
        s = g.sum_rows(xt)
        return [g.argsort(xt, gl.SORT_DESC), g.argsort(xt, gl.SORT_ASC), s, g.div(xt, s)]

    hs, cs = both(hip, cpu, build)
    for a, b in zip(hs, cs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(hs[0].view(np.int32).reshape(3, n), np.argsort(-x, axis=1, kind="stable"))


@pytest.mark.parametrize("qtype", [gl.Q4_0, gl.Q8_0, gl.Q4_K, gl.Q5_K, gl.Q6_K])
@pytest.mark.parametrize("n_tok", [1, 3, 16, 37])
def test_moe_ffn(hip, cpu, qtype, n_tok):
    """The routed expert FFN (router, top-k, renormalized weights, mul_mat_id gate/up/down, SwiGLU,
    weighted slot sum, residual): fused into the GEMV and weighted-sum kernels or node by node."""
    n_embd, E, k, ff = 512, 32, 8, 256
    r = rng(70)
    y = r.standard_normal((n_tok, n_embd)).astype(np.float32)
    res = r.standard_normal((n_tok, n_embd)).astype(np.float32)
    router = (r.standard_normal((E, n_embd)) * 0.05).astype(np.float32)
    wg, wu = (qweight(qtype, n_embd, E * ff, s, std=0.05) for s in (71, 72))
    wd = qweight(qtype, ff, E * n_embd, 73, std=0.05)

    def build(g):
        return moe_ffn_graph(g, g.tensor(gl.F32, n_embd, n_tok, data=y), g.tensor(gl.F32, n_embd, E, data=router),
                             g.tensor(qtype, n_embd, ff, E, data=wg), g.tensor(qtype, n_embd, ff, E, data=wu),
                             g.tensor(qtype, ff, n_embd, E, data=wd), k, g.tensor(gl.F32, n_embd, n_tok, data=res))

    for fusion in (True, False):
        a, b = both(hip, cpu, build, fusion)
        assert np.array_equal(a, b), (fusion, rel_err(a, b))
    _, names = profiled(hip, lambda: run_on(hip, build))
    assert "argsort" not in names, names
    # one token on the single-column Q4_K kernel: the routing runs inside the gate/up launch
    in_gemv = qtype == gl.Q4_K and n_tok == 1
    assert ("moe_route" in names) != in_gemv and ("gemv_q4_K_swiglu_route" in names) == in_gemv, names
    if qtype in (gl.Q5_K, gl.Q6_K):
        # no multi-column kernel for these types: each (token, slot) column reads its expert
        assert "moe_group" not in names, names
    else:
        assert (n_tok >= 2) == ("moe_group" in names), names   # several tokens: experts read once for all of theirs


@pytest.mark.parametrize("n_tok", [1, 5])
def test_moe_ffn_norm_folded_into_router(hip, cpu, n_tok):
    """The MoE FFN norm (rms_norm -> mul) whose first reader is the F32 router: no launch of its own;
    the router launch normalizes each column (the rms_norm op's roundings) and writes the normalized
    activation the expert GEMVs read afterwards."""
    n_embd, E, k, ff = 512, 32, 8, 256
    r = rng(74)
    x = (r.standard_normal((n_tok, n_embd)) * 3).astype(np.float32)
    nw = (1 + 0.01 * r.standard_normal(n_embd)).astype(np.float32)
    router = (r.standard_normal((E, n_embd)) * 0.05).astype(np.float32)
    wg, wu = (qweight(gl.Q4_K, n_embd, E * ff, s, std=0.05) for s in (75, 76))
    wd = qweight(gl.Q4_K, ff, E * n_embd, 77, std=0.05)

    def build(g):
        xt = g.tensor(gl.F32, n_embd, n_tok, data=x)
        y = g.mul(g.rms_norm(xt, 1e-6), g.tensor(gl.F32, n_embd, data=nw))
        return moe_ffn_graph(g, y, g.tensor(gl.F32, n_embd, E, data=router),
                             g.tensor(gl.Q4_K, n_embd, ff, E, data=wg), g.tensor(gl.Q4_K, n_embd, ff, E, data=wu),
                             g.tensor(gl.Q4_K, ff, n_embd, E, data=wd), k, xt)

    for fusion in (True, False):
        a, b = both(hip, cpu, build, fusion)
        assert np.array_equal(a, b), (fusion, rel_err(a, b))
    _, names = profiled(hip, lambda: run_on(hip, build))
    assert "router_norm" in names and "rms_norm_mul" not in names, names


@pytest.mark.parametrize("ptype,n_tok,with_res", [(gl.Q4_K, 16, True), (gl.Q4_K, 5, True), (gl.Q6_K, 3, False),
                                                  (gl.Q4_0, 5, True), (gl.Q4_K, 1, True)])
def test_moe_sum_feeds_next_norm_q8k(hip, cpu, ptype, n_tok, with_res):
    """The MoE weighted sum (+ residual) read by the next rms_norm -> mul whose readers are K-quant
    GEMVs, over several tokens: one launch writes the residual stream and its normalized Q8_K copy
    (the act_quant launch's arithmetic), and every output is the oracle's."""
    n_embd, E, k, ff = 512, 32, 8, 256
    r = rng(82 + n_tok)
    y = r.standard_normal((n_tok, n_embd)).astype(np.float32)
    res = r.standard_normal((n_tok, n_embd)).astype(np.float32)
    nw = (1 + 0.01 * r.standard_normal(n_embd)).astype(np.float32)
    router = (r.standard_normal((E, n_embd)) * 0.05).astype(np.float32)
    wg, wu = (qweight(gl.Q4_K, n_embd, E * ff, s, std=0.05) for s in (83, 84))
    wd = qweight(gl.Q4_K, ff, E * n_embd, 85, std=0.05)
    wq, wk = qweight(ptype, n_embd, 512, 86), qweight(ptype, n_embd, 256, 87)

    def build(g):
        out = moe_ffn_graph(g, g.tensor(gl.F32, n_embd, n_tok, data=y), g.tensor(gl.F32, n_embd, E, data=router),
                            g.tensor(gl.Q4_K, n_embd, ff, E, data=wg), g.tensor(gl.Q4_K, n_embd, ff, E, data=wu),
                            g.tensor(gl.Q4_K, ff, n_embd, E, data=wd), k,
                            g.tensor(gl.F32, n_embd, n_tok, data=res) if with_res else None)
        h = g.mul(g.rms_norm(out, 1e-6), g.tensor(gl.F32, n_embd, data=nw))
        return [out, g.mul_mat(g.tensor(ptype, n_embd, 512, data=wq), h), g.mul_mat(g.tensor(ptype, n_embd, 256, data=wk), h)]

    for fusion in (True, False):
        hs, cs = both(hip, cpu, build, fusion)
        for a, b in zip(hs, cs):
            assert np.array_equal(a, b), (fusion, rel_err(a, b))
    _, names = profiled(hip, lambda: run_on(hip, build))
    fused = n_tok >= 2 and ptype != gl.Q4_0
    assert ("moe_wsum_q8k" in names) == fused and ("moe_wsum" in names) != fused, names
    if fused:
        assert "act_quant" not in names and "rms_norm_mul" not in names, names


@pytest.mark.parametrize("n_tok", [1, 5])
def test_moe_router_norm_kept_apart_when_its_input_dies(hip, cpu, n_tok):
    """The norm's input computed in the graph and read by nothing after the norm: the allocator may
    reuse its memory before the router runs, so the norm keeps a launch of its own instead of being
    folded into the router launch (which reads the input later), and the result is the oracle's."""
    n_embd, E, k, ff = 512, 32, 8, 256
    r = rng(78)
    x = (r.standard_normal((n_tok, n_embd)) * 3).astype(np.float32)
    res = r.standard_normal((n_tok, n_embd)).astype(np.float32)
    nw = (1 + 0.01 * r.standard_normal(n_embd)).astype(np.float32)
    router = (r.standard_normal((E, n_embd)) * 0.05).astype(np.float32)
    wg, wu = (qweight(gl.Q4_K, n_embd, E * ff, s, std=0.05) for s in (79, 80))
    wd = qweight(gl.Q4_K, ff, E * n_embd, 81, std=0.05)

    def build(g):
        xin = g.tensor(gl.F32, n_embd, n_tok, data=x)
        xt = g.scale(xin, 0.5)                                  # a node: dead after the norm
        y = g.mul(g.rms_norm(xt, 1e-6), g.tensor(gl.F32, n_embd, data=nw))
        return moe_ffn_graph(g, y, g.tensor(gl.F32, n_embd, E, data=router),
                             g.tensor(gl.Q4_K, n_embd, ff, E, data=wg), g.tensor(gl.Q4_K, n_embd, ff, E, data=wu),
                             g.tensor(gl.Q4_K, ff, n_embd, E, data=wd), k, g.tensor(gl.F32, n_embd, n_tok, data=res))

    for fusion in (True, False):
        a, b = both(hip, cpu, build, fusion)
        assert np.array_equal(a, b), (fusion, rel_err(a, b))
    _, names = profiled(hip, lambda: run_on(hip, build))
    assert "router_norm" not in names, names


@pytest.mark.parametrize("E,k,n_tok", [(128, 8, 1), (128, 8, 16), (60, 4, 3), (1024, 32, 2), (8, 8, 1)])
def test_moe_route_fused(hip, cpu, E, k, n_tok):
    """Router softmax -> top-k -> renormalized weights in one kernel: the same ids (ties: the lower
    expert first) and weights as the op chain, logits with many exact ties included."""
    r = rng(E + k + n_tok)
    lg = r.standard_normal((n_tok, E)).astype(np.float32)
    lg[0, ::3] = 0.75          # many equal probabilities, some of them among the top
    if n_tok > 1:
        lg[1] = np.round(lg[1])

    ids_table = np.tile(np.arange(E, dtype=np.float32), (n_tok, 1))   # row t: expert e -> float(e)

    def build(g):
        probs = g.soft_max_ext(g.tensor(gl.F32, E, n_tok, data=lg), None, 1.0, 0.0)
        sel = g.top_k(probs, k)
        w = g.reshape_2d(g.get_rows(g.reshape_3d(probs, 1, E, n_tok), sel), k, n_tok)
        w = g.div(w, g.sum_rows(w))
        ids = g.get_rows(g.tensor(gl.F32, 1, E, n_tok, data=ids_table), sel)   # the selected ids, as floats
        return [ids, w]

    (ia, wa), names = profiled(hip, lambda: run_on(hip, build))
    ib, wb = run_on(cpu, build)
    assert "moe_route" in names, names
    assert np.array_equal(ia, ib)
    assert np.array_equal(wa, wb)
    order = np.argsort(-lg, axis=1, kind="stable")[:, :k]
    assert np.array_equal(ia.reshape(n_tok, k).astype(np.int64), order)


@pytest.mark.parametrize("E,k,fold_norm", [(128, 8, True), (128, 8, False), (256, 8, False), (60, 4, True), (8, 8, False)])
def test_moe_route_inside_gate_up_gemv(hip, cpu, E, k, fold_norm):
    """One token's routing run by the workgroups of the routed gate/up + SwiGLU launch (no
    launch of its own), with exact ties straddling the top-k boundary (duplicated router rows: the
    lower expert id wins) and the column pre-quantized by the router launch (fold_norm) or
    quantized in the prologue: the whole FFN bit-exact against the op-by-op oracle. The tied
    experts' weights differ, so a tie decided the other way shows in the output."""
    n_embd, ff = 1024, 256
    r = rng(90 + E + k)
    x = (r.standard_normal((1, n_embd)) * 2).astype(np.float32)
    res = r.standard_normal((1, n_embd)).astype(np.float32)
    nw = (1 + 0.01 * r.standard_normal(n_embd)).astype(np.float32)
    router = (r.standard_normal((E, n_embd)) * 0.002).astype(np.float32)   # logits well below the planted ones
    # router rows along x (logits about a_e, or a_e / rms(x) after the norm): the top k - 1
    # distinct, then three equal rows at random ids, the lowest of which takes the last slot
    u = x[0] / float(np.dot(x[0], x[0]))
    top = r.permutation(E)[: k + 2]
    for j, e in enumerate(top[: k - 1]):
        router[e] = (4.0 - 0.3 * j) * u
    for e in top[k - 1:]:
        router[e] = 1.5 * u
    wg, wu = (qweight(gl.Q4_K, n_embd, E * ff, s, std=0.05) for s in (91, 92))
    wd = qweight(gl.Q4_K, ff, E * n_embd, 93, std=0.05)

    def build(g):
        xt = g.tensor(gl.F32, n_embd, 1, data=x)
        y = g.mul(g.rms_norm(xt, 1e-6), g.tensor(gl.F32, n_embd, data=nw)) if fold_norm else xt
        return moe_ffn_graph(g, y, g.tensor(gl.F32, n_embd, E, data=router),
                             g.tensor(gl.Q4_K, n_embd, ff, E, data=wg), g.tensor(gl.Q4_K, n_embd, ff, E, data=wu),
                             g.tensor(gl.Q4_K, ff, n_embd, E, data=wd), k, g.tensor(gl.F32, n_embd, 1, data=res))

    for fusion in (True, False):
        a, b = both(hip, cpu, build, fusion)
        assert np.array_equal(a, b), (fusion, rel_err(a, b))
    _, names = profiled(hip, lambda: run_on(hip, build))
    assert "gemv_q4_K_swiglu_route" in names and "moe_route" not in names, names
    if fold_norm:
        assert "router_norm" in names, names


def test_other_arch_ops(hip, cpu):
    """The ops the reference's other graphs add (model.cpp:1156-1295, dory.c:722-724): sub, abs,
    softplus, l2_norm, concat, swiglu_split, bit-exact against the oracle."""
    r = rng(31)
    a = (r.standard_normal((3, 5, 130)) * 6).astype(np.float32)
    b = r.standard_normal((3, 5, 130)).astype(np.float32)
    c = r.standard_normal((3, 2, 130)).astype(np.float32)
    row = r.standard_normal(130).astype(np.float32)

    def build(g):
        ta = g.tensor(gl.F32, 130, 5, 3, data=a)
        tb = g.tensor(gl.F32, 130, 5, 3, data=b)
        tc = g.tensor(gl.F32, 130, 2, 3, data=c)
        tr = g.tensor(gl.F32, 130, data=row)
        return [g.sub(ta, tr), g.abs(ta), g.softplus(ta), g.l2_norm(ta, 1e-6), g.concat(ta, tc, 1),
                g.concat(ta, tb, 2), g.swiglu_split(ta, tb)]

    got, ref = run_on(hip, build), run_on(cpu, build)
    for k, (x, y) in enumerate(zip(got, ref)):
        assert np.array_equal(x, y), k
