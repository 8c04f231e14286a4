"""Pins the oracle (oracle/ggml_cpu_oracle.c, the CPU restatement of ggml-cpu) before it is trusted
as the checker of the HIP backend. Runs on the CPU only.

Each check is chosen so that a plausible mistake in the restatement (a wrong nibble order, sign,
scale index, pair index or GQA mapping, a dropped term) fails it:
  * golden vectors of the reference's own decoders and scalar primitives (tests/golden/*.npz, made
    by tests/golden/make_golden.py from src/moe_stream/dequant.c and compute_backend.c);
  * IEEE binary16 (numpy) for the f16 conversions, exhaustively / on 2M patterns;
  * closed forms: Q4_0 decode over every nibble, quantizer error bounds, RoPE at position 0,
    rotation norms, NORMAL/NEOX index relation, softmax row sums, attention special cases;
  * fp64 brute force over the same quantized operands for every dot/GEMV path.
The product's own host-side quantizers and decoders (libggml.so) are held to the oracle byte for
byte here as well.
"""
import ctypes as C
import os

import numpy as np
import pytest

from gl import GOLDEN, Graph, attention_graph, cpu_backend, dequantize, gl, oracle, ptr, quantize, rel_err

Q8_K = 15


@pytest.fixture(scope="module")
def cpu():
    b = cpu_backend(8)
    yield b
    gl.libs()["core"].ggml_backend_free(b)


def rng(seed):
    return np.random.default_rng(seed)


def run_cpu(cpu, build):
    with Graph() as g:
        return g.compute(cpu, build(g))


def golden(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


# ---- IEEE binary16 ---------------------------------------------------------------------------

def test_fp16_to_fp32_exhaustive(cpu):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    got = run_cpu(cpu, lambda g: g.cast(g.tensor(gl.F16, 65536, data=codes), gl.F32))
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    o = oracle()
    for h in (0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0x7C00, 0x8001, 0xFBFF):
        assert o.oracle_fp16_to_fp32(h) == float(np.uint16(h).view(np.float16))


def test_fp32_to_fp16_rounding(cpu):
    r = rng(1)
    bits = r.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    # concentrate on the f16 range, ties, subnormals and the overflow threshold
    near = (r.integers(0x33000000, 0x47800000, 1_000_000, dtype=np.uint64).astype(np.uint32) & ~np.uint32(0xFFF)) | 0x1000
    special = np.array([0x477FEFFF, 0x477FF000, 0x477FF001, 0x38800000, 0x387FC000, 0x33800000, 0x33000000,
                        0x33000001, 0x80000000, 0x7F800000, 0xFF800000, 0x3F800000], dtype=np.uint32)
    x = np.concatenate([bits, near, special]).view(np.float32)
    x = x[~np.isnan(x)]
    got = run_cpu(cpu, lambda g: g.cast(g.tensor(gl.F32, x.size, data=x), gl.F16))
    got = got.view(np.uint16)[: x.size]
    with np.errstate(over="ignore"):
        expect = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, expect), int(np.sum(got != expect))


# ---- block decoders --------------------------------------------------------------------------

def test_q4_0_decode_closed_form():
    """Q4_0 = {f16 d; u8 qs[16]}: element j = (lo nibble of qs[j] - 8) d, element j+16 = (hi - 8) d.
    Every nibble value at every position, scales of both signs, zero, subnormal and the largest."""
    scales = np.array([0.01, -0.037, 0.0, 6e-8, 6.1e-5, 1.0, 65504.0, -2.5], dtype=np.float16)
    blocks, expect = [], []
    for d in scales:
        for b in range(16):
            lo = (np.arange(16) + b) % 16
            hi = (15 - np.arange(16) - b) % 16
            blk = np.zeros(18, dtype=np.uint8)
            blk[0:2] = np.atleast_1d(d).view(np.uint8)
            blk[2:] = (lo | (hi << 4)).astype(np.uint8)
            blocks.append(blk)
            df = np.float32(d)
            expect.append(np.concatenate([(lo - 8).astype(np.float32) * df, (hi - 8).astype(np.float32) * df]))
    q = np.concatenate(blocks)
    expect = np.concatenate(expect)
    for impl in ("oracle", "product"):
        got = dequantize(q, gl.Q4_0, expect.size, impl)
        assert np.array_equal(got.view(np.uint32), expect.view(np.uint32)), impl


@pytest.mark.parametrize("qtype,key", [(gl.Q4_K, "q4k"), (gl.Q8_0, "q8_0")])
def test_decode_matches_reference_golden(qtype, key):
    z = golden("dequant_ref.npz")
    q, ref = z[f"{key}_in"], z[f"{key}_out"]
    for impl in ("oracle", "product"):
        got = dequantize(q, qtype, ref.size, impl)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), impl


def test_decode_golden_discriminates():
    """The Q4_K golden vectors tell apart the two nibble halves and the scale/min pairing: a decoder
    that swaps them would fail the test above."""
    z = golden("dequant_ref.npz")
    q, ref = z["q4k_in"].copy(), z["q4k_out"]
    blk = q[9 * 144:10 * 144]
    blk[16:] = ((blk[16:] >> 4) | (blk[16:] << 4)).astype(np.uint8)   # swap nibbles of one block
    got = dequantize(q, gl.Q4_K, ref.size)
    assert not np.array_equal(got, ref)


# ---- quantizers ------------------------------------------------------------------------------

def q8_k_decode(q):
    """Q8_K block = {f32 d; i8 qs[256]; i16 bsums[16]} (292 bytes)."""
    nb = q.size // 292
    blk = q.reshape(nb, 292)
    d = blk[:, 0:4].copy().view(np.float32).reshape(nb, 1)
    qs = blk[:, 4:260].copy().view(np.int8).astype(np.int64)
    bs = blk[:, 260:292].copy().view(np.int16).astype(np.int64)
    return d, qs, bs


@pytest.mark.parametrize("qtype", [gl.Q4_0, gl.Q8_0, gl.Q4_K, Q8_K])
def test_product_quantizer_matches_oracle(qtype):
    x = (rng(2).standard_normal(256 * 24) * 0.3).astype(np.float32)
    x[:256] = 0.0
    x[256:512] = 0.125
    if qtype == Q8_K:
        a = np.zeros(x.size // 256 * 292, dtype=np.uint8)
        oracle().oracle_quantize_q8_K(ptr(x), ptr(a), x.size)
        b = np.zeros_like(a)
        gl.libs()["core"].ggml_quantize_chunk(Q8_K, ptr(x), ptr(b), 0, 1, x.size, None)
    else:
        a = quantize(x, qtype, "oracle")
        b = quantize(x, qtype, "product")
    assert np.array_equal(a, b)


def test_q4_0_quantizer_bounds():
    x = (rng(3).standard_normal(32 * 200) * rng(4).uniform(0.01, 5, 32 * 200)).astype(np.float32)
    x[:32] = 0
    x[32:64] = -1.5
    q = quantize(x, gl.Q4_0)
    y = dequantize(q, gl.Q4_0, x.size)
    d = np.abs(q.reshape(-1, 18)[:, 0:2].copy().view(np.float16).astype(np.float64)).repeat(32)
    err = np.abs(y.astype(np.float64) - x)
    xb = x.reshape(-1, 32)
    amax = xb[np.arange(xb.shape[0]), np.abs(xb).argmax(1)]
    # the element of largest magnitude is the block's -8 code: reproduced up to the f16 rounding of d
    assert np.all(np.abs(y.reshape(-1, 32)[np.arange(xb.shape[0]), np.abs(xb).argmax(1)] - amax) <= 8 * 2 ** -11 * np.abs(amax) + 1e-30)
    # in range codes round to nearest (plus the f16 rounding of d); the +8 end clips to 7
    assert np.all(err <= d * (1 + 2 ** -10) + 1e-30)
    # a zero block: d = 0 / -8 = -0.0 and every code 8, so every element decodes to (-)0
    assert np.all(y[:32] == 0) and q[:2].view(np.float16)[0] == 0
    assert np.all(np.abs(y[32:64] + 1.5) < 1e-6)


def test_q8_0_quantizer_bounds():
    x = (rng(5).standard_normal(32 * 200) * 3).astype(np.float32)
    q = quantize(x, gl.Q8_0)
    y = dequantize(q, gl.Q8_0, x.size)
    xb = np.abs(x.reshape(-1, 32)).max(1).astype(np.float64)
    dd = (xb / 127).repeat(32)
    assert np.all(np.abs(y - x) <= dd * 0.5 + 127 * dd * 2 ** -11 + 1e-30)
    qs = q.reshape(-1, 34)[:, 2:].view(np.int8)
    assert np.all(np.abs(qs).max(1) == 127)


def test_q8_K_quantizer_invariants():
    x = (rng(6).standard_normal(256 * 8) * 2).astype(np.float32)
    x[:256] = 0
    q = np.zeros(8 * 292, dtype=np.uint8)
    oracle().oracle_quantize_q8_K(ptr(x), ptr(q), x.size)
    d, qs, bs = q8_k_decode(q)
    assert np.all(d[0] == 0) and np.all(qs[0] == 0)
    assert np.array_equal(bs, qs.reshape(8, 16, 16).sum(2))
    assert np.all(np.abs(qs[1:]).max(1) == 127)
    err = np.abs(d.astype(np.float64) * qs - x.reshape(8, 256))
    assert np.all(err <= np.abs(d) * 0.5 * (1 + 1e-6) + 1e-30)


def test_q4_K_quantizer_quality():
    x = (rng(7).standard_normal(256 * 64) * 0.02).astype(np.float32)
    x[:256] = 0
    y = dequantize(quantize(x, gl.Q4_K), gl.Q4_K, x.size)
    assert np.all(y[:256] == 0)
    # 4-bit codes with 6-bit sub-block scales: RMS error near 1/15 of a sub-block range
    rms = np.sqrt(np.mean((y[256:] - x[256:]) ** 2)) / np.std(x[256:])
    assert rms < 0.12, rms


# ---- dots and GEMV ---------------------------------------------------------------------------

def act_dequant(x, qtype):
    """The activation the oracle's dot sees: x quantized to the weight's dot type, decoded."""
    if qtype in (gl.Q4_0, gl.Q8_0):
        return dequantize(quantize(x, gl.Q8_0), gl.Q8_0, x.size).astype(np.float64)
    q = np.zeros(x.size // 256 * 292, dtype=np.uint8)
    oracle().oracle_quantize_q8_K(ptr(x), ptr(q), x.size)
    d, qs, _ = q8_k_decode(q)
    return (d.astype(np.float64) * qs).reshape(-1)


@pytest.mark.parametrize("qtype,K,N", [(gl.Q4_0, 4096, 64), (gl.Q8_0, 3072, 48), (gl.Q4_K, 2560, 40)])
def test_gemv_fp64_brute_force(qtype, K, N):
    W = quantize((rng(K).standard_normal((N, K)) * 0.02).astype(np.float32), qtype)
    Wd = dequantize(W, qtype, N * K).reshape(N, K).astype(np.float64)
    x = rng(K + 1).standard_normal(K).astype(np.float32)
    y = np.zeros(N, dtype=np.float32)
    oracle().oracle_gemv(qtype, ptr(W), N, K, ptr(x), ptr(y), 4)
    ref = Wd @ act_dequant(x, qtype)
    assert rel_err(y, ref) < 2e-6
    # and the graph path of the CPU backend computes the same floats as oracle_gemv
    cpu = cpu_backend(4)
    try:
        got = run_cpu(cpu, lambda g: g.mul_mat(g.tensor(qtype, K, N, data=W), g.tensor(gl.F32, K, 1, data=x)))
    finally:
        gl.libs()["core"].ggml_backend_free(cpu)
    assert np.array_equal(got, y)


def test_gemv_one_hot_column():
    """x = e_j: the output is column j of the decoded weight times the decoded activation value."""
    K, N = 1024, 32
    W = quantize((rng(9).standard_normal((N, K)) * 0.02).astype(np.float32), gl.Q4_0)
    Wd = dequantize(W, gl.Q4_0, N * K).reshape(N, K).astype(np.float64)
    for j in (0, 17, 31, 32, 1023):
        x = np.zeros(K, dtype=np.float32)
        x[j] = 1.0
        y = np.zeros(N, dtype=np.float32)
        oracle().oracle_gemv(gl.Q4_0, ptr(W), N, K, ptr(x), ptr(y), 1)
        xd = act_dequant(x, gl.Q4_0)[j]
        assert np.allclose(y, Wd[:, j] * xd, rtol=1e-6, atol=0)


def test_q4_K_gemv_against_reference_matmul():
    """The reference's sc_matmul (exact f32 activations) agrees with the fp64 dot of the decoded rows,
    and the oracle's Q8_K-activation GEMV stays within the activation quantization bound of it."""
    z = golden("scalar_ref.npz")
    K, N = int(z["mm_k"]), int(z["mm_n"])
    W, x, yref = z["mm_w"], z["mm_x"], z["mm_y"]
    Wd = dequantize(W, gl.Q4_K, N * K).reshape(N, K).astype(np.float64)
    assert rel_err(yref, Wd @ x.astype(np.float64)) < 1e-5
    y = np.zeros(N, dtype=np.float32)
    oracle().oracle_gemv(gl.Q4_K, ptr(W), N, K, ptr(x), ptr(y), 1)
    xq = act_dequant(x, gl.Q4_K)
    bound = np.abs(Wd) @ np.abs(xq - x) + 1e-5 * np.abs(yref)
    assert np.all(np.abs(y - yref) <= bound)


@pytest.mark.parametrize("fn,wt,n", [("oracle_vec_dot_q4_0_q8_0", gl.Q4_0, 512), ("oracle_vec_dot_q8_0_q8_0", gl.Q8_0, 512),
                                     ("oracle_vec_dot_q4_K_q8_K", gl.Q4_K, 1024)])
def test_vec_dot_brute_force(fn, wt, n):
    w = quantize((rng(10).standard_normal(n) * 0.1).astype(np.float32), wt)
    x = rng(11).standard_normal(n).astype(np.float32)
    if wt == gl.Q4_K:
        xq = np.zeros(n // 256 * 292, dtype=np.uint8)
        oracle().oracle_quantize_q8_K(ptr(x), ptr(xq), n)
    else:
        xq = quantize(x, gl.Q8_0)
    got = getattr(oracle(), fn)(n, ptr(w), ptr(xq))
    ref = float(dequantize(w, wt, n).astype(np.float64) @ act_dequant(x, wt))
    assert abs(got - ref) <= 1e-6 * np.sum(np.abs(dequantize(w, wt, n)) * np.abs(act_dequant(x, wt))) + 1e-12


# ---- float primitives against the reference's scalar engine ----------------------------------

def test_rms_norm_mul_matches_reference(cpu):
    z = golden("scalar_ref.npz")
    x, w, eps, ref = z["rms_x"], z["rms_w"], float(z["rms_eps"]), z["rms_out"]
    got = run_cpu(cpu, lambda g: g.mul(g.rms_norm(g.tensor(gl.F32, x.shape[1], x.shape[0], data=x), eps),
                                       g.tensor(gl.F32, x.shape[1], data=w)))
    assert rel_err(got, ref) < 1e-6


def test_softmax_matches_reference(cpu):
    z = golden("scalar_ref.npz")
    x, ref = z["sm_x"], z["sm_out"]
    got = run_cpu(cpu, lambda g: g.soft_max_ext(g.tensor(gl.F32, x.shape[1], x.shape[0], data=x), None, 1.0, 0.0))
    assert rel_err(got, ref) < 1e-6
    assert np.allclose(got.reshape(x.shape).sum(1), 1.0, atol=1e-6)


def test_softmax_mask_and_scale(cpu):
    n_kv, n_q = 40, 3
    x = (rng(12).standard_normal((n_q, n_kv)) * 5).astype(np.float32)
    m = np.zeros((n_q, n_kv), dtype=np.float32)
    m[0, 10:] = -np.inf
    m[1, 1:] = -np.inf
    got = run_cpu(cpu, lambda g: g.soft_max_ext(g.tensor(gl.F32, n_kv, n_q, data=x), g.tensor(gl.F32, n_kv, n_q, data=m),
                                                0.25, 0.0)).reshape(n_q, n_kv)
    assert np.all(got[0, 10:] == 0) and got[1, 0] == 1.0 and np.all(got[1, 1:] == 0)
    w = x.astype(np.float64) * 0.25 + m
    ref = np.exp(w - w.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    assert rel_err(got, ref) < 1e-6


def test_swiglu_matches_reference(cpu):
    z = golden("scalar_ref.npz")
    gt, up, ref = z["swi_gate"], z["swi_up"], z["swi_out"]
    got = run_cpu(cpu, lambda g: g.mul(g.silu(g.tensor(gl.F32, gt.size, data=gt)), g.tensor(gl.F32, up.size, data=up)))
    assert rel_err(got, ref) < 1e-6


def rope_cpu(cpu, x, pos, n_dims, mode, base):
    n_tok, n_head, hd = x.shape
    return run_cpu(cpu, lambda g: g.rope_ext(g.tensor(gl.F32, hd, n_head, n_tok, data=x),
                                             g.tensor(gl.I32, n_tok, data=np.asarray(pos, dtype=np.int32)), None,
                                             n_dims, mode, 4096, base, 1.0, 0.0, 1.0, 0.0, 0.0)).reshape(x.shape)


def test_rope_neox_matches_reference(cpu):
    z = golden("scalar_ref.npz")
    hd, base, pos, x, ref = int(z["rope_hd"]), float(z["rope_base"]), z["rope_pos"], z["rope_x"], z["rope_out"]
    got = rope_cpu(cpu, x.reshape(len(pos), 1, hd), pos, hd, gl.ROPE_NEOX, base).reshape(ref.shape)
    # ggml forms the angles by repeated float multiplication; the reference tables are double
    assert rel_err(got, ref) < 2e-5
    assert np.array_equal(got[0], x[0])


@pytest.mark.parametrize("mode", [gl.ROPE_NORMAL, gl.ROPE_NEOX])
def test_rope_identities(cpu, mode):
    hd, n_head = 128, 4
    pos = [0, 3, 2048, 8191]
    x = rng(13).standard_normal((len(pos), n_head, hd)).astype(np.float32)
    y = rope_cpu(cpu, x, pos, hd, mode, 500000.0)
    assert np.array_equal(y[0], x[0])
    if mode == gl.ROPE_NORMAL:
        a, b, ya, yb = x[..., 0::2], x[..., 1::2], y[..., 0::2], y[..., 1::2]
    else:
        a, b, ya, yb = x[..., :64], x[..., 64:], y[..., :64], y[..., 64:]
    assert np.allclose(np.hypot(ya, yb), np.hypot(a, b), rtol=2e-6, atol=1e-7)
    # the first pair rotates by the position itself (theta_0 = pos)
    p = 3
    c, s = np.cos(p), np.sin(p)
    assert np.allclose(ya[1, :, 0], a[1, :, 0] * c - b[1, :, 0] * s, atol=1e-6)
    assert np.allclose(yb[1, :, 0], a[1, :, 0] * s + b[1, :, 0] * c, atol=1e-6)


def test_rope_normal_is_neox_on_interleaved_pairs(cpu):
    """NORMAL rotates (2i, 2i+1), NEOX rotates (i, i + n/2), both by theta_i: they agree exactly
    once the pair layout is permuted."""
    hd = 96
    x = rng(14).standard_normal((3, 2, hd)).astype(np.float32)
    pos = [1, 77, 4000]
    perm = np.concatenate([np.arange(0, hd, 2), np.arange(1, hd, 2)])     # interleaved -> halves
    normal = rope_cpu(cpu, x, pos, hd, gl.ROPE_NORMAL, 10000.0)
    neox = rope_cpu(cpu, np.ascontiguousarray(x[..., perm]), pos, hd, gl.ROPE_NEOX, 10000.0)
    assert np.array_equal(normal[..., perm], neox)


def test_rope_partial_dims_pass_through(cpu):
    x = rng(15).standard_normal((2, 2, 128)).astype(np.float32)
    y = rope_cpu(cpu, x, [5, 9], 64, gl.ROPE_NEOX, 10000.0)
    assert np.array_equal(y[..., 64:], x[..., 64:])


# ---- attention chain -------------------------------------------------------------------------

def attention_fp64(kc, vc, q, n_kv, n_head_kv, mapping=lambda h, G, hkv: h // G):
    """Textbook softmax(q k^T / sqrt(d)) v in float64, no F16 operand rounding."""
    n_new, n_head, hd = q.shape
    G = n_head // n_head_kv
    out = np.zeros((n_new, n_head, hd))
    n_past = n_kv - n_new
    for t in range(n_new):
        for h in range(n_head):
            kv = mapping(h, G, n_head_kv)
            k = kc[: n_past + t + 1, kv].astype(np.float64)
            v = vc[: n_past + t + 1, kv].astype(np.float64)
            s = k @ q[t, h].astype(np.float64) / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ v
    return out.reshape(n_new, -1)


def causal_mask(n_kv, n_new):
    m = np.zeros((n_new, n_kv), dtype=np.float32)
    for i in range(n_new):
        m[i, n_kv - n_new + i + 1:] = -np.inf
    return m


@pytest.mark.parametrize("flash", [False, True])
def test_attention_gqa_fp64(cpu, flash):
    hd, n_head, n_head_kv, n_kv, n_new = 64, 8, 2, 50, 3
    r = rng(16)
    kc = r.standard_normal((n_kv, n_head_kv, hd)).astype(np.float16)
    vc = (r.standard_normal((n_kv, n_head_kv, hd)) + 3 * np.arange(n_head_kv)[None, :, None]).astype(np.float16)
    q = r.standard_normal((n_new, n_head, hd)).astype(np.float32)
    got = run_cpu(cpu, lambda g: attention_graph(g, hd, n_head, n_head_kv, n_kv, n_new, n_kv, kc, vc, q,
                                                 causal_mask(n_kv, n_new), flash))
    ref = attention_fp64(kc, vc, q, n_kv, n_head_kv)
    assert rel_err(got, ref) < 2e-3
    wrong = attention_fp64(kc, vc, q, n_kv, n_head_kv, mapping=lambda h, G, hkv: h % hkv)
    assert rel_err(wrong, ref) > 0.1          # the check tells the GQA mappings apart


def test_attention_special_cases(cpu):
    hd, n_head, n_head_kv = 128, 4, 2
    r = rng(17)
    # one key: the output is that key's V row for each head of the group
    kc = r.standard_normal((1, n_head_kv, hd)).astype(np.float16)
    vc = r.standard_normal((1, n_head_kv, hd)).astype(np.float16)
    q = r.standard_normal((1, n_head, hd)).astype(np.float32)
    got = run_cpu(cpu, lambda g: attention_graph(g, hd, n_head, n_head_kv, 1, 1, 1, kc, vc, q, causal_mask(1, 1)))
    assert np.array_equal(got, np.repeat(vc[0].astype(np.float32), 2, axis=0).reshape(-1))
    # identical keys: uniform weights 1/64 (exact in F16), the output is the mean of V
    n_kv = 64
    kc = np.repeat(r.standard_normal((1, n_head_kv, hd)), n_kv, axis=0).astype(np.float16)
    vc = r.standard_normal((n_kv, n_head_kv, hd)).astype(np.float16)
    got = run_cpu(cpu, lambda g: attention_graph(g, hd, n_head, n_head_kv, n_kv, 1, n_kv, kc, vc, q, causal_mask(n_kv, 1)))
    mean = vc.astype(np.float64).mean(0).astype(np.float32)
    assert np.array_equal(got, np.repeat(mean, 2, axis=0).reshape(-1))


# ---- MoE routing -----------------------------------------------------------------------------

def test_moe_route_brute_force():
    """Softmax over the experts, top-k (ties keep the lower id), weights renormalized to sum 1
    (the routing of qwen_model.c:551-606)."""
    n_expert, k = 128, 8
    for seed in range(5):
        logits = (rng(30 + seed).standard_normal(n_expert) * 2).astype(np.float32)
        if seed == 1:
            logits[[3, 40, 41]] = logits.max() + 1      # a three-way tie at the top
        ids = np.zeros(k, dtype=np.int32)
        w = np.zeros(k, dtype=np.float32)
        oracle().oracle_moe_route(ptr(logits), n_expert, k, ptr(ids), ptr(w))
        order = sorted(range(n_expert), key=lambda i: (-float(logits[i]), i))[:k]
        assert ids.tolist() == order
        e = np.exp(logits.astype(np.float64) - logits.max())
        ref = e[order] / e[order].sum()
        assert np.allclose(w, ref, rtol=1e-6, atol=0)
        assert abs(float(w.astype(np.float64).sum()) - 1.0) < 1e-6


# ---- MoE routing ops and mul_mat_id ----------------------------------------------------------

def test_argsort_is_stable_and_top_k_is_its_prefix(cpu):
    x = rng(40).integers(-3, 4, (6, 50)).astype(np.float32)     # many ties
    for order in (gl.SORT_ASC, gl.SORT_DESC):
        got = run_cpu(cpu, lambda g: g.argsort(g.tensor(gl.F32, 50, 6, data=x), order)).view(np.int32).reshape(6, 50)
        expect = np.argsort(x if order == gl.SORT_ASC else -x, axis=1, kind="stable")
        assert np.array_equal(got, expect), order


def test_sum_rows_and_div(cpu):
    x = (rng(41).standard_normal((5, 37)) * 3).astype(np.float32)
    s = run_cpu(cpu, lambda g: g.sum_rows(g.tensor(gl.F32, 37, 5, data=x)))
    assert np.array_equal(s, x.astype(np.float64).sum(1).astype(np.float32))
    d = run_cpu(cpu, lambda g: g.div(g.tensor(gl.F32, 37, 5, data=x), g.tensor(gl.F32, 1, 5, data=s)))
    assert np.array_equal(d.reshape(5, 37), x / s[:, None])


@pytest.mark.parametrize("qtype", [gl.Q4_0, gl.Q4_K])
def test_mul_mat_id_brute_force(cpu, qtype):
    """dst[:, s, t] = W[ids[s, t]] . x[:, s % x_cols, t] on the activation ggml quantizes"""
    K, N, E, k, T = 512, 48, 6, 3, 2
    W = quantize((rng(42).standard_normal((E, N, K)) * 0.05).astype(np.float32), qtype)
    Wd = dequantize(W, qtype, E * N * K).reshape(E, N, K).astype(np.float64)
    ids = np.array([[4, 0, 4], [1, 5, 2]], dtype=np.int32)          # [T][k]: repeats allowed
    for x_cols in (1, k):
        x = rng(43 + x_cols).standard_normal((T, x_cols, K)).astype(np.float32)
        got = run_cpu(cpu, lambda g: g.mul_mat_id(g.tensor(qtype, K, N, E, data=W), g.tensor(gl.F32, K, x_cols, T, data=x),
                                                   g.tensor(gl.I32, k, T, data=ids))).reshape(T, k, N)
        for t in range(T):
            for s in range(k):
                ref = Wd[ids[t, s]] @ act_dequant(x[t, s % x_cols], qtype)
                assert rel_err(got[t, s], ref) < 2e-6


def test_moe_ffn_graph_routing(cpu):
    """The graph's router picks the experts of largest probability (ties to the lower id) and
    renormalizes their weights: with a one-hot expert FFN the output exposes both."""
    n_embd, E, k, ff = 256, 8, 3, 256
    y = rng(44).standard_normal((1, n_embd)).astype(np.float32)
    router = (rng(45).standard_normal((E, n_embd)) * 0.1).astype(np.float32)
    logits = router.astype(np.float64) @ y[0].astype(np.float64)
    with Graph() as g:
        yt = g.tensor(gl.F32, n_embd, 1, data=y)
        rt = g.tensor(gl.F32, n_embd, E, data=router)
        probs = g.soft_max_ext(g.mul_mat(rt, yt), None, 1.0, 0.0)
        sel = g.argsort(probs, gl.SORT_DESC)
        p, order = g.compute(cpu, [probs, sel])
    order = order.view(np.int32)
    assert order[:k].tolist() == sorted(range(E), key=lambda i: (-logits[i], i))[:k]
    assert np.allclose(p, np.exp(logits - logits.max()) / np.exp(logits - logits.max()).sum(), rtol=1e-6)
