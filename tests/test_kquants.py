"""Q5_K and Q6_K weights (the K-quant types of the reference's real checkpoints: Q4_K_M and its
UD-Q4_K_XL MoE file mix them with Q4_K), CPU tier.

  * decode: the oracle's and the product's decoders equal the reference's own dequant_row
    (src/moe_stream/dequant.c:135-197, 208-251) bit for bit on the fixture tests/golden/kquant_ref.npz
    (arbitrary block bytes with edge scales, and quantizer-made blocks);
  * quantizers (ggml's quantize_row_q5_K_ref / q6_K_ref, restated; upstream ggml is absent):
    - Q5_K: its make_qkx2_quants search (5-bit codes, 16 rescalings from -0.5) against a float64
      statement; the codes re-rounded under the decoded sub-block scales and mins; 63 for the
      largest scale and min codes;
    - Q6_K: make_qx_quants against a float64 statement of its search (codes -32..31, weights x^2,
      18 rescalings); d = binary16(max_scale / -128) of the largest-magnitude sub-block scale; the
      signed scale codes; the codes re-rounded under the decoded scales;
    - a planted mistake (make_qx_quants without its search) fails;
    - the product's quantizers equal the oracle's byte for byte;
  * dots: ggml's generic q5_K x q8_K and q6_K x q8_K kernels against float64 brute force over the
    same quantized operands, and the oracle backend's mul_mat / mul_mat_id over them.
"""
import ctypes as C
import math
import os

import numpy as np
import pytest

from gl import GOLDEN, Graph, cpu_backend, dequantize, gl, oracle, ptr, quantize
from test_oracle_pins import fails_when_planted, oracle_qkx2, qkx2_search

KQ = [gl.Q5_K, gl.Q6_K]
BYTES = {gl.Q5_K: 176, gl.Q6_K: 210}


def rng(seed):
    return np.random.default_rng(seed)


@pytest.fixture(scope="module")
def cpu():
    b = cpu_backend(8)
    yield b
    gl.libs()["core"].ggml_backend_free(b)


# ---- decode ----------------------------------------------------------------------------------

@pytest.mark.parametrize("qtype,key", [(gl.Q5_K, "q5k"), (gl.Q6_K, "q6k")])
@pytest.mark.parametrize("impl", ["oracle", "product"])
def test_decode_matches_reference_golden(qtype, key, impl):
    z = np.load(os.path.join(GOLDEN, "kquant_ref.npz"), allow_pickle=False)
    q, ref = z[f"{key}_in"], z[f"{key}_out"]
    got = dequantize(q, qtype, ref.size, impl)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_decode_golden_discriminates():
    """A decoder with Q6_K's two high bits taken from the wrong pair differs from the fixture."""
    z = np.load(os.path.join(GOLDEN, "kquant_ref.npz"), allow_pickle=False)
    q = z["q6k_in"].copy().reshape(-1, 210)
    q[:, 128:192] = ((q[:, 128:192] >> 2) | (q[:, 128:192] << 6)).astype(np.uint8)   # rotate the bit pairs
    got = dequantize(q.reshape(-1), gl.Q6_K, z["q6k_out"].size)
    assert not np.array_equal(got, z["q6k_out"])


# ---- quantizers ------------------------------------------------------------------------------

def kq_input(seed, n_super, scale=0.02):
    r = rng(seed)
    x = (r.standard_normal(256 * n_super) * scale).astype(np.float32)
    x *= np.repeat(r.uniform(0.05, 3.0, 16 * n_super), 16).astype(np.float32)
    x += np.repeat(r.uniform(-0.02, 0.02, 8 * n_super) * (r.uniform(0, 1, 8 * n_super) < 0.5), 32).astype(np.float32)
    x[:256] = 0                     # an all-zero super-block
    x[256 + 32: 256 + 64] = 0       # a flat sub-block in a live one
    x[512:768] = 0.125              # a constant super-block
    return x.astype(np.float32)


@pytest.mark.parametrize("qtype", KQ)
def test_product_quantizer_matches_oracle(qtype):
    x = kq_input(501, 40)
    assert np.array_equal(quantize(x, qtype, "oracle"), quantize(x, qtype, "product"))


def q5k_fields(q):
    from test_oracle_pins import q4_k_fields
    blk = q.reshape(-1, 176)
    as_q4k = np.concatenate([blk[:, :16], blk[:, 48:176]], axis=1).reshape(-1)   # header + low nibbles
    d, dmin, sc, mn, L = q4_k_fields(as_q4k)
    qh = blk[:, 16:48].astype(np.int64)
    hi = np.stack([(qh >> j) & 1 for j in range(8)], axis=1)   # [block][sub-block][l]
    return d, dmin, sc, mn, L + 16 * hi.reshape(-1, 256)


def test_q5_k_search_is_the_grid_optimum():
    r = rng(502)
    decided = 0
    for _ in range(300):
        x = (r.standard_normal(32) * r.uniform(0.005, 2.0) + r.uniform(-0.5, 0.5) * r.uniform(0, 1)).astype(np.float32)
        av = np.float32(math.sqrt(float(np.sum(x.astype(np.float64) ** 2)) / 32))
        w = (av + np.abs(x)).astype(np.float32)
        L = np.zeros(32, np.uint8)
        mn = C.c_float(0)
        s = oracle().oracle_make_qkx2_quants(32, 31, ptr(x), ptr(w), ptr(L), C.byref(mn), -0.5, 0.1, 15)
        best, first, margin = qkx2_search(x, w, nmax=31, rmin=-0.5, rdelta=0.1, nstep=15)
        if margin > 1e-4:
            assert np.array_equal(L.astype(np.int64), best[0])
            assert abs(s - best[1]) <= 1e-4 * abs(best[1]) + 1e-9
            decided += 1
    assert decided >= 200


def test_q5_k_quantizer_invariants():
    x = kq_input(503, 48)
    q = quantize(x, gl.Q5_K, "oracle")
    d16, dmin16, sc, mn, L = q5k_fields(q)
    xb = x.reshape(-1, 256)
    for i in range(xb.shape[0]):
        if sc[i].max() > 0:
            assert sc[i].max() == 63
        if mn[i].max() > 0:
            assert mn[i].max() == 63
        for j in range(8):
            dj = np.float32(d16[i]) * np.float32(sc[i, j])
            if dj == 0:
                continue
            dm = np.float32(dmin16[i]) * np.float32(mn[i, j])
            v = xb[i, 32 * j: 32 * j + 32]
            assert np.array_equal(L[i, 32 * j: 32 * j + 32], np.clip(np.rint((v + dm) / dj), 0, 31)), (i, j)
    # 5-bit codes reach the top of their range somewhere (the fifth bit is used)
    assert L.max() == 31 and (L >= 16).mean() > 0.05
    y = dequantize(q, gl.Q5_K, x.size)
    rms = np.sqrt(np.mean((y[768:] - x[768:]) ** 2)) / np.std(x[768:])
    assert rms < 0.06, rms


def qx_candidates(x, nmax=32):
    """The 19 grid points of make_qx_quants (rmse_type 1): codes -nmax..nmax-1 of (nmax + 0.1 is) /
    max (is = 0, then -9..9 without 0) formed from float32 operands, each with its float64
    objective sum(w x l)^2 / sum(w l^2), w = x^2, and least-squares scale sum(w x l) / sum(w l^2)."""
    x32 = x.astype(np.float32)
    mx = x32[int(np.argmax(np.abs(x32)))]
    x64 = x32.astype(np.float64)
    w = x64 * x64
    out = []
    for k in [0] + [k for k in range(-9, 10) if k != 0]:
        iscale = (np.float32(-nmax) if k == 0 else -(np.float32(nmax) + np.float32(0.1) * np.float32(k))) / mx
        l = np.clip(np.rint((iscale * x32).astype(np.float32)), -nmax, nmax - 1).astype(np.int64)
        sxl, sl2 = float(np.sum(w * x64 * l)), float(np.sum(w * l * l))
        if sl2 > 0:
            out.append((l + nmax, sxl * sxl / sl2, sxl / sl2))
    return out


def check_qx(n_blocks, seed):
    """The search's pick is one of its grid points, within 1e-5 of the best objective (float32
    arithmetic decides near-ties), with that point's least-squares scale."""
    r = rng(seed)
    searched = 0
    for _ in range(n_blocks):
        x = (r.standard_normal(16) * r.uniform(0.01, 2.0)).astype(np.float32)
        L = np.zeros(16, np.int8)
        s = oracle().oracle_make_qx_quants(16, 32, ptr(x), ptr(L))
        cands = qx_candidates(x)
        best = max(c[1] for c in cands)
        mine = [c for c in cands if np.array_equal(c[0], L.astype(np.int64))]
        assert mine, "codes of no grid point"
        assert mine[0][1] >= best * (1 - 1e-5)
        assert abs(s - mine[0][2]) <= 1e-5 * abs(mine[0][2])
        searched += cands[0][1] < best * (1 - 1e-5)      # the first point alone would fail the check
    assert searched >= n_blocks // 5, searched


def test_q6_k_make_qx_quants_is_the_search_optimum():
    check_qx(600, 504)


def test_q6_k_search_matters():
    fails_when_planted(256, check_qx, 300, 505)


def q6k_fields(q):
    blk = q.reshape(-1, 210)
    ql, qh = blk[:, :128].astype(np.int64), blk[:, 128:192].astype(np.int64)
    sc = blk[:, 192:208].copy().view(np.int8).astype(np.int64)
    d = blk[:, 208:210].copy().view(np.float16).reshape(-1)
    L = np.zeros((blk.shape[0], 256), np.int64)
    for h in range(2):
        for g in range(4):
            lo = (ql[:, 64 * h + 32 * (g & 1): 64 * h + 32 * (g & 1) + 32] >> (4 * (g >> 1))) & 15
            hi = (qh[:, 32 * h: 32 * h + 32] >> (2 * g)) & 3
            L[:, 128 * h + 32 * g: 128 * h + 32 * g + 32] = lo | (hi << 4)
    return d, sc, L


def test_q6_k_quantizer_invariants():
    x = kq_input(506, 48)
    q = quantize(x, gl.Q6_K, "oracle")
    d16, sc, L = q6k_fields(q)
    xb = x.reshape(-1, 256)
    compared = 0
    for i in range(xb.shape[0]):
        scales = []
        for j in range(16):
            v = xb[i, 16 * j: 16 * j + 16]
            Lq = np.zeros(16, np.int8)
            scales.append(oracle().oracle_make_qx_quants(16, 32, ptr(np.ascontiguousarray(v)), ptr(Lq)))
        scales = np.array(scales, np.float32)
        k = int(np.argmax(np.abs(scales)))
        if abs(scales[k]) < 1e-15:
            assert float(d16[i]) == 0 and np.all(sc[i] == 0)
            continue
        iscale = np.float32(-128) / scales[k]
        # d = binary16(1 / iscale); the largest-magnitude scale is code -128 (or 127 at the clip)
        assert d16[i] == (np.float32(1) / iscale).astype(np.float16)
        expect = np.minimum(127, np.rint((iscale * scales).astype(np.float32))).astype(np.int64)
        assert np.array_equal(sc[i], expect)
        for j in range(16):
            dj = np.float32(d16[i]) * np.float32(sc[i, j])
            if dj == 0:
                continue
            v = xb[i, 16 * j: 16 * j + 16]
            assert np.array_equal(L[i, 16 * j: 16 * j + 16], np.clip(np.rint(v / dj), -32, 31) + 32), (i, j)
            compared += 1
    assert compared > 500
    y = dequantize(q, gl.Q6_K, x.size)
    live = slice(768, None)
    assert np.sqrt(np.mean((y[live] - x[live]) ** 2)) / np.std(x[live]) < 0.03


# ---- dots ------------------------------------------------------------------------------------

def q8k(x):
    q = np.zeros(x.size // 256 * 292, dtype=np.uint8)
    oracle().oracle_quantize_q8_K(ptr(x), ptr(q), x.size)
    blk = q.reshape(-1, 292)
    d = blk[:, 0:4].copy().view(np.float32).reshape(-1, 1).astype(np.float64)
    qs = blk[:, 4:260].copy().view(np.int8).astype(np.float64)
    return q, (d * qs).reshape(-1)


@pytest.mark.parametrize("qtype", KQ)
@pytest.mark.parametrize("n", [256, 2560, 9728])
def test_vec_dot_brute_force(qtype, n):
    w = quantize((rng(n + qtype).standard_normal(n) * 0.1).astype(np.float32), qtype)
    x = (rng(n + 7).standard_normal(n) * 2).astype(np.float32)
    xq, xd = q8k(x)
    fn = {gl.Q5_K: "oracle_vec_dot_q5_K_q8_K", gl.Q6_K: "oracle_vec_dot_q6_K_q8_K"}[qtype]
    got = getattr(oracle(), fn)(n, ptr(w), ptr(xq))
    wd = dequantize(w, qtype, n).astype(np.float64)
    ref = float(wd @ xd)
    assert abs(got - ref) <= 2e-6 * float(np.sum(np.abs(wd) * np.abs(xd))) + 1e-12


@pytest.mark.parametrize("qtype", KQ)
def test_mul_mat_and_mul_mat_id_brute_force(cpu, qtype):
    K, N, E, T = 512, 24, 4, 3
    W = quantize((rng(qtype).standard_normal((E, N, K)) * 0.05).astype(np.float32), qtype)
    Wd = dequantize(W, qtype, E * N * K).reshape(E, N, K).astype(np.float64)
    x = rng(qtype + 1).standard_normal((T, K)).astype(np.float32)
    ids = np.array([[2, 0], [3, 3], [1, 2]], dtype=np.int32)
    with Graph() as g:
        w2 = g.tensor(qtype, K, N, data=W[: N * K // 256 * BYTES[qtype]])
        y = g.compute(cpu, g.mul_mat(w2, g.tensor(gl.F32, K, T, data=x))).reshape(T, N)
    xd = np.stack([q8k(np.ascontiguousarray(x[t]))[1] for t in range(T)])
    ref = xd @ Wd[0].T
    assert np.max(np.abs(y - ref)) <= 2e-6 * np.max(np.abs(xd) @ np.abs(Wd[0]).T) + 1e-9
    with Graph() as g:
        ws = g.tensor(qtype, K, N, E, data=W)
        xt = g.tensor(gl.F32, K, 1, T, data=x)
        it = g.tensor(gl.I32, 2, T, data=ids)
        yid = g.compute(cpu, g.mul_mat_id(ws, xt, it)).reshape(T, 2, N)
    for t in range(T):
        for s in range(2):
            r = Wd[ids[t, s]] @ xd[t]
            assert np.max(np.abs(yid[t, s] - r)) <= 2e-6 * float(np.max(np.abs(Wd[ids[t, s]]) @ np.abs(xd[t]))) + 1e-9
