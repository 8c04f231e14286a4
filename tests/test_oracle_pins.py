"""Pins the oracle's quantizers and its YaRN / frequency-factor RoPE branch (CPU only).

Upstream ggml is absent from the reference (an empty submodule), so ggml's
quantize_row_q4_0_ref, quantize_row_q4_K_ref (with make_qkx2_quants) and rope_yarn cannot be run
here. Each is pinned instead by what its published algorithm fixes, computed independently:

  * Q4_0: every code is x / d rounded half up in units of d (ties go to the larger code: the
    `+ 8.5f` truncation), the block's largest magnitude maps to code 0 (d = max / -8, stored as
    IEEE binary16), and a code is clipped to 15 only where x / d >= 7.5. Constructed ties decide
    the rounding mode: truncation and round-half-away-from-zero both fail them.
  * Q4_K: make_qkx2_quants' result is the lowest-weighted-error candidate among the 22 its grid
    search tries (float64 brute force); through the full quantizer, the sub-block scale and min
    codes are those of the float64 optimum under the weights av_x + |x| (63 for the largest),
    d and dmin are binary16 of max / 63, and every nibble is re-rounded under the decoded scales.
  * RoPE: all-ones frequency factors change nothing; factors divide each pair's angle (float64
    rotation); attn_factor 2 doubles the output exactly; freq_scale 1/2 at position 2p equals
    position p; with ext_factor 1 the pairs below the YaRN ramp equal the extrapolated rotation,
    the pairs above it the interpolated one, both times 1 + 0.1 ln(1 / freq_scale), and the pairs
    on the ramp the float64 blend.

Every check also runs once with a planted mistake in the oracle (oracle_set_planted) and must fail
then: truncated Q4_0 codes, make_qkx2_quants without its search, Q4_K weights of 1, the YaRN blend
reversed, frequency factors multiplying the angle.
"""
import ctypes as C
import math

import numpy as np
import pytest

from gl import dequantize, gl, oracle, ptr, quantize


def rng(seed):
    return np.random.default_rng(seed)


class planted:
    def __init__(self, bits):
        self.bits = bits

    def __enter__(self):
        oracle().oracle_set_planted(self.bits)

    def __exit__(self, *exc):
        oracle().oracle_set_planted(0)


def fails_when_planted(bits, check, *args):
    with planted(bits):
        with pytest.raises(AssertionError):
            check(*args)


# ---- Q4_0 ------------------------------------------------------------------------------------

def q4_0_fields(q):
    blk = q.reshape(-1, 18)
    d16 = blk[:, 0:2].copy().view(np.float16).reshape(-1)
    qs = blk[:, 2:]
    codes = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int64)   # elements 0-15, 16-31
    return d16, codes


def check_q4_0(x):
    """The properties ggml's quantize_row_q4_0_ref fixes, on float32 blocks x[n, 32]."""
    xb = x.reshape(-1, 32)
    d16, codes = q4_0_fields(quantize(x, gl.Q4_0, "oracle"))
    # the scale: the element of largest magnitude (the first such) over -8, rounded to binary16
    imax = np.abs(xb).argmax(1)
    mx = xb[np.arange(xb.shape[0]), imax]
    d = mx / np.float32(-8)
    assert np.array_equal(d16, d.astype(np.float16))
    live = d != 0
    # that element is code 0 (it is -8 d)
    assert np.all(codes[live, imax[live]] == 0)
    # the codes: p = x * (1/d) as the float32 product; (code - 8) - p in (-0.5, 0.5] up to the
    # float32 rounding of p + 8.5 (2^-20 at 8..16), clipped to 15 exactly where p >= 7.5
    inv = np.zeros_like(d)
    inv[live] = np.float32(1) / d[live]
    p = (xb[live] * inv[live, None]).astype(np.float64)
    c = codes[live]
    clipped = p >= 7.5
    assert np.all(c[clipped] == 15)
    off = (c - 8) - p
    assert np.all(off[~clipped] > -0.5) and np.all(off[~clipped] <= 0.5 + 2 ** -20)
    # decoded values are within half a step of x (plus the binary16 rounding of d), unless clipped
    y = dequantize(quantize(x, gl.Q4_0, "oracle"), gl.Q4_0, x.size).reshape(-1, 32)
    step = np.abs(d.astype(np.float64))
    err = np.abs(y.astype(np.float64) - xb)[live]
    bound = step[live, None] * 0.5 * (1 + 2e-6) + 8 * np.abs(d16.astype(np.float64) - d)[live, None] + 1e-30
    bound = np.broadcast_to(bound, err.shape)
    assert np.all(err[~clipped] <= bound[~clipped])
    # a zero block: every code 8, d = -0
    assert np.all(codes[~live] == 8)


def q4_0_tie_blocks():
    """Blocks whose products x / d are exactly k + 1/2 (d a power of two): ties in every code."""
    rows = []
    for d in (1.0, 0.25, -0.5, 2.0 ** -6):
        mx = -8 * d                                            # the block maximum that makes d
        ties = (np.arange(-8, 8) + 0.5) * d                    # x / d = -7.5 ... 7.5
        mids = (np.arange(-8, 7) + 0.25) * d
        row = np.concatenate([[mx], ties, mids])
        rows.append(row.astype(np.float32))
    return np.concatenate(rows)


def test_q4_0_codes_round_half_up_with_ties():
    x = q4_0_tie_blocks()
    check_q4_0(x)
    d16, codes = q4_0_fields(quantize(x, gl.Q4_0, "oracle"))
    # ties round to the larger code: x / d = k + 1/2 -> code k + 9 (15 at most); never k + 8
    expect_ties = np.minimum(np.arange(-8, 8) + 9, 15)
    for b in range(codes.shape[0]):
        assert np.array_equal(codes[b, 1:17], expect_ties), (b, codes[b, 1:17])
        assert np.array_equal(codes[b, 17:32], np.arange(-8, 7) + 8)


def test_q4_0_quantizer_random_blocks():
    r = rng(101)
    x = (r.standard_normal(32 * 4000) * r.uniform(0.001, 10, 32 * 4000)).astype(np.float32)
    x[:32] = 0
    x[32:64] = 3.0                       # all equal, positive maximum: d = -3/8, every code 0
    x[64:96] = np.float32(-1e-7)         # tiny scale (binary16 subnormal d)
    check_q4_0(x)


def test_q4_0_pins_fail_on_truncation():
    fails_when_planted(8, test_q4_0_codes_round_half_up_with_ties)
    fails_when_planted(8, check_q4_0, (rng(102).standard_normal(32 * 64)).astype(np.float32))


# ---- Q4_K: make_qkx2_quants ------------------------------------------------------------------

def nearest_int_f32(v):
    """ggml's nearest_int: round half to even of a float32 value."""
    return np.rint(v.astype(np.float32)).astype(np.int64)


def qkx2_search(x, w, nmax=15, rmin=-1.0, rdelta=0.1, nstep=20):
    """make_qkx2_quants' search (ggml's published algorithm) with float64 fits and errors.

    The first candidate splits [min(x, 0), max(x)] into nmax steps. Then nstep + 1 grid points
    rescale the codes by (rmin + rdelta * is + nmax) / (max - min), each refit by weighted least
    squares with the offset kept <= 0; a candidate with a lower weighted error replaces the best,
    and its offset becomes the `min` that the later grid points start from. The codes of a grid
    point are formed from float32 operands as the oracle forms them. Returns the best (L, scale,
    min, error), the initial candidate's error, and the smallest relative margin of any
    comparison the search made (near-ties can go either way in float32)."""
    x32 = x.astype(np.float32)
    mn = np.float32(min(x32.min(), 0))
    mx = np.float32(x32.max())
    x64, w64 = x32.astype(np.float64), w.astype(np.float64)
    if mx == mn:                                  # a flat block: every code 0, offset min(x, 0)
        return (np.zeros(x.size, np.int64), 0.0, float(mn), float(np.sum(w64 * (float(mn) - x64) ** 2))), 0.0, np.inf
    iscale = np.float32(nmax) / (mx - mn)
    L = np.clip(nearest_int_f32(iscale * (x32 - mn)), 0, nmax)
    sc = 1.0 / float(iscale)
    best = (L, sc, float(mn), float(np.sum(w64 * (sc * L + float(mn) - x64) ** 2)))
    first_err, margin = best[3], np.inf
    cur_min = mn
    for i in range(nstep + 1):
        iscale = (np.float32(rmin) + np.float32(rdelta) * np.float32(i) + np.float32(nmax)) / (mx - cur_min)
        L = np.clip(nearest_int_f32(iscale * (x32 - cur_min)), 0, nmax).astype(np.float64)
        sw, sl, sl2 = w64.sum(), np.sum(w64 * L), np.sum(w64 * L * L)
        sx, sxl = np.sum(w64 * x64), np.sum(w64 * L * x64)
        D = sw * sl2 - sl * sl
        if D <= 1e-9 * sw * sl2:
            margin = min(margin, D / (sw * sl2)) if D > 0 else margin
            if D <= 0:
                continue
        a = (sw * sxl - sx * sl) / D
        b = (sl2 * sx - sl * sxl) / D
        if b > 0:
            b = 0.0
            a = sxl / sl2
        err = float(np.sum(w64 * (a * L + b - x64) ** 2))
        if not np.array_equal(L, best[0]):     # the same codes give the same fit in any precision
            margin = min(margin, abs(err - best[3]) / max(best[3], 1e-30))
        if err < best[3]:
            best = (L.astype(np.int64), a, b, err)
            cur_min = np.float32(b)
    return best, first_err, margin


def oracle_qkx2(x, w):
    L = np.zeros(x.size, dtype=np.uint8)
    the_min = C.c_float(0)
    x32, w32 = np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w, np.float32)
    s = oracle().oracle_make_qkx2_quants(x.size, 15, ptr(x32), ptr(w32), ptr(L), C.byref(the_min), -1.0, 0.1, 20)
    return L.astype(np.int64), float(s), -float(the_min.value)


def check_qkx2(n_blocks, seed):
    r = rng(seed)
    decided = 0
    for _ in range(n_blocks):
        x = (r.standard_normal(32) * r.uniform(0.005, 2.0) + r.uniform(-0.5, 0.5) * r.uniform(0, 1)).astype(np.float32)
        av = np.float32(math.sqrt(float(np.sum(x.astype(np.float64) ** 2)) / 32))
        w = (av + np.abs(x)).astype(np.float32)
        L, s, m = oracle_qkx2(x, w)
        best, first_err, margin = qkx2_search(x, w)
        got = float(np.sum(w.astype(np.float64) * (s * L + m - x.astype(np.float64)) ** 2))
        assert got <= first_err * (1 + 1e-5) + 1e-12        # the search never ends worse than it began
        if margin > 1e-4:
            # every comparison of the search is clear of float32 rounding: the same pick
            assert np.array_equal(L, best[0])
            assert abs(s - best[1]) <= 1e-4 * abs(best[1]) + 1e-9
            # the offset is a difference of float32 sums: its error is relative to the block range
            assert abs(m - best[2]) <= 1e-4 * (abs(best[2]) + 15 * abs(s))
            assert abs(got - best[3]) <= 1e-4 * best[3] + 1e-12
            decided += 1
    assert decided >= n_blocks * 3 // 4, decided


def test_make_qkx2_quants_is_the_grid_optimum():
    check_qkx2(600, 201)


def test_make_qkx2_quants_search_matters():
    fails_when_planted(16, check_qkx2, 200, 202)


# ---- Q4_K: the full quantizer ----------------------------------------------------------------

def q4_k_fields(q):
    blk = q.reshape(-1, 144)
    d = blk[:, 0:2].copy().view(np.float16).reshape(-1)
    dmin = blk[:, 2:4].copy().view(np.float16).reshape(-1)
    s = blk[:, 4:16].astype(np.int64)
    sc = np.zeros((blk.shape[0], 8), np.int64)
    mn = np.zeros((blk.shape[0], 8), np.int64)
    for j in range(8):                                   # the 6-bit packing (dequant.c:132-141)
        if j < 4:
            sc[:, j], mn[:, j] = s[:, j] & 63, s[:, j + 4] & 63
        else:
            sc[:, j] = (s[:, j + 4] & 15) | ((s[:, j - 4] >> 6) << 4)
            mn[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    qs = blk[:, 16:].reshape(-1, 4, 32)
    L = np.concatenate([np.concatenate([qs[:, g] & 15, qs[:, g] >> 4], axis=1) for g in range(4)], axis=1)
    return d, dmin, sc, mn, L.astype(np.int64)


def check_q4_k(x):
    xb = x.reshape(-1, 256)
    d16, dmin16, sc, mn, L = q4_k_fields(quantize(x, gl.Q4_K, "oracle"))
    n = xb.shape[0]
    mismatched, compared = 0, 0
    for i in range(n):
        subs, scales, mins, clear = [], [], [], []
        for j in range(8):
            v = xb[i, 32 * j: 32 * j + 32]
            av = np.float32(math.sqrt(float(np.sum(v.astype(np.float64) ** 2)) / 32))
            w = (av + np.abs(v)).astype(np.float32)
            best, _, margin = qkx2_search(v, w)
            clear.append(margin > 1e-4)
            if v.max() == min(v.min(), 0):
                scales.append(0.0)
                mins.append(-min(float(v.min()), 0.0))
            else:
                scales.append(best[1])
                mins.append(-best[2])
        max_s, max_m = max(scales), max(mins)
        # the largest scale and min codes are 63, d and dmin are binary16 of max / 63
        if max_s > 0:
            assert sc[i].max() == 63
            if all(clear):
                assert abs(float(d16[i]) / (max_s / 63) - 1) <= 2 ** -11 + 1e-4, (i, float(d16[i]), max_s / 63)
        if max_m > 0:
            assert mn[i].max() == 63
            if all(clear):
                assert abs(float(dmin16[i]) / (max_m / 63) - 1) <= 2 ** -11 + 1e-4
        # the codes of the other sub-blocks: nearest(63 * s_j / max), away from rounding boundaries
        if all(clear):
            for j in range(8):
                for val, mx, code in ((scales[j], max_s, sc[i, j]), (mins[j], max_m, mn[i, j])):
                    if mx <= 0:
                        continue
                    t = 63 * val / mx
                    if abs(t - math.floor(t) - 0.5) > 0.02:
                        compared += 1
                        mismatched += int(code != min(round(t), 63))
        # every nibble is re-rounded under the decoded sub-block scale and min (float32 ops)
        for j in range(8):
            dj = np.float32(d16[i]) * np.float32(sc[i, j])
            if dj == 0:
                continue
            dm = np.float32(dmin16[i]) * np.float32(mn[i, j])
            v = xb[i, 32 * j: 32 * j + 32]
            expect = np.clip(np.rint((v + dm) / dj), 0, 15)
            assert np.array_equal(L[i, 32 * j: 32 * j + 32], expect), (i, j)
    assert compared > 0 and mismatched == 0, (mismatched, compared)


def q4_k_input(seed, n_super):
    r = rng(seed)
    x = (r.standard_normal(256 * n_super) * 0.02).astype(np.float32)
    # sub-blocks of very different ranges and offsets inside one super-block
    x *= np.repeat(r.uniform(0.05, 3.0, 8 * n_super), 32).astype(np.float32)
    x += np.repeat(r.uniform(-0.02, 0.02, 8 * n_super) * (r.uniform(0, 1, 8 * n_super) < 0.5), 32).astype(np.float32)
    x[:256] = 0
    x[256 + 32: 256 + 64] = 0            # one flat sub-block inside a live super-block
    return x.astype(np.float32)


def test_q4_k_quantizer_invariants():
    check_q4_k(q4_k_input(301, 96))


def test_q4_k_pins_fail_without_search_or_weights():
    x = q4_k_input(302, 48)
    fails_when_planted(16, check_q4_k, x)
    fails_when_planted(32, check_q4_k, x)


# ---- RoPE: frequency factors and the YaRN blend ----------------------------------------------

def oracle_rope(x, n_dims, mode, pos, base, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0,
                beta_fast=0.0, beta_slow=0.0, n_ctx_orig=4096, ff=None):
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros_like(x)
    f = None if ff is None else np.ascontiguousarray(ff, np.float32)
    oracle().oracle_rope(ptr(y), ptr(x), x.size, n_dims, mode, pos, base, freq_scale, ext_factor, attn_factor,
                         beta_fast, beta_slow, n_ctx_orig, None if f is None else ptr(f))
    return y


def rotate64(x, n_dims, mode, angles, scale=1.0):
    """Float64 rotation of x's pairs by the given per-pair angles (NORMAL or NEOX pairing)."""
    x = x.astype(np.float64)
    y = x.copy()
    for i, t in enumerate(angles):
        a, b = (2 * i, 2 * i + 1) if mode == gl.ROPE_NORMAL else (i, i + n_dims // 2)
        c, s = math.cos(t) * scale, math.sin(t) * scale
        y[a], y[b] = x[a] * c - x[b] * s, x[a] * s + x[b] * c
    return y


MODES = [gl.ROPE_NORMAL, gl.ROPE_NEOX]


def check_freq_factors(mode):
    n_dims, base = 96, 10000.0
    r = rng(401)
    x = r.standard_normal(n_dims).astype(np.float32)
    ones = np.ones(n_dims // 2, np.float32)
    ff = r.uniform(1.0, 8.0, n_dims // 2).astype(np.float32)
    for pos in (0, 1, 7, 61):
        plain = oracle_rope(x, n_dims, mode, pos, base)
        assert np.array_equal(oracle_rope(x, n_dims, mode, pos, base, ff=ones), plain)
        got = oracle_rope(x, n_dims, mode, pos, base, ff=ff)
        ang = [pos * base ** (-2 * i / n_dims) / float(ff[i]) for i in range(n_dims // 2)]
        ref = rotate64(x, n_dims, mode, ang)
        assert np.max(np.abs(got - ref)) <= 2e-5 * (1 + pos / 8), (pos, np.max(np.abs(got - ref)))


@pytest.mark.parametrize("mode", MODES)
def test_rope_freq_factors_divide_the_angle(mode):
    check_freq_factors(mode)


@pytest.mark.parametrize("mode", MODES)
def test_rope_attn_factor_and_freq_scale_identities(mode):
    n_dims, base = 64, 500000.0
    x = rng(402).standard_normal(n_dims).astype(np.float32)
    for pos in (3, 100, 2048):
        plain = oracle_rope(x, n_dims, mode, pos, base)
        # attn_factor scales cos and sin: a power of two scales the output exactly
        assert np.array_equal(oracle_rope(x, n_dims, mode, pos, base, attn_factor=2.0), 2 * plain)
        # without the YaRN blend, freq_scale 1/2 at position 2p is position p (exact halving)
        assert np.array_equal(oracle_rope(x, n_dims, mode, 2 * pos, base, freq_scale=0.5), plain)


def yarn_ramp_dims(n_dims, n_ctx_orig, base, beta_fast, beta_slow):
    def corr(n_rot):
        return n_dims * math.log(n_ctx_orig / (n_rot * 2 * math.pi)) / (2 * math.log(base))
    return max(0.0, math.floor(corr(beta_fast))), min(n_dims - 1.0, math.ceil(corr(beta_slow)))


def check_yarn(mode):
    n_dims, base, n_ctx_orig, s = 96, 10000.0, 4096, 0.25
    low, high = yarn_ramp_dims(n_dims, n_ctx_orig, base, 32.0, 1.0)
    assert (low, high) == (15.0, 34.0)      # the ramp lies inside the 48 pairs: all three regions
    r = rng(403)
    x = r.standard_normal(n_dims).astype(np.float32)
    mscale = 1 + 0.1 * math.log(1 / s)
    for pos in (1, 9, 40):
        got = oracle_rope(x, n_dims, mode, pos, base, freq_scale=s, ext_factor=1.0, beta_fast=32.0, beta_slow=1.0,
                          n_ctx_orig=n_ctx_orig)
        extrap = oracle_rope(x, n_dims, mode, pos, base, attn_factor=mscale)
        interp = oracle_rope(x, n_dims, mode, pos, base, freq_scale=s, attn_factor=mscale)
        angles = []
        for i in range(n_dims // 2):
            t = pos * base ** (-2 * i / n_dims)
            ramp = 1 - min(1.0, max(0.0, (i - low) / max(0.001, high - low)))
            angles.append(s * t * (1 - ramp) + t * ramp)
        ref = rotate64(x, n_dims, mode, angles, mscale)
        idx = lambda i: [2 * i, 2 * i + 1] if mode == gl.ROPE_NORMAL else [i, i + n_dims // 2]
        below = sum((idx(i) for i in range(int(low))), [])
        above = sum((idx(i) for i in range(int(high) + 1, n_dims // 2)), [])
        tol = 3e-6 * (1 + pos)
        assert np.max(np.abs(got[below] - extrap[below])) <= tol
        assert np.max(np.abs(got[above] - interp[above])) <= tol
        assert np.max(np.abs(got - ref)) <= 2e-5 * (1 + pos / 4)


@pytest.mark.parametrize("mode", MODES)
def test_rope_yarn_blend(mode):
    check_yarn(mode)


def test_rope_pins_fail_on_planted_mistakes():
    fails_when_planted(64, check_yarn, gl.ROPE_NEOX)
    fails_when_planted(128, check_freq_factors, gl.ROPE_NORMAL)


def test_rope_longrope_graph_matches_single_vector(tmp_path):
    """The graph op (op_rope with a factors tensor, as phi3's LongRoPE builds it: ext_factor 1,
    beta 32 / 1, freq_scale 1) gives the single-vector function's values on every head and
    position."""
    from gl import Graph, cpu_backend
    b = cpu_backend(4)
    try:
        hd, n_head, pos = 96, 3, [0, 5, 4095, 70000]
        x = rng(404).standard_normal((len(pos), n_head, hd)).astype(np.float32)
        ff = rng(405).uniform(1.0, 20.0, hd // 2).astype(np.float32)
        with Graph() as g:
            y = g.compute(b, g.rope_ext(g.tensor(gl.F32, hd, n_head, len(pos), data=x),
                                        g.tensor(gl.I32, len(pos), data=np.asarray(pos, np.int32)),
                                        g.tensor(gl.F32, hd // 2, data=ff),
                                        hd, gl.ROPE_NEOX, 4096, 10000.0, 1.0, 1.0, 1.1, 32.0, 1.0)).reshape(x.shape)
        for t, p in enumerate(pos):
            for h in range(n_head):
                one = oracle_rope(x[t, h], hd, gl.ROPE_NEOX, p, 10000.0, 1.0, 1.0, 1.1, 32.0, 1.0, 4096, ff)
                assert np.array_equal(y[t, h], one)
    finally:
        gl.libs()["core"].ggml_backend_free(b)
