"""Writes the golden fixtures of tests/golden/ from the reference's own arithmetic.

The reference's scalar engine (GGML-Loader src/moe_stream: dequant.c, compute_backend.c) is built
from its sources in place by oracle/Makefile.ref into oracle/_ref/libmoe_ref.so. This script calls
that library and stores inputs and outputs as small .npz files; the tests compare the oracle (and
the product's own decoders) against them without needing the reference at run time.

    make -C oracle -f Makefile.ref && python tests/golden/make_golden.py

Fixtures:
  dequant_ref.npz   Q4_K and Q8_0 blocks -> dequant_row (dequant.c:199-251), incl. edge blocks
  kquant_ref.npz    Q5_K and Q6_K blocks -> dequant_row (dequant.c:135-197, 208-251): arbitrary
                    bytes with edge scales, and blocks of the product's quantizers
  scalar_ref.npz    sc_rmsnorm, sc_softmax, sc_swiglu, sc_rope (NEOX, tables as qwen_model.c:346-355)
                    and sc_matmul on Q4_K rows with f32 activations (compute_backend.c:14-96)

Input blocks come from numpy's seeded generator and from the product's quantizer
(ggml_quantize_chunk), so they exercise realistic as well as arbitrary bit patterns.
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libmoe_ref.so")
sys.path.insert(0, os.path.dirname(HERE))

T_F32, T_F16, T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0 = 0, 1, 12, 13, 14, 8

fp = C.POINTER(C.c_float)
MATMUL = C.CFUNCTYPE(None, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, fp, fp)
RMSNORM = C.CFUNCTYPE(None, C.c_void_p, fp, fp, fp, C.c_int, C.c_float)
ROPE = C.CFUNCTYPE(None, C.c_void_p, fp, C.c_int, fp, fp)
SOFTMAX = C.CFUNCTYPE(None, C.c_void_p, fp, C.c_int)
SWIGLU = C.CFUNCTYPE(None, C.c_void_p, fp, fp, fp, C.c_int)


class ComputeBackend(C.Structure):
    """struct compute_backend (compute_backend.h:26-63)"""
    _fields_ = [("name", C.c_char_p), ("self", C.c_void_p), ("matmul", MATMUL), ("matmul_batch", C.c_void_p),
                ("rmsnorm", RMSNORM), ("rope", ROPE), ("softmax", SOFTMAX), ("swiglu", SWIGLU),
                ("begin_batch", C.c_void_p), ("end_batch", C.c_void_p), ("sync", C.c_void_p)]


def f32p(a):
    return a.ctypes.data_as(fp)


def load_ref():
    if not os.path.exists(REF_SO):
        raise SystemExit(f"{REF_SO} missing: run `make -C oracle -f Makefile.ref`")
    lib = C.CDLL(REF_SO)
    lib.f16_to_f32.restype = C.c_float
    lib.f16_to_f32.argtypes = [C.c_uint16]
    lib.dequant_row.restype = None
    lib.dequant_row.argtypes = [C.c_uint32, C.c_void_p, fp, C.c_uint64]
    lib.compute_backend_scalar.restype = C.POINTER(ComputeBackend)
    return lib


def product_quantize(x, qtype):
    from gl import quantize
    return quantize(x, qtype, impl="product")


def fp16_bits(v):
    return np.atleast_1d(np.asarray(v, dtype=np.float16)).view(np.uint16)


def q4k_blocks(r):
    """Arbitrary Q4_K blocks: random scales/qs bytes; d, dmin of both signs, zero, subnormal and
    the largest 6-bit scales, followed by quantizer-made blocks."""
    blocks = []
    ds = [0.01, -0.02, 0.0, 6e-8, 3.0e-5, 1.0, 0.5, 1e-3]
    dmins = [0.003, 0.0, -0.01, 6e-8, 1e-4, 0.25, 0.002, 0.0]
    for d, dm in zip(ds, dmins):
        b = r.integers(0, 256, 144, dtype=np.uint8)
        b[0:2] = fp16_bits(d).view(np.uint8)
        b[2:4] = fp16_bits(dm).view(np.uint8)
        blocks.append(b)
    b = r.integers(0, 256, 144, dtype=np.uint8)
    b[4:16] = 0xFF                            # every 6-bit scale and min at 63
    blocks.append(b)
    from_quant = product_quantize((r.standard_normal(256 * 7) * 0.05).astype(np.float32), 12)
    return np.concatenate(blocks + [from_quant])


def q5k_blocks(r):
    """Arbitrary Q5_K blocks (every fifth bit pattern through random qh bytes; d, dmin of both
    signs, zero, subnormal; all 6-bit scales and mins at 63), then quantizer-made blocks."""
    blocks = []
    for d, dm in zip([0.01, -0.02, 0.0, 6e-8, 1.0, 2e-3], [0.003, 0.0, -0.01, 6e-8, 0.25, 0.0]):
        b = r.integers(0, 256, 176, dtype=np.uint8)
        b[0:2] = fp16_bits(d).view(np.uint8)
        b[2:4] = fp16_bits(dm).view(np.uint8)
        blocks.append(b)
    b = r.integers(0, 256, 176, dtype=np.uint8)
    b[4:16] = 0xFF
    b[16:48] = 0xFF                           # every fifth bit set
    blocks.append(b)
    x = (r.standard_normal(256 * 5) * 0.05).astype(np.float32)
    x[256:512] += 0.03                        # a block with an offset
    return np.concatenate(blocks + [product_quantize(x, T_Q5_K)])


def q6k_blocks(r):
    """Arbitrary Q6_K blocks (random ql/qh/scales bytes: signed scales of both signs incl. -128
    and 127; d of both signs, zero, subnormal), then quantizer-made blocks."""
    blocks = []
    for d in [0.01, -0.02, 0.0, 6e-8, 1.0, 3e-5]:
        b = r.integers(0, 256, 210, dtype=np.uint8)
        b[208:210] = fp16_bits(d).view(np.uint8)
        blocks.append(b)
    b = r.integers(0, 256, 210, dtype=np.uint8)
    b[192:208] = np.array([-128, 127] * 8, dtype=np.int8).view(np.uint8)
    b[128:192] = 0xFF                         # every code's high bits set
    b[208:210] = fp16_bits(0.125).view(np.uint8)
    blocks.append(b)
    x = (r.standard_normal(256 * 5) * 0.05).astype(np.float32)
    x[:256] *= 20                             # a block of larger range
    return np.concatenate(blocks + [product_quantize(x, T_Q6_K)])


def kquant_fixture(lib):
    r = np.random.default_rng(20261202)
    q5 = q5k_blocks(r)
    q6 = q6k_blocks(r)
    n5, n6 = q5.size // 176 * 256, q6.size // 210 * 256
    np.savez(os.path.join(HERE, "kquant_ref.npz"),
             q5k_in=q5, q5k_out=dequant(lib, T_Q5_K, q5, n5),
             q6k_in=q6, q6k_out=dequant(lib, T_Q6_K, q6, n6))


def q8_0_blocks(r):
    blocks = []
    for d in [0.01, -0.5, 0.0, 6e-8, 65504.0, 1e-4]:
        b = np.empty(34, dtype=np.uint8)
        b[0:2] = fp16_bits(d).view(np.uint8)
        b[2:] = r.integers(-128, 128, 32).astype(np.int8).view(np.uint8)
        blocks.append(b)
    b = np.empty(34, dtype=np.uint8)
    b[0:2] = fp16_bits(0.25).view(np.uint8)
    b[2:] = np.array([-128, 127] * 16, dtype=np.int8).view(np.uint8)
    blocks.append(b)
    from_quant = product_quantize((r.standard_normal(32 * 9) * 2).astype(np.float32), 8)
    return np.concatenate(blocks + [from_quant])


def dequant(lib, qtype, q, n):
    out = np.zeros(n, dtype=np.float32)
    lib.dequant_row(qtype, q.ctypes.data_as(C.c_void_p), f32p(out), n)
    return out


def main():
    lib = load_ref()
    r = np.random.default_rng(20240601)

    # f16 decode of the reference agrees with IEEE binary16 (numpy) on every non-NaN code: the oracle
    # is held to numpy exhaustively by the tests, so no table is stored.
    codes = np.arange(65536, dtype=np.uint32)
    ref16 = np.array([lib.f16_to_f32(int(h)) for h in codes], dtype=np.float32)
    ieee = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ieee)
    assert np.array_equal(np.isnan(ref16), nan)
    assert np.array_equal(ref16[~nan].view(np.uint32), ieee[~nan].view(np.uint32))

    q4k = q4k_blocks(r)
    q80 = q8_0_blocks(r)
    n4k = q4k.size // 144 * 256
    n80 = q80.size // 34 * 32
    np.savez(os.path.join(HERE, "dequant_ref.npz"),
             q4k_in=q4k, q4k_out=dequant(lib, T_Q4_K, q4k, n4k),
             q8_0_in=q80, q8_0_out=dequant(lib, T_Q8_0, q80, n80))

    be = lib.compute_backend_scalar().contents

    x = (r.standard_normal((3, 3072)) * 3).astype(np.float32)
    w = (1 + 0.01 * r.standard_normal(3072)).astype(np.float32)
    rms = np.zeros_like(x)
    for i in range(x.shape[0]):
        row, out = np.ascontiguousarray(x[i]), np.zeros(3072, dtype=np.float32)
        be.rmsnorm(None, f32p(out), f32p(row), f32p(w), 3072, C.c_float(1e-5))
        rms[i] = out

    sx = (r.standard_normal((4, 300)) * 4).astype(np.float32)
    sm = sx.copy()
    for i in range(sm.shape[0]):
        row = np.ascontiguousarray(sm[i])
        be.softmax(None, f32p(row), 300)
        sm[i] = row

    gate = (r.standard_normal(2048) * 2).astype(np.float32)
    up = r.standard_normal(2048).astype(np.float32)
    swi = np.zeros(2048, dtype=np.float32)
    be.swiglu(None, f32p(gate), f32p(up), f32p(swi), 2048)

    hd, base = 128, 1e6
    pos = np.array([0, 1, 2, 5, 13, 31], dtype=np.int32)
    rv = r.standard_normal((len(pos), hd)).astype(np.float32)
    ro = rv.copy()
    half = hd // 2
    for k, p in enumerate(pos):
        # the rope tables of qwen_model.c:346-355 (double angles, float cos/sin)
        freq = 1.0 / np.power(base, (2.0 * np.arange(half)) / hd)
        cs = np.cos(p * freq).astype(np.float32)
        sn = np.sin(p * freq).astype(np.float32)
        row = np.ascontiguousarray(ro[k])
        be.rope(None, f32p(row), hd, f32p(cs), f32p(sn))
        ro[k] = row

    K, N = 1024, 8
    W = product_quantize((r.standard_normal((N, K)) * 0.02).astype(np.float32), T_Q4_K)
    mx = r.standard_normal(K).astype(np.float32)
    my = np.zeros(N, dtype=np.float32)
    be.matmul(None, T_Q4_K, W.ctypes.data_as(C.c_void_p), 0, K, N, f32p(mx), f32p(my))

    np.savez(os.path.join(HERE, "scalar_ref.npz"),
             rms_x=x, rms_w=w, rms_eps=np.float32(1e-5), rms_out=rms,
             sm_x=sx, sm_out=sm,
             swi_gate=gate, swi_up=up, swi_out=swi,
             rope_hd=np.int32(hd), rope_base=np.float32(base), rope_pos=pos, rope_x=rv, rope_out=ro,
             mm_w=W, mm_k=np.int32(K), mm_n=np.int32(N), mm_x=mx, mm_y=my)
    kquant_fixture(lib)
    for f in ("dequant_ref.npz", "scalar_ref.npz", "kquant_ref.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
