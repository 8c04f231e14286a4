"""Device token sampling (ggml_backend_hip_sample, gl_generate) against the oracle's sampler
(oracle_sample, pinned on the reference's own sample() in test_sampler.py) for identical uniform
variates: the same token id and the same report of whether the variate was used, on every call.

Cases cover both device paths: the one-launch path (top-k up to 1024 from the thread-maxima bound,
rows up to 4096 sorted whole) and the sorted path (larger top-k, top-k 0, more than 1024 distinct
penalized ids, and rows whose candidates overflow, e.g. all logits equal). Rows hold exact ties,
-inf and NaN entries (NaN orders and weighs as -inf; argmax keeps a leading NaN's index 0). Then
whole sampled generations (gl_generate, the cmd_run loop) must reproduce the oracle-driven loop's
token sequence: the logits are the oracle's bit for bit, so every sampled id must be too.
"""
import os
import tempfile

import numpy as np
import pytest

from gl import Draws, Graph, cpu_backend, gl, oracle_sample, ptr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    b = gl.hip_backend(0)
    yield b
    gl.libs()["core"].ggml_backend_free(b)


class DeviceRows:
    """rows (nrows x n float32) in an F32 tensor [n, nrows] of the backend's buffer"""

    def __init__(self, backend, rows):
        rows = np.ascontiguousarray(rows, dtype=np.float32)
        self.g = Graph(mem=1 << 20)
        self.t = self.g.tensor(gl.F32, rows.shape[1], rows.shape[0])
        core = self.g.core
        self.g.buf = core.ggml_backend_alloc_ctx_tensors(self.g.ctx, backend)
        core.ggml_backend_tensor_set(self.t, ptr(rows), 0, rows.nbytes)

    def close(self):
        self.g.close()


def kinds(rng, n):
    tie_free = rng.permutation(np.unique((rng.standard_normal(n * 2 + 16) * 3).astype(np.float32)))[:n]
    ties = (np.round(rng.standard_normal(n) * 8) / 4).astype(np.float32)
    masked = tie_free.copy()
    masked[rng.random(n) < 0.1] = -np.inf
    nan = ties.copy()
    nan[rng.random(n) < 0.05] = np.nan
    if n > 1:
        nan[1] = np.nan
    peaked = (rng.standard_normal(n) * 0.5).astype(np.float32)
    peaked[rng.integers(0, n)] = 30.0
    flat = np.full(n, 0.75, np.float32)
    return dict(tie_free=tie_free, ties=ties, masked=masked, nan=nan, peaked=peaked, flat=flat)


PARAMS = [
    dict(temp=0.0),
    dict(temp=0.0, repeat_penalty=1.3),
    dict(temp=0.8),
    dict(temp=1.0, top_k=1),
    dict(temp=1.5, top_k=1024, top_p=1.0),
    dict(temp=0.7, top_k=40, top_p=0.3, repeat_penalty=1.2),
    dict(temp=1.2, top_k=2000, top_p=0.99, repeat_penalty=0.8, repeat_last_n=-1),
    dict(temp=1.0, top_k=0, top_p=1.0),
    dict(temp=3.0, top_k=0, top_p=0.9),
]


def check(backend, dr, rows, row, recent, u, params, what):
    dev = gl.hip_sample(backend, dr.t, row, recent, u, **params)
    ora = oracle_sample(rows[row], recent, u, **params)
    assert dev == ora, (what, params, u, dev, ora)
    return dev


@pytest.mark.parametrize("n", [7, 4096, 32064, 151936])
def test_sample_matches_oracle(hip, n):
    rng = np.random.default_rng(n)
    ks = kinds(rng, n)
    names = list(ks)
    rows = np.stack([ks[k] for k in names])
    recent = np.concatenate([rng.integers(0, n, 96), rng.integers(0, min(n, 8), 32), [-5, n + 3]]).astype(np.int32)
    dr = DeviceRows(hip, rows)
    calls = paths = 0
    try:
        for r, name in enumerate(names):
            for params in PARAMS:
                for u in (float(rng.random()), 0.0, float(np.nextafter(1.0, 0.0))):
                    check(hip, dr, rows, r, recent, u, params, (n, name))
                    calls += 1
                paths += 1
    finally:
        dr.close()
    print(f"n={n}: {calls} calls over {paths} (row kind, parameter) pairs, all equal to the oracle", flush=True)


def test_many_penalized_ids_take_the_sorted_path(hip):
    rng = np.random.default_rng(5)
    n = 50000
    x = rng.permutation(np.unique((rng.standard_normal(n * 2) * 2).astype(np.float32)))[:n]
    rows = x[None, :]
    recent = rng.permutation(np.repeat(np.arange(3000, dtype=np.int32), 2))    # 3000 distinct ids, twice each
    dr = DeviceRows(hip, rows)
    try:
        for params in (dict(temp=0.0, repeat_penalty=1.5, repeat_last_n=-1),
                       dict(temp=0.9, repeat_penalty=1.5, repeat_last_n=-1),
                       dict(temp=0.9, top_k=0, repeat_penalty=0.5, repeat_last_n=4000)):
            for u in (0.1, 0.5, 0.93):
                check(hip, dr, rows, 0, recent, u, params, "3000 penalized ids")
    finally:
        dr.close()


def test_rejects_bad_requests(hip):
    core = gl.libs()["core"]
    g = Graph(mem=1 << 20)
    try:
        t16 = g.tensor(gl.F16, 64, 2)
        t32 = g.tensor(gl.F32, 64, 2)
        g.buf = core.ggml_backend_alloc_ctx_tensors(g.ctx, hip)
        for t, row in ((t16, 0), (t32, 2), (t32, -1)):
            with pytest.raises(RuntimeError):
                gl.hip_sample(hip, t, row, [], 0.5, temp=1.0)
        inf = np.full((2, 64), -np.inf, np.float32)
        core.ggml_backend_tensor_set(t32, ptr(inf), 0, inf.nbytes)
        with pytest.raises(RuntimeError):
            gl.hip_sample(hip, t32, 1, [], 0.5, temp=1.0)          # no finite maximum
        assert gl.hip_sample(hip, t32, 1, [], 0.5, temp=0.0) == (0, False)
    finally:
        g.close()


def oracle_generate(c, n_past, prompt, n_steps, seed, **params):
    """cmd_run's loop (cmd_run.cpp:503-510, 576-620) on the oracle backend with oracle_sample"""
    d, all_tokens, out = Draws(seed), list(prompt), []

    def pick(logits):
        tok, used = oracle_sample(logits, all_tokens, d.peek(), **params)
        if used:
            d.consume()
        return tok

    tok = pick(c.forward(n_past, prompt))
    out.append(tok)
    pos = n_past + len(prompt)
    for _ in range(1, n_steps):
        all_tokens.append(tok)
        tok = pick(c.forward(pos, [tok]))
        pos += 1
        out.append(tok)
    return np.array(out, dtype=np.int32)


def test_generate_matches_oracle_loop():
    gl.libs()["core"].ggml_backend_free(cpu_backend(1))
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "tiny.gguf")
        gl.synth_model(path, arch="llama", n_embd=256, n_layer=2, n_head=4, n_head_kv=2, head_dim=64, n_ff=512,
                       n_vocab=5000, rope_theta=500000.0, wtype=gl.Q4_0, seed=21)
        prompt = [1, 17, 300, 4999, 42, 42]
        n_steps = 24
        for i, params in enumerate((dict(temp=0.8, top_k=40, top_p=0.95, repeat_penalty=1.1),
                                    dict(temp=1.3, top_k=0, top_p=1.0),
                                    dict(temp=0.0, repeat_penalty=1.3, repeat_last_n=8),
                                    dict(temp=2.0, top_k=3000, top_p=0.8, repeat_penalty=0.9, repeat_last_n=-1))):
            seed = 100 + i
            with gl.Session(path, "cpu", n_ctx=64, n_threads=8) as c:
                c.kv_fill_random(3, seed=5)
                want = oracle_generate(c, 3, prompt, n_steps, seed, **params)
            with gl.Session(path, "hip", n_ctx=64) as h:
                h.kv_fill_random(3, seed=5)
                got, _ = h.generate(3, prompt, n_steps, seed=seed, **params)
            print(f"{params}: {len(set(want.tolist()))} distinct tokens, equal: {np.array_equal(got, want)}", flush=True)
            assert np.array_equal(got, want), (params, got, want)
