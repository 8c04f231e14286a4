"""A seeded synthetic dory (looped normalized-GPT) GGUF and an independent float64 statement of
the dory forward pass, for the tests that run the reference's own dory graph builder on the
oracle's and the hip backend.

The file carries the metadata dory_load_hparams reads (reference src/dory.c:54-200: block counts,
widths, window, the two rope bases, the nGPT constants init_std / alpha_init / gate_init, the
per-block rope profile and layer pattern), the eos id load_hparams requires (model.cpp:200) and
the tensors dory_load_model binds (dory.c:228-331).

DoryRef restates the architecture from its documented recipe (dory.h:33-45) and the cache
contract (dory.h:47-75, dory_fill_attn_mask dory.c:553-575) in float64 numpy:
  L2(x)      x / sqrt(sum x^2 + 1e-6)
  MLP        g = Wg x * (s_g sqrt(n_embd)); u = Wu x * (s_u sqrt(n_embd)); Wd L2(silu(g) u)
  attention  q, k, v = Wq x, Wk x, Wv x per head; rope NEOX over the full head width with the
             block's base (profile 1 -> rope.freq_base, 2 -> rope.freq_base_2);
             q = L2(q) (s_qk sqrt(hd) / init_std)^2; k = L2(k); gate = sigmoid(Wgate x
             (s_gate sqrt(gate_init) / init_std)^2); attend over the block's ring with
             scale 1/sqrt(hd), query head h reading KV head h / (n_head / n_head_kv);
             Wo L2(attn * gate)
  update     a = L2(residual), b = L2(block), alpha = |s_res alpha_init / init_std|,
             L2(a + (b - a) alpha)
  schedule   input blocks; num_loops passes over the recurrent blocks, each opening with
             h = L2(h + input_state) and closing with L2; output blocks; logits = Wout h
             (output_scale / init_std)
  cache      one ring per attention block (last-loop mode: every loop writes the same ring),
             n_swa cells for 'S' blocks and n_ctx for '*' blocks, position p in cell p mod n;
             a query at position p sees a cell when the position last written there is in
             [0, p]. K and V are stored as F16, and the query is rounded to F16 before its dots,
             as the graph's F16 ring and ggml's flash attention do.
"""
import struct

import numpy as np

from gl import dequantize, gl, quantize

GGUF_U32, GGUF_F32, GGUF_STR, GGUF_ARR, GGUF_I32 = 4, 6, 8, 9, 5

BASE = dict(n_embd=256, n_ff=512, n_head=4, n_head_kv=2, head_dim=64, n_vocab=384, n_ctx_train=4096, n_swa=8,
            pattern="S-*-S-S-S-", n_input=2, n_recurrent=6, n_output=2, num_loops=2, rope_base=1e7,
            rope_base_2=1e4, init_std=0.02, alpha_init=0.05, w_std=0.05, tied=False, output_scale=True, seed=5)


def _s(v):
    b = v.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key, t, v):
    out = _s(key) + struct.pack("<I", t)
    if t == GGUF_STR:
        return out + _s(v)
    if t == GGUF_ARR:
        et, vals = v
        return out + struct.pack("<IQ", et, len(vals)) + b"".join(struct.pack("<i", x) for x in vals)
    return out + struct.pack("<I" if t == GGUF_U32 else "<f", v)


def make_weights(cfg):
    """{name: float32 array in ggml order (ne0 last)} for the configuration"""
    rng = np.random.default_rng(cfg["seed"])
    E, F, nh, nkv, hd = cfg["n_embd"], cfg["n_ff"], cfg["n_head"], cfg["n_head_kv"], cfg["head_dim"]
    std, init_std, gate_init = cfg["w_std"], cfg["init_std"], float(np.sqrt(E))

    def mat(rows, cols):                      # ggml [cols, rows]: rows of length cols
        return (rng.standard_normal((rows, cols)) * std).astype(np.float32)

    def uni(n, lo, hi):
        return rng.uniform(lo, hi, n).astype(np.float32)

    w = {"token_embd.weight": rng.standard_normal((cfg["n_vocab"], E)).astype(np.float32)}
    for il, pc in enumerate(cfg["pattern"]):
        b = f"blk.{il}."
        if pc == "-":
            w[b + "ffn_gate.weight"] = mat(F, E)
            w[b + "ffn_up.weight"] = mat(F, E)
            w[b + "ffn_down.weight"] = mat(E, F)
            w[b + "ffn_gate_scale.weight"] = uni(F, 0.5, 1.5) / (std * np.sqrt(E))
            w[b + "ffn_up_scale.weight"] = uni(F, 0.5, 1.5) / (std * np.sqrt(E))
        else:
            w[b + "attn_q.weight"] = mat(nh * hd, E)
            w[b + "attn_k.weight"] = mat(nkv * hd, E)
            w[b + "attn_v.weight"] = mat(nkv * hd, E)
            w[b + "attn_output.weight"] = mat(E, nh * hd)
            w[b + "attn_gate.weight"] = mat(nh * hd, E)
            w[b + "attn_qk_scale.weight"] = np.sqrt(uni(nh * hd, 10.0, 30.0)) * init_std / np.sqrt(hd)
            w[b + "attn_gate_scale.weight"] = np.sqrt(uni(nh * hd, 20.0, 60.0)) * init_std / np.sqrt(gate_init)
        sign = np.where(rng.random(E) < 0.5, -1.0, 1.0).astype(np.float32)
        w[b + "residual_alpha.weight"] = sign * uni(E, 0.1, 0.5) * init_std / cfg["alpha_init"]
    if not cfg["tied"]:
        w["output.weight"] = mat(cfg["n_vocab"], E)
    if cfg["output_scale"]:
        w["output_scale.weight"] = uni(cfg["n_vocab"], 2.4, 3.6) * init_std / std
    return {k: v.astype(np.float32) for k, v in w.items()}


def weight_type(name, arr, wtype):
    """matrices in wtype (the token embedding and output too), vectors F32"""
    return wtype if arr.ndim == 2 else gl.F32


def write_dory_gguf(path, cfg, wtype=gl.F32, align=32):
    """Writes the model; returns the weights as stored (quantized matrices decoded back to float)."""
    E = cfg["n_embd"]
    prof = [0 if pc == "-" else (1 if pc == "*" else 2) for pc in cfg["pattern"]]
    kvs = [_kv("general.architecture", GGUF_STR, "dory"),
           _kv("general.alignment", GGUF_U32, align),
           _kv("dory.block_count", GGUF_U32, len(cfg["pattern"])),
           _kv("dory.input_layer_count", GGUF_U32, cfg["n_input"]),
           _kv("dory.recurrent_layer_count", GGUF_U32, cfg["n_recurrent"]),
           _kv("dory.output_layer_count", GGUF_U32, cfg["n_output"]),
           _kv("dory.num_loops", GGUF_U32, cfg["num_loops"]),
           _kv("dory.embedding_length", GGUF_U32, E),
           _kv("dory.feed_forward_length", GGUF_U32, cfg["n_ff"]),
           _kv("dory.attention.head_count", GGUF_U32, cfg["n_head"]),
           _kv("dory.attention.head_count_kv", GGUF_U32, cfg["n_head_kv"]),
           _kv("dory.attention.key_length", GGUF_U32, cfg["head_dim"]),
           _kv("dory.attention.value_length", GGUF_U32, cfg["head_dim"]),
           _kv("dory.rope.dimension_count", GGUF_U32, cfg["head_dim"]),
           _kv("dory.context_length", GGUF_U32, cfg["n_ctx_train"]),
           _kv("dory.attention.sliding_window", GGUF_U32, cfg["n_swa"]),
           _kv("dory.rope.freq_base", GGUF_F32, cfg["rope_base"]),
           _kv("dory.rope.freq_base_2", GGUF_F32, cfg["rope_base_2"]),
           _kv("dory.init_std", GGUF_F32, cfg["init_std"]),
           _kv("dory.alpha_init", GGUF_F32, cfg["alpha_init"]),
           _kv("dory.gate_init", GGUF_F32, float(np.sqrt(E))),
           _kv("dory.rope.profile", GGUF_ARR, (GGUF_I32, prof)),
           _kv("dory.layer_pattern", GGUF_STR, cfg["pattern"]),
           _kv("dory.recurrent_kv_cache_mode", GGUF_STR, "last_loop"),
           _kv("tokenizer.ggml.eos_token_id", GGUF_U32, 2)]
    w = make_weights(cfg)
    stored, blobs, infos, off = {}, [], b"", 0
    for name, arr in w.items():
        t = weight_type(name, arr, wtype)
        if t == gl.F32:
            data = arr.tobytes()
            stored[name] = arr.astype(np.float64)
        else:
            data = quantize(arr, t).tobytes()
            stored[name] = dequantize(np.frombuffer(data, np.uint8), t, arr.size).reshape(arr.shape).astype(np.float64)
        ne = list(reversed(arr.shape))
        infos += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        infos += struct.pack("<IQ", t, off)
        blobs.append(data + b"\0" * ((-len(data)) % align))
        off += len(blobs[-1])
    head = b"GGUF" + struct.pack("<IQQ", 3, len(w), len(kvs)) + b"".join(kvs) + infos
    head += b"\0" * ((-len(head)) % align)
    with open(path, "wb") as f:
        f.write(head + b"".join(blobs))
    return stored


def f16(x):
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def l2(x):
    return x / np.sqrt((x * x).sum(axis=-1, keepdims=True) + 1e-6)


def rope_neox(x, pos, base):
    """x [n_tokens, heads, hd], rotated as pairs (i, i + hd/2) by pos * base^(-2i/hd)"""
    hd = x.shape[-1]
    i = np.arange(hd // 2)
    ang = np.asarray(pos, np.float64)[:, None] * base ** (-2.0 * i / hd)[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b = x[..., : hd // 2], x[..., hd // 2:]
    return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)


def rope_normal(x, pos, base):
    """the other pairing, (2i, 2i + 1): a planted mistake for the tests"""
    hd = x.shape[-1]
    i = np.arange(hd // 2)
    ang = np.asarray(pos, np.float64)[:, None] * base ** (-2.0 * i / hd)[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2], out[..., 1::2] = a * c - b * s, a * s + b * c
    return out


class DoryRef:
    """plant: names of deliberate mistakes, for the tests that show the comparison catches them:
    "rope_normal" (pairs (2i, 2i+1)), "no_window" (sliding blocks see the whole history),
    "qk_unsquared" (the q scale not squared), "no_reinjection" (loops skip h = L2(h + input)),
    "kv_head_mod" (query head h reads KV head h % n_head_kv)"""

    def __init__(self, cfg, w, n_ctx, plant=()):
        self.c, self.w, self.plant = cfg, w, set(plant)
        E = cfg["n_embd"]
        self.gate_init = float(np.sqrt(E))
        self.rings = {}
        for il, pc in enumerate(cfg["pattern"]):
            if pc != "-":
                n = min(n_ctx, cfg["n_ctx_train"]) if pc == "*" or "no_window" in self.plant else cfg["n_swa"]
                nkv, hd = cfg["n_head_kv"], cfg["head_dim"]
                self.rings[il] = dict(n=n, k=np.zeros((n, nkv, hd)), v=np.zeros((n, nkv, hd)),
                                      pos=np.full(n, -1, np.int64))

    def attn(self, il, x, pos):
        c, w = self.c, self.w
        b = f"blk.{il}."
        nh, nkv, hd = c["n_head"], c["n_head_kv"], c["head_dim"]
        T = x.shape[0]
        q = (x @ w[b + "attn_q.weight"].T).reshape(T, nh, hd)
        k = (x @ w[b + "attn_k.weight"].T).reshape(T, nkv, hd)
        v = (x @ w[b + "attn_v.weight"].T).reshape(T, nkv, hd)
        base = c["rope_base"] if c["pattern"][il] == "*" else c["rope_base_2"]
        rope = rope_normal if "rope_normal" in self.plant else rope_neox
        q, k = rope(q, pos, base), rope(k, pos, base)
        sq = (w[b + "attn_qk_scale.weight"] * np.sqrt(hd) / c["init_std"]) ** (1 if "qk_unsquared" in self.plant else 2)
        q = l2(q) * sq.reshape(nh, hd)
        k = l2(k)
        sg = (w[b + "attn_gate_scale.weight"] * np.sqrt(self.gate_init) / c["init_std"]) ** 2
        gate = 1.0 / (1.0 + np.exp(-((x @ w[b + "attn_gate.weight"].T) * sg)))
        r = self.rings[il]
        for t in range(T):
            cell = pos[t] % r["n"]
            r["k"][cell], r["v"][cell], r["pos"][cell] = f16(k[t]), f16(v[t]), pos[t]
        out = np.zeros((T, nh, hd))
        grp = nh // nkv
        for t in range(T):
            vis = (r["pos"] >= 0) & (r["pos"] <= pos[t])
            for h in range(nh):
                kvh = h % nkv if "kv_head_mod" in self.plant else h // grp
                kk, vv = r["k"][vis, kvh], r["v"][vis, kvh]
                s = kk @ f16(q[t, h]) / np.sqrt(hd)
                p = np.exp(s - s.max())
                out[t, h] = (p / p.sum()) @ vv
        o = l2(out.reshape(T, nh * hd) * gate)
        return o @ w[b + "attn_output.weight"].T

    def ffn(self, il, x):
        c, w = self.c, self.w
        b = f"blk.{il}."
        f = np.sqrt(c["n_embd"])
        g = (x @ w[b + "ffn_gate.weight"].T) * (w[b + "ffn_gate_scale.weight"] * f)
        u = (x @ w[b + "ffn_up.weight"].T) * (w[b + "ffn_up_scale.weight"] * f)
        return l2(g / (1.0 + np.exp(-g)) * u) @ w[b + "ffn_down.weight"].T

    def block(self, il, x, pos):
        c, w = self.c, self.w
        y = self.ffn(il, x) if c["pattern"][il] == "-" else self.attn(il, x, pos)
        a, b = l2(x), l2(y)
        alpha = np.abs(w[f"blk.{il}.residual_alpha.weight"] * c["alpha_init"] / c["init_std"])
        return l2(a + (b - a) * alpha)

    def forward(self, pos0, tokens):
        """logits [n_tokens, n_vocab] for one forward call at positions pos0 .. pos0 + n - 1"""
        c, w = self.c, self.w
        pos = np.arange(pos0, pos0 + len(tokens))
        x = w["token_embd.weight"][np.asarray(tokens)]
        n_in, n_rec = c["n_input"], c["n_recurrent"]
        for il in range(n_in):
            x = self.block(il, x, pos)
        inp = x
        for _ in range(c["num_loops"]):
            for il in range(n_in, n_in + n_rec):
                if il == n_in and "no_reinjection" not in self.plant:
                    x = l2(x + inp)
                x = self.block(il, x, pos)
            x = l2(x)
        for il in range(n_in + n_rec, len(c["pattern"])):
            x = self.block(il, x, pos)
        logits = x @ w.get("output.weight", w["token_embd.weight"]).T
        if "output_scale.weight" in w:
            logits = logits * (w["output_scale.weight"] / c["init_std"])
        return logits
