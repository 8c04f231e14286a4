"""A float64 numpy transformer over a GGUF file: the textbook math of the reference's build_graph
(model.cpp:1296-1474) with none of ggml's operand roundings (no Q8 activation quantization, no F16
KV cache or F16 attention operands). The tests hold the oracle's whole forward_step to it, so a
wrong RoPE mode or pair layout, GQA mapping, QK-norm, bias, fused-weight split or tied head shows up
as a large error, while ggml's roundings stay within a small tolerance.

Per layer (model.cpp:1318-1467):
    h = rms_norm(x) * attn_norm
    q, k, v = W_q h (+b_q), W_k h (+b_k), W_v h (+b_v)         separate (build_qkv :1095-1106)
            = rows [0, H d), [H d, (H + Hkv) d), [(H + Hkv) d, ...) of W_qkv h   (phi3, :1087-1094)
    q, k = rms_norm_per_head(q) * q_norm, ... (qwen3 QK-norm, :1382-1387)
    q, k = rope(q, pos), rope(k, pos): NORMAL (pairs 2i, 2i+1) for llama, NEOX (i, i + d/2) otherwise
    o = W_o softmax(q k^T / sqrt(d) + causal) v, query head h reading KV head h // (H / Hkv)
    x = x + o
    h = rms_norm(x) * ffn_norm
    x = x + W_down (silu(W_gate h) * W_up h)       (phi3: gate/up = halves of W_up h, :1116-1121)
Head: logits = W_out (rms_norm(x) * output_norm), W_out = token_embd when output.weight is absent.
MoE FFN (qwen3moe; the routing of qwen_model.c:551-606 and the expert sum of :608-734):
    p = softmax(W_router h); the k experts of largest p (an earlier expert wins a tie);
    w = p_sel / sum(p_sel); x = x + sum_k w_k W_down[e_k] (silu(W_gate[e_k] h) * W_up[e_k] h)
"""
import numpy as np

from gguf_py import GGUFFile


def _dequant(raw, ttype, ne):
    from gl import dequantize
    n = int(np.prod(ne))
    if ttype == 0:
        out = raw.view(np.float32)[:n]
    elif ttype == 1:
        out = raw.view(np.float16)[:n].astype(np.float32)
    else:
        out = dequantize(np.ascontiguousarray(raw), ttype, n)
    return out.astype(np.float64).reshape(list(reversed(ne)))


class RefModel:
    def __init__(self, path, rope_mode=None, gqa=None):
        g = GGUFFile(path)
        a = g.kv["general.architecture"]
        self.arch = a
        kv = lambda k, d=None: g.kv.get(f"{a}.{k}", d)
        self.n_embd = kv("embedding_length")
        self.n_layer = kv("block_count")
        self.n_head = kv("attention.head_count")
        self.n_head_kv = kv("attention.head_count_kv")
        self.hd = kv("attention.key_length", self.n_embd // self.n_head)
        self.n_rot = kv("rope.dimension_count", self.hd)
        self.n_ff = kv("feed_forward_length")
        self.eps = kv("attention.layer_norm_rms_epsilon")
        self.base = kv("rope.freq_base", 10000.0)
        self.n_expert_used = kv("expert_used_count", 0)
        self.neox = (a != "llama") if rope_mode is None else rope_mode == "neox"
        self.gqa = gqa or (lambda h, G, hkv: h // G)
        self.w = {n: _dequant(*g.raw(n)) for n in g.tensors}
        self.k_cache = [[] for _ in range(self.n_layer)]
        self.v_cache = [[] for _ in range(self.n_layer)]

    @staticmethod
    def rms(x, w, eps):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w

    def rope(self, x, pos):
        """x [n_new, heads, d]; rotates the first n_rot dims by theta_i = pos * base^(-2i/n_rot)."""
        n_rot = self.n_rot
        half = n_rot // 2
        theta = pos[:, None] * self.base ** (-2.0 * np.arange(half) / n_rot)     # [n_new, half]
        c, s = np.cos(theta)[:, None, :], np.sin(theta)[:, None, :]
        y = x.copy()
        if self.neox:
            a, b = x[..., :half], x[..., half:n_rot]
            y[..., :half], y[..., half:n_rot] = a * c - b * s, a * s + b * c
        else:
            a, b = x[..., 0:n_rot:2], x[..., 1:n_rot:2]
            y[..., 0:n_rot:2], y[..., 1:n_rot:2] = a * c - b * s, a * s + b * c
        return y

    def moe(self, p, h):
        W = self.w
        out = np.zeros_like(h)
        for t in range(h.shape[0]):
            logits = W[p + "ffn_gate_inp.weight"] @ h[t]
            e = np.exp(logits - logits.max())
            probs = e / e.sum()
            order = sorted(range(len(probs)), key=lambda i: (-probs[i], i))
            sel = order[: self.n_expert_used]
            # relative gap between the last selected expert and the first one left out
            gap = (probs[order[self.n_expert_used - 1]] - probs[order[self.n_expert_used]]) / probs[order[self.n_expert_used - 1]]
            self.route_margin = min(self.route_margin, gap)
            wk = probs[sel] / probs[sel].sum()
            for k, ex in enumerate(sel):
                g = W[p + "ffn_gate_exps.weight"][ex] @ h[t]
                u = W[p + "ffn_up_exps.weight"][ex] @ h[t]
                out[t] += wk[k] * (W[p + "ffn_down_exps.weight"][ex] @ (g / (1 + np.exp(-g)) * u))
        return out

    def forward(self, n_past, tokens):
        """Logits of the last token; route_margin is then the smallest relative gap between the
        k-th and (k+1)-th expert probability over the step's MoE layers (inf without MoE)."""
        self.route_margin = float("inf")
        W = self.w
        H, Hkv, d = self.n_head, self.n_head_kv, self.hd
        tokens = np.asarray(tokens)
        n_new = len(tokens)
        pos = np.arange(n_past, n_past + n_new, dtype=np.float64)
        x = W["token_embd.weight"][tokens]
        for il in range(self.n_layer):
            p = f"blk.{il}."
            h = self.rms(x, W[p + "attn_norm.weight"], self.eps)
            if p + "attn_qkv.weight" in W:
                qkv = h @ W[p + "attn_qkv.weight"].T
                q, k, v = qkv[:, :H * d], qkv[:, H * d:(H + Hkv) * d], qkv[:, (H + Hkv) * d:]
            else:
                q, k, v = (h @ W[p + f"attn_{t}.weight"].T for t in "qkv")
                if p + "attn_q.bias" in W:
                    q, k, v = q + W[p + "attn_q.bias"], k + W[p + "attn_k.bias"], v + W[p + "attn_v.bias"]
            q, k, v = q.reshape(n_new, H, d), k.reshape(n_new, Hkv, d), v.reshape(n_new, Hkv, d)
            if p + "attn_q_norm.weight" in W:
                q = self.rms(q, W[p + "attn_q_norm.weight"], self.eps)
                k = self.rms(k, W[p + "attn_k_norm.weight"], self.eps)
            q, k = self.rope(q, pos), self.rope(k, pos)
            self.k_cache[il].extend(k)
            self.v_cache[il].extend(v)
            K, V = np.array(self.k_cache[il]), np.array(self.v_cache[il])   # [n_kv, Hkv, d]
            out = np.zeros((n_new, H, d))
            G = H // Hkv
            for t in range(n_new):
                n_kv = n_past + t + 1
                for hh in range(H):
                    kv = self.gqa(hh, G, Hkv)
                    s = K[:n_kv, kv] @ q[t, hh] / np.sqrt(d)
                    e = np.exp(s - s.max())
                    out[t, hh] = (e / e.sum()) @ V[:n_kv, kv]
            x = x + out.reshape(n_new, H * d) @ W[p + "attn_output.weight"].T
            h = self.rms(x, W[p + "ffn_norm.weight"], self.eps)
            if p + "ffn_gate_inp.weight" in W:
                x = x + self.moe(p, h)
                continue
            if p + "ffn_gate.weight" in W:
                gate, up = h @ W[p + "ffn_gate.weight"].T, h @ W[p + "ffn_up.weight"].T
            else:
                gu = h @ W[p + "ffn_up.weight"].T
                gate, up = gu[:, :self.n_ff], gu[:, self.n_ff:]
            act = gate / (1 + np.exp(-gate)) * up
            x = x + act @ W[p + "ffn_down.weight"].T
        x = self.rms(x, W["output_norm.weight"], self.eps)
        head = W.get("output.weight", W["token_embd.weight"])
        return (x[-1] @ head.T)
