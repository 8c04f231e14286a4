// synth.cpp — seeded synthetic GGUF models for the benchmark configurations.
//
// Tensor names, shapes and metadata keys are the ones load_hparams/load_model read (reference
// model.cpp:74-206, 534-665). Values: every tensor has its own stream keyed by (seed, name);
// element e of the stream is the normal variate z(e) from a counter-based splitmix64 ->
// Box-Muller (double) generator, so any row can be produced independently and the bytes do not
// depend on the thread count. Weights are quantized with ggml's reference quantizers
// (ggml_quantize_chunk). The file is streamed: metadata first, then tensors chunk by chunk.
#include "ggml-loader.h"
#include "gguf.h"

#include <omp.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

namespace {

inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

inline uint64_t name_hash(const std::string & s) {
    uint64_t h = 1469598103934665603ull; // FNV-1a
    for (unsigned char c : s) { h ^= c; h *= 1099511628211ull; }
    return h;
}

// normal variate number e of the stream `key`
inline double normal_at(uint64_t key, int64_t e) {
    const uint64_t pair = (uint64_t) e >> 1;
    const uint64_t a = splitmix64(key + 2 * pair);
    const uint64_t b = splitmix64(key + 2 * pair + 1);
    const double u1 = ((double) (a >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    const double u2 = (double) (b >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1));
    const double t = 6.283185307179586 * u2;
    return (e & 1) ? r * sin(t) : r * cos(t);
}

struct tensor_spec {
    std::string name;
    ggml_type type;
    int n_dims;
    int64_t ne[4];
    float mean, std;
};

} // namespace

extern "C" void gl_fill_normal(float * out, int64_t n, uint64_t seed, int64_t first, float mean, float std) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = (float) (mean + std * normal_at(seed, first + i));
}

extern "C" int gl_synth_model(const char * path, const gl_synth_params * p, char * err, size_t err_size) {
    auto fail = [&](const std::string & m) { if (err && err_size) snprintf(err, err_size, "%s", m.c_str()); return 1; };
    const std::string arch = p->arch ? p->arch : "";
    const bool phi3 = arch == "phi3", qwen2 = arch == "qwen2", qwen3 = arch == "qwen3", llama = arch == "llama";
    const bool moe = arch == "qwen3moe";
    if (!(phi3 || qwen2 || qwen3 || llama || moe)) return fail("synth: unsupported arch '" + arch + "'");
    const int64_t E = p->n_embd, hd = p->head_dim, nh = p->n_head, nkv = p->n_head_kv, ff = p->n_ff, V = p->n_vocab;
    if (E <= 0 || hd <= 0 || nh <= 0 || nkv <= 0 || V <= 0 || p->n_layer <= 0) return fail("synth: bad shape");
    const ggml_type wt = (ggml_type) p->wtype;
    if (p->kquant_mix && wt != GGML_TYPE_Q4_K) return fail("synth: kquant_mix needs wtype Q4_K");
    // the matrix type of a layer's tensor under kquant_mix (role: 'v' attn_v / ffn_down, 'q' attn_q /
    // ffn_gate / ffn_up, anything else keeps wtype)
    auto mix = [&](int64_t il, char role) {
        if (!p->kquant_mix) return wt;
        if (role == 'v' && il % 2 == 0) return GGML_TYPE_Q6_K;
        if (role == 'q' && il % 2 == 1) return GGML_TYPE_Q5_K;
        return wt;
    };
    auto fits = [&](ggml_type t, int64_t k) { return ggml_type_size(t) > 0 && k % ggml_blck_size(t) == 0; };

    std::vector<tensor_spec> specs;
    auto add = [&](const std::string & name, ggml_type t, std::initializer_list<int64_t> ne, float mean, float std) {
        tensor_spec s{ name, t, (int) ne.size(), { 1, 1, 1, 1 }, mean, std };
        int i = 0;
        for (int64_t v : ne) s.ne[i++] = v;
        specs.push_back(s);
    };
    const float ws = p->w_std, ns = p->norm_std;
    add("token_embd.weight", (ggml_type) p->embd_type, { E, V }, 0.0f, ws);
    add("output_norm.weight", GGML_TYPE_F32, { E }, 1.0f, ns);
    if (p->rope_scaling_orig_ctx > 0) {
        if (!phi3) return fail("synth: LongRoPE keys are written for phi3 only");
        add("rope_factors_short.weight", GGML_TYPE_F32, { hd / 2 }, 2.0f, 0.25f);
    }
    if (!p->tied_output) add("output.weight", p->kquant_mix ? GGML_TYPE_Q6_K : (ggml_type) p->output_type, { E, V }, 0.0f, ws);
    for (int64_t il = 0; il < p->n_layer; il++) {
        const std::string b = "blk." + std::to_string(il) + ".";
        add(b + "attn_norm.weight", GGML_TYPE_F32, { E }, 1.0f, ns);
        if (phi3) {
            add(b + "attn_qkv.weight", wt, { E, (nh + 2 * nkv) * hd }, 0.0f, ws);
        } else {
            add(b + "attn_q.weight", mix(il, 'q'), { E, nh * hd }, 0.0f, ws);
            add(b + "attn_k.weight", wt, { E, nkv * hd }, 0.0f, ws);
            add(b + "attn_v.weight", mix(il, 'v'), { E, nkv * hd }, 0.0f, ws);
            if (qwen2) {
                add(b + "attn_q.bias", GGML_TYPE_F32, { nh * hd }, 0.0f, ws);
                add(b + "attn_k.bias", GGML_TYPE_F32, { nkv * hd }, 0.0f, ws);
                add(b + "attn_v.bias", GGML_TYPE_F32, { nkv * hd }, 0.0f, ws);
            }
            if (qwen3 || moe) {
                add(b + "attn_q_norm.weight", GGML_TYPE_F32, { hd }, 1.0f, ns);
                add(b + "attn_k_norm.weight", GGML_TYPE_F32, { hd }, 1.0f, ns);
            }
        }
        add(b + "attn_output.weight", wt, { nh * hd, E }, 0.0f, ws);
        add(b + "ffn_norm.weight", GGML_TYPE_F32, { E }, 1.0f, ns);
        if (moe) {
            const int64_t ne_ = p->n_expert, fe = p->n_ff_exp;
            add(b + "ffn_gate_inp.weight", GGML_TYPE_F32, { E, ne_ }, 0.0f, ws);
            add(b + "ffn_gate_exps.weight", mix(il, 'q'), { E, fe, ne_ }, 0.0f, ws);
            add(b + "ffn_up_exps.weight", mix(il, 'q'), { E, fe, ne_ }, 0.0f, ws);
            add(b + "ffn_down_exps.weight", mix(il, 'v'), { fe, E, ne_ }, 0.0f, ws);
        } else if (phi3) {
            add(b + "ffn_up.weight", wt, { E, 2 * ff }, 0.0f, ws);
            add(b + "ffn_down.weight", wt, { ff, E }, 0.0f, ws);
        } else {
            add(b + "ffn_gate.weight", mix(il, 'q'), { E, ff }, 0.0f, ws);
            add(b + "ffn_up.weight", mix(il, 'q'), { E, ff }, 0.0f, ws);
            add(b + "ffn_down.weight", mix(il, 'v'), { ff, E }, 0.0f, ws);
        }
    }
    for (const tensor_spec & s : specs) {
        if (!fits(s.type, s.ne[0])) return fail("synth: tensor " + s.name + " row length does not fit its type");
    }

    gguf_context * g = gguf_init_empty();
    const std::string a = arch;
    auto key = [&](const char * k) { return a + "." + k; };
    gguf_set_val_str(g, "general.architecture", arch.c_str());
    gguf_set_val_str(g, "general.name", ("synthetic-" + arch).c_str());
    gguf_set_val_u32(g, "general.alignment", 32);
    gguf_set_val_u32(g, key("embedding_length").c_str(), (uint32_t) E);
    gguf_set_val_u32(g, key("block_count").c_str(), (uint32_t) p->n_layer);
    gguf_set_val_u32(g, key("context_length").c_str(), (uint32_t) p->n_ctx_train);
    gguf_set_val_u32(g, key("feed_forward_length").c_str(), (uint32_t) ff);
    gguf_set_val_u32(g, key("attention.head_count").c_str(), (uint32_t) nh);
    gguf_set_val_u32(g, key("attention.head_count_kv").c_str(), (uint32_t) nkv);
    gguf_set_val_u32(g, key("attention.key_length").c_str(), (uint32_t) hd);
    gguf_set_val_u32(g, key("attention.value_length").c_str(), (uint32_t) hd);
    gguf_set_val_f32(g, key("attention.layer_norm_rms_epsilon").c_str(), p->rms_eps);
    gguf_set_val_f32(g, key("rope.freq_base").c_str(), p->rope_theta);
    gguf_set_val_u32(g, key("rope.dimension_count").c_str(), (uint32_t) hd);
    if (p->rope_scaling_orig_ctx > 0) {
        gguf_set_val_u32(g, key("rope.scaling.original_context_length").c_str(), (uint32_t) p->rope_scaling_orig_ctx);
        gguf_set_val_f32(g, key("rope.scaling.attn_factor").c_str(), p->rope_attn_factor);
    }
    if (moe) {
        gguf_set_val_u32(g, key("expert_count").c_str(), (uint32_t) p->n_expert);
        gguf_set_val_u32(g, key("expert_used_count").c_str(), (uint32_t) p->n_expert_used);
        gguf_set_val_u32(g, key("expert_feed_forward_length").c_str(), (uint32_t) p->n_ff_exp);
    }
    gguf_set_val_u32(g, "tokenizer.ggml.bos_token_id", 1);
    gguf_set_val_u32(g, "tokenizer.ggml.eos_token_id", 2);
    for (const tensor_spec & s : specs) gguf_add_tensor_info(g, s.name.c_str(), s.type, s.n_dims, s.ne);

    if (!gguf_write_to_file(g, path, /*only_meta=*/true)) { gguf_free(g); return fail(std::string("synth: cannot write ") + path); }
    FILE * f = fopen(path, "ab");
    if (!f) { gguf_free(g); return fail(std::string("synth: cannot append to ") + path); }
    const size_t align = gguf_get_alignment(g);
    const int nth = p->n_threads > 0 ? p->n_threads : omp_get_max_threads();
    size_t pos = 0;
    std::vector<uint8_t> out;
    std::vector<float> tmp;
    std::map<std::string, std::vector<uint8_t>> shared;
    // progress on stderr in tenths of the data for files over 1 GiB (a large model takes minutes)
    size_t total = 0;
    for (const tensor_spec & s : specs) total += ggml_row_size(s.type, s.ne[0]) * (size_t) (s.ne[1] * s.ne[2] * s.ne[3]);
    int tenth = 0;
    auto progress = [&]() {
        if (total < ((size_t) 1 << 30)) return;
        for (; tenth < 10 && pos * 10 >= total * (size_t) (tenth + 1); tenth++) {
            fprintf(stderr, "[synth] %s: %d%% of %.2f GB\n", path, 10 * (tenth + 1), total / 1e9);
        }
    };
    bool ok = true;
    for (size_t ti = 0; ti < specs.size() && ok; ti++) {
        const tensor_spec & s = specs[ti];
        const size_t off = gguf_get_tensor_offset(g, (int64_t) ti);
        if (off > pos) {
            std::vector<uint8_t> z(off - pos, 0);
            ok = fwrite(z.data(), 1, z.size(), f) == z.size();
            pos = off;
        }
        // share_experts: layer 0's expert tensors are kept in memory and written again for every layer
        const bool expert = s.name.rfind("blk.", 0) == 0 && s.name.find("_exps.weight") != std::string::npos;
        const std::string suffix = expert ? s.name.substr(s.name.find('.', 4) + 1) : std::string();
        const bool reuse = p->share_experts && expert && shared.count(suffix) && s.name.rfind("blk.0.", 0) != 0;
        if (reuse) {
            const std::vector<uint8_t> & bytes = shared[suffix];
            ok = fwrite(bytes.data(), 1, bytes.size(), f) == bytes.size();
            pos += bytes.size();
            progress();
            continue;
        }
        std::vector<uint8_t> * keep = p->share_experts && expert ? &shared[suffix] : nullptr;
        const uint64_t k = splitmix64(p->seed ^ name_hash(s.name));
        const int64_t ne0 = s.ne[0];
        const int64_t nrows = s.ne[1] * s.ne[2] * s.ne[3];
        const size_t row_bytes = ggml_row_size(s.type, ne0);
        const int64_t chunk = std::max<int64_t>(1, (int64_t) ((64u << 20) / (size_t) (ne0 * 4)));
        for (int64_t r0 = 0; r0 < nrows && ok; r0 += chunk) {
            const int64_t nr = std::min(chunk, nrows - r0);
            out.resize((size_t) nr * row_bytes);
            tmp.resize((size_t) nr * ne0);
            #pragma omp parallel for num_threads(nth) schedule(static)
            for (int64_t r = 0; r < nr; r++) {
                float * row = tmp.data() + r * ne0;
                const int64_t e0 = (r0 + r) * ne0;
                for (int64_t i = 0; i < ne0; i++) row[i] = (float) (s.mean + s.std * normal_at(k, e0 + i));
                ggml_quantize_chunk(s.type, row, out.data() + r * row_bytes, 0, 1, ne0, nullptr);
            }
            ok = fwrite(out.data(), 1, out.size(), f) == out.size();
            pos += out.size();
            if (keep) keep->insert(keep->end(), out.begin(), out.end());
            progress();
        }
    }
    const size_t end = (pos + align - 1) / align * align;
    if (ok && end > pos) {
        std::vector<uint8_t> z(end - pos, 0);
        ok = fwrite(z.data(), 1, z.size(), f) == z.size();
    }
    ok = (fclose(f) == 0) && ok;
    gguf_free(g);
    if (!ok) return fail(std::string("synth: write error on ") + path);
    return 0;
}
