// main.cpp — `ggml-loader` CLI of this build:
//   ggml-loader bench <model.gguf> [--backend hip|cpu] [--cpu-lib PATH] [-p n_prompt] [-n n_gen]
//                     [-r reps] [--ctx N] [--flash-attn]
//       pp/tg tok/s exactly as the reference's cmd_bench (cmd_bench.cpp:30-165): one untimed
//       warmup cycle, then r reps of {prefill n_prompt tokens; n_gen greedy decode steps},
//       mean +- sample stddev. `--backend cpu` needs the CPU reference backend library, loaded
//       with --cpu-lib (it is test infrastructure, not part of this product).
//   ggml-loader synth <out.gguf> --arch A --embd E --layers L --heads H --heads-kv HK --head-dim D
//                     --ff F --vocab V --type q4_0|q8_0|q4_K [--theta T] [--seed S] [--tied]
//       writes a seeded synthetic model (see ggml-loader.h)
//   ggml-loader inspect <model.gguf>
//       metadata and tensor directory (reference cmd_inspect.cpp:41-90)
#include "ggml-loader.h"
#include "gguf.h"
#include "model.h"
#include "runtime_error.h"

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

static int type_from_name(const std::string & s) {
    if (s == "q4_0") return GGML_TYPE_Q4_0;
    if (s == "q8_0") return GGML_TYPE_Q8_0;
    if (s == "q4_K" || s == "q4_k") return GGML_TYPE_Q4_K;
    if (s == "f16") return GGML_TYPE_F16;
    if (s == "f32") return GGML_TYPE_F32;
    return -1;
}

struct stats { double mean; double stddev; };
static stats compute_stats(const std::vector<double> & xs) {
    double sum = 0.0;
    for (double x : xs) sum += x;
    const double mean = sum / (double) xs.size();
    double var = 0.0;
    for (double x : xs) var += (x - mean) * (x - mean);
    var /= xs.size() > 1 ? (double) (xs.size() - 1) : 1.0;
    return { mean, sqrt(var) };
}

static int cmd_bench(int argc, char ** argv) {
    std::string model_path, backend_name = "hip", cpu_lib;
    int n_pp = 128, n_tg = 64, n_reps = 3;
    bool flash_attn = false;
    int64_t n_ctx = 0;
    for (int i = 2; i < argc; i++) {
        std::string a = argv[i];
        if (a == "--backend" && i + 1 < argc) backend_name = argv[++i];
        else if (a == "--cpu-lib" && i + 1 < argc) cpu_lib = argv[++i];
        else if (a == "-p" && i + 1 < argc) n_pp = atoi(argv[++i]);
        else if (a == "-n" && i + 1 < argc) n_tg = atoi(argv[++i]);
        else if (a == "-r" && i + 1 < argc) n_reps = atoi(argv[++i]);
        else if (a == "--flash-attn") flash_attn = true;
        else if (a == "--ctx" && i + 1 < argc) n_ctx = atoll(argv[++i]);
        else if (model_path.empty()) model_path = a;
    }
    if (model_path.empty()) { fprintf(stderr, "usage: ggml-loader bench <model.gguf> [options]\n"); return 1; }
    if (!cpu_lib.empty() && !ggml_backend_load(cpu_lib.c_str())) return 1;
    if (n_ctx == 0) n_ctx = n_pp + n_tg;
    if ((int64_t) n_pp + n_tg > n_ctx) {
        fprintf(stderr, "error: -p (%d) + -n (%d) exceeds n_ctx (%lld)\n", n_pp, n_tg, (long long) n_ctx);
        return 1;
    }
    try {
        ggml_backend_t backend = init_backend(backend_name, 8);
        gguf_context * gctx = nullptr;
        weights_store ws = load_weights(model_path.c_str(), backend, &gctx);
        hparams hp = load_hparams(gctx);
        model m = load_model(ws.ctx, hp);
        const int64_t n_vocab = m.token_embd->ne[1];
        kv_cache kv = init_kv_cache(m, hp, backend, n_ctx);
        decode_session ds = init_decode_session(backend, hp, flash_attn);
        auto run_cycle = [&](double & pp, double & tg) {
            std::vector<int32_t> pp_tokens(n_pp);
            for (int i = 0; i < n_pp; i++) pp_tokens[i] = (int32_t) (i % (n_vocab - 1)) + 1;
            auto t0 = std::chrono::steady_clock::now();
            std::vector<float> logits = forward_step(m, hp, kv, ds, backend, 0, pp_tokens, n_vocab);
            auto t1 = std::chrono::steady_clock::now();
            int64_t n_past = n_pp;
            int32_t next = argmax(logits);
            auto t2 = std::chrono::steady_clock::now();
            for (int i = 0; i < n_tg; i++) {
                std::vector<float> sl = forward_step(m, hp, kv, ds, backend, n_past, { next }, n_vocab);
                n_past += 1;
                next = argmax(sl);
            }
            auto t3 = std::chrono::steady_clock::now();
            pp = n_pp / std::chrono::duration<double>(t1 - t0).count();
            tg = n_tg / std::chrono::duration<double>(t3 - t2).count();
        };
        fprintf(stderr, "model=%s arch=%s backend=%s n_layer=%lld -- pp%d, tg%d, %d reps (+1 warmup)\n", model_path.c_str(),
                hp.arch_name.c_str(), backend_name.c_str(), (long long) hp.n_layer, n_pp, n_tg, n_reps);
        double pp, tg;
        run_cycle(pp, tg);
        std::vector<double> pps, tgs;
        for (int r = 0; r < n_reps; r++) {
            run_cycle(pp, tg);
            pps.push_back(pp);
            tgs.push_back(tg);
            fprintf(stderr, "  rep %d/%d: pp %.2f tok/s, tg %.2f tok/s\n", r + 1, n_reps, pp, tg);
        }
        const stats a = compute_stats(pps), b = compute_stats(tgs);
        printf("\n| model      | backend | test  |          t/s |\n");
        printf("| ---------- | ------- | ----- | ------------ |\n");
        printf("| %-10s | %-7s | pp%-3d | %6.2f ± %5.2f |\n", hp.arch_name.c_str(), backend_name.c_str(), n_pp, a.mean, a.stddev);
        printf("| %-10s | %-7s | tg%-3d | %6.2f ± %5.2f |\n", hp.arch_name.c_str(), backend_name.c_str(), n_tg, b.mean, b.stddev);
        free_decode_session(ds);
        ggml_backend_buffer_free(kv.buffer);
        ggml_free(kv.ctx);
        ggml_backend_buffer_free(ws.buffer);
        ggml_free(ws.ctx);
        ggml_backend_free(backend);
        gguf_free(gctx);
    } catch (const gl_error & e) {
        fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
    return 0;
}

static int cmd_synth(int argc, char ** argv) {
    if (argc < 3) { fprintf(stderr, "usage: ggml-loader synth <out.gguf> [options]\n"); return 1; }
    gl_synth_params p{};
    std::string arch = "llama";
    p.n_embd = 256; p.n_layer = 2; p.n_head = 4; p.n_head_kv = 2; p.head_dim = 64; p.n_ff = 512; p.n_vocab = 1024;
    p.n_ctx_train = 4096; p.rope_theta = 10000.0f; p.rms_eps = 1e-5f; p.wtype = GGML_TYPE_Q4_0;
    p.embd_type = -1; p.output_type = -1; p.w_std = 0.02f; p.norm_std = 0.01f; p.seed = 1;
    for (int i = 3; i < argc; i++) {
        std::string a = argv[i];
        auto next = [&]() { return i + 1 < argc ? std::string(argv[++i]) : std::string(); };
        if (a == "--arch") arch = next();
        else if (a == "--embd") p.n_embd = atoll(next().c_str());
        else if (a == "--layers") p.n_layer = atoll(next().c_str());
        else if (a == "--heads") p.n_head = atoll(next().c_str());
        else if (a == "--heads-kv") p.n_head_kv = atoll(next().c_str());
        else if (a == "--head-dim") p.head_dim = atoll(next().c_str());
        else if (a == "--ff") p.n_ff = atoll(next().c_str());
        else if (a == "--vocab") p.n_vocab = atoll(next().c_str());
        else if (a == "--experts") p.n_expert = atoll(next().c_str());
        else if (a == "--experts-used") p.n_expert_used = atoll(next().c_str());
        else if (a == "--ff-exp") p.n_ff_exp = atoll(next().c_str());
        else if (a == "--theta") p.rope_theta = (float) atof(next().c_str());
        else if (a == "--seed") p.seed = strtoull(next().c_str(), nullptr, 10);
        else if (a == "--type") p.wtype = type_from_name(next());
        else if (a == "--tied") p.tied_output = 1;
        else { fprintf(stderr, "synth: unknown option %s\n", a.c_str()); return 1; }
    }
    if (p.wtype < 0) { fprintf(stderr, "synth: unknown --type\n"); return 1; }
    if (p.embd_type < 0) p.embd_type = p.wtype;
    if (p.output_type < 0) p.output_type = p.wtype;
    p.arch = arch.c_str();
    char err[512] = { 0 };
    if (gl_synth_model(argv[2], &p, err, sizeof(err)) != 0) { fprintf(stderr, "error: %s\n", err); return 1; }
    return 0;
}

// cmd_inspect.cpp:11-38: the value column of a metadata key (integers and floats as
// std::to_string prints them, strings cut to 77 characters + "..." past 80, arrays as
// array<type>[n])
static std::string inspect_value(const gguf_context * g, int64_t i) {
    switch (gguf_get_kv_type(g, i)) {
        case GGUF_TYPE_UINT8:   return std::to_string(gguf_get_val_u8(g, i));
        case GGUF_TYPE_INT8:    return std::to_string(gguf_get_val_i8(g, i));
        case GGUF_TYPE_UINT16:  return std::to_string(gguf_get_val_u16(g, i));
        case GGUF_TYPE_INT16:   return std::to_string(gguf_get_val_i16(g, i));
        case GGUF_TYPE_UINT32:  return std::to_string(gguf_get_val_u32(g, i));
        case GGUF_TYPE_INT32:   return std::to_string(gguf_get_val_i32(g, i));
        case GGUF_TYPE_FLOAT32: return std::to_string(gguf_get_val_f32(g, i));
        case GGUF_TYPE_UINT64:  return std::to_string(gguf_get_val_u64(g, i));
        case GGUF_TYPE_INT64:   return std::to_string(gguf_get_val_i64(g, i));
        case GGUF_TYPE_FLOAT64: return std::to_string(gguf_get_val_f64(g, i));
        case GGUF_TYPE_BOOL:    return gguf_get_val_bool(g, i) ? "true" : "false";
        case GGUF_TYPE_STRING: {
            const std::string v = gguf_get_val_str(g, i);
            return v.size() > 80 ? v.substr(0, 77) + "..." : v;
        }
        case GGUF_TYPE_ARRAY:
            return "array<" + std::string(gguf_type_name(gguf_get_arr_type(g, i))) + ">[" +
                   std::to_string(gguf_get_arr_n(g, i)) + "]";
        default:
            return "?";
    }
}

// cmd_inspect.cpp:41-90: file header, metadata keys, tensor directory, total tensor bytes, in the
// reference's layout (a model given as a file path; Ollama references are not resolved here)
static int cmd_inspect(int argc, char ** argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: %s <model.gguf>\n", argv[1]);
        return 1;
    }
    const char * path = argv[2];
    gguf_init_params gp = { true, nullptr };
    gguf_context * g = gguf_init_from_file(path, gp);
    if (!g) {
        fprintf(stderr, "error: failed to load '%s' as GGUF\n", path);
        return 1;
    }
    printf("file:      %s\n", path);
    printf("version:   %u\n", gguf_get_version(g));
    printf("alignment: %zu\n", gguf_get_alignment(g));
    const int64_t n_kv = gguf_get_n_kv(g);
    printf("\n-- metadata (%lld keys) --\n", (long long) n_kv);
    for (int64_t i = 0; i < n_kv; i++) printf("  %-40s = %s\n", gguf_get_key(g, i), inspect_value(g, i).c_str());
    const int64_t n_t = gguf_get_n_tensors(g);
    size_t total = 0;
    printf("\n-- tensors (%lld) --\n", (long long) n_t);
    for (int64_t i = 0; i < n_t; i++) {
        const int64_t * ne = gguf_get_tensor_ne(g, i);
        const size_t size = gguf_get_tensor_size(g, i);
        total += size;
        printf("  %-40s %6s  [%5lld, %5lld, %5lld, %5lld]  %10zu bytes\n", gguf_get_tensor_name(g, i),
               ggml_type_name(gguf_get_tensor_type(g, i)), (long long) ne[0], (long long) ne[1], (long long) ne[2],
               (long long) ne[3], size);
    }
    printf("\ntotal tensor data: %.2f MiB\n", total / 1024.0 / 1024.0);
    gguf_free(g);
    return 0;
}

int main(int argc, char ** argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: ggml-loader <bench|synth|inspect> ...\n");
        return 1;
    }
    const std::string cmd = argv[1];
    if (cmd == "bench") return cmd_bench(argc, argv);
    if (cmd == "synth") return cmd_synth(argc, argv);
    if (cmd == "inspect") return cmd_inspect(argc, argv);
    fprintf(stderr, "unknown command '%s'\n", cmd.c_str());
    return 1;
}
