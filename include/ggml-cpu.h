// ggml-cpu.h — the CPU backend entry points GGML-Loader calls in init_backend("cpu")
// (model.cpp:791-799; n_threads=8 from cmd_bench.cpp:107, cmd_run.cpp:400).
//
// In this build the CPU backend is the test oracle: a separate library (oracle/) that restates
// ggml-cpu's arithmetic. The product libraries never link it; it registers itself under the
// name "CPU" when loaded, and init_backend("cpu") finds it through ggml_backend_init_by_name.
#pragma once

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

GGML_API ggml_backend_t ggml_backend_cpu_init(void);
GGML_API bool           ggml_backend_is_cpu(ggml_backend_t backend);
GGML_API void           ggml_backend_cpu_set_n_threads(ggml_backend_t backend_cpu, int n_threads);

#ifdef __cplusplus
}
#endif
