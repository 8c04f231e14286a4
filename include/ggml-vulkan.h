// ggml-vulkan.h — the Vulkan backend entry points model.cpp includes (model.cpp:5) and calls from
// init_backend (model.cpp:800-813). This build has no Vulkan backend: the device count is 0, so
// init_backend("vulkan") takes the reference's own "no Vulkan devices" exit, and the other two
// report nothing. `--backend hip` (ggml-hip.h) is the GPU backend here.
#pragma once

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

// reference call site: model.cpp:801; always 0 in this build
GGML_API int  ggml_backend_vk_get_device_count(void);
// reference call site: model.cpp:806; writes an empty string
GGML_API void ggml_backend_vk_get_device_description(int device, char * description, size_t description_size);
// reference call site: model.cpp:808; always NULL in this build
GGML_API ggml_backend_t ggml_backend_vk_init(size_t dev_num);

#ifdef __cplusplus
}
#endif
