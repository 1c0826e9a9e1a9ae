// ggml-qwmoe.h -- the libqwmoe ggml backend's registration (ggml backend API v3).
// A process may link it and call ggml_backend_qwmoe_reg(), or load the shared
// object with ggml_backend_load(), which calls its exported ggml_backend_init.
#pragma once

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

GGML_BACKEND_API ggml_backend_reg_t ggml_backend_qwmoe_reg(void);

#ifdef __cplusplus
}
#endif
