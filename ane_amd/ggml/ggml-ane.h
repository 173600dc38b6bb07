/*
 * ggml-ane.h -- registry entry point of the ggml backend on MI355X.
 *
 * Replaces ggml_backend_ane_reg() (src/ggml-backend/ggml-ane.h:20): the same
 * name and signature, so a ggml build that registered the reference backend
 * registers this one unchanged.  The implementation (ggml-ane.cpp) is
 * compiled inside a ggml tree against ggml's own headers and links
 * libane_amd.so; see ggml-ane.cpp for the interface revision it targets.
 */
#pragma once

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

GGML_BACKEND_API ggml_backend_reg_t ggml_backend_ane_reg(void);

#ifdef __cplusplus
}
#endif
