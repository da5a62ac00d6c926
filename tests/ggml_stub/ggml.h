/* Test-only stand-in for ggml.h, used to unit-test the HELIX ggml bridge
 * (helix_amd/integration/ggml) without llama.cpp, which is absent offline.
 * It declares only what the bridge uses, with upstream ggml's names and
 * meanings (ggml/include/ggml.h): ne[] element counts and nb[] byte strides,
 * fastest dimension first; src[]; op_params; data (a device pointer on the
 * HIP backend). The field order is this file's own and is mirrored by
 * tests/ggml_fake.py; the real header orders and extends it differently,
 * which the bridge does not depend on. */
#ifndef HELIX_TEST_GGML_STUB_H
#define HELIX_TEST_GGML_STUB_H

#include <stddef.h>
#include <stdint.h>

#define GGML_MAX_DIMS 4
#define GGML_MAX_SRC 10
#define GGML_MAX_OP_PARAMS 64

enum ggml_type {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_I32 = 26,
};

struct ggml_tensor {
    enum ggml_type type;
    int64_t ne[GGML_MAX_DIMS];
    size_t  nb[GGML_MAX_DIMS];
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    struct ggml_tensor * src[GGML_MAX_SRC];
    void * data;
};

static inline int64_t ggml_nelements(const struct ggml_tensor * t) {
    return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3];
}

#endif
