// device.cpp -- context lifetime, device probe and code-object loading.
//
// Counterpart of the reference's src/runtime/device.mm:7-85 and
// library.mm:51-142. The Metal device / metallib / lazily-built pipeline
// cache becomes one hipModule:
//   1. explicit code_object_path argument
//   2. $HELIX_HSACO
//   3. the gfx950 code object embedded in this library at build time
// and every kernel is resolved with hipModuleGetFunction before the context is
// returned, so encoding never creates anything and a missing kernel fails at
// creation rather than mid-encode.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "helix/helix_host.h"
#include "helix_internal.h"

extern "C" {
extern const unsigned char helix_hsaco_data[];
extern const size_t helix_hsaco_len;
}

namespace {

std::string hip_msg(const char* what, hipError_t e) {
    return std::string(what) + ": " + hipGetErrorString(e);
}

}  // namespace

extern "C" helix_status helix_ctx_create(helix_ctx** out, void* device, const char* code_object_path) {
    using helix::rt::set_error;
    if (!out) return HELIX_ERR_INVALID_ARG;
    *out = nullptr;

    int dev = -1;
    if (device) {
        dev = *static_cast<const int*>(device);
    } else if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        set_error(nullptr, "no HIP device");
        return HELIX_ERR_NO_DEVICE;
    }
    int n_dev = 0;
    if (hipGetDeviceCount(&n_dev) != hipSuccess || dev < 0 || dev >= n_dev) {
        (void)hipGetLastError();
        set_error(nullptr, "HIP device ordinal out of range");
        return HELIX_ERR_NO_DEVICE;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        (void)hipGetLastError();
        set_error(nullptr, "hipGetDeviceProperties failed");
        return HELIX_ERR_NO_DEVICE;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error(nullptr, std::string("device is ") + prop.gcnArchName + ", this build targets gfx950");
        return HELIX_ERR_NO_DEVICE;
    }

    int prev = -1;
    (void)hipGetDevice(&prev);
    if (prev != dev && hipSetDevice(dev) != hipSuccess) {
        (void)hipGetLastError();
        set_error(nullptr, "hipSetDevice failed");
        return HELIX_ERR_NO_DEVICE;
    }

    auto* ctx = new helix_ctx();
    ctx->tuning = helix::rt::tuning_from_env();
    ctx->device = dev;
    ctx->arch = prop.gcnArchName;
    ctx->n_cu = prop.multiProcessorCount;

    const char* path = code_object_path;
    if (!path) path = std::getenv("HELIX_HSACO");
    hipError_t e;
    if (path && *path) {
        e = hipModuleLoad(&ctx->module, path);
        ctx->code_object = path;
    } else {
        e = hipModuleLoadData(&ctx->module, helix_hsaco_data);
        ctx->code_object = "<embedded>";
    }
    helix_status st = HELIX_OK;
    std::string err;
    if (e != hipSuccess) {
        (void)hipGetLastError();
        err = hip_msg(("failed to load code object " + ctx->code_object).c_str(), e);
        st = HELIX_ERR_NO_DEVICE;
    } else {
        size_t n = 0;
        const char* const* names = helix::rt::all_kernel_names(&n);
        for (size_t i = 0; i < n; ++i) {
            hipFunction_t f = nullptr;
            e = hipModuleGetFunction(&f, ctx->module, names[i]);
            if (e != hipSuccess || !f) {
                (void)hipGetLastError();
                err = hip_msg((std::string("kernel ") + names[i] + " missing from code object").c_str(), e);
                st = HELIX_ERR_PIPELINE;
                break;
            }
            ctx->kernels[names[i]] = f;
        }
    }
    if (prev >= 0 && prev != dev) (void)hipSetDevice(prev);

    if (st != HELIX_OK) {
        if (ctx->module) (void)hipModuleUnload(ctx->module);
        delete ctx;
        set_error(nullptr, err);
        return st;
    }
    *out = ctx;
    return HELIX_OK;
}

extern "C" helix_status helix_ctx_create_host(helix_ctx** out) {
    if (!out) return HELIX_ERR_INVALID_ARG;
    auto* ctx = new helix_ctx();
    ctx->tuning = helix::rt::tuning_from_env();
    ctx->device = -1;
    ctx->code_object = "<none: host-only context>";
    *out = ctx;
    return HELIX_OK;
}

extern "C" void helix_ctx_free(helix_ctx* ctx) {
    if (!ctx) return;
    if (ctx->module) {
        int prev = -1;
        (void)hipGetDevice(&prev);
        if (prev != ctx->device) (void)hipSetDevice(ctx->device);
        (void)hipModuleUnload(ctx->module);
        if (prev >= 0 && prev != ctx->device) (void)hipSetDevice(prev);
    }
    delete ctx;
}
