// noalloc.hip -- the scratch of helix_scan_encode_noalloc: a fixed device
// array the library holds on each GPU, for callers that cannot allocate.
//
// This translation unit is compiled by hipcc (host and gfx950 device code)
// and linked into libhelix.so beside the C++ runtime. The array lives in its
// code object; the scan kernels (in the embedded hipModule) take its address
// as their scratch pointer, exactly as they take a caller's buffer.
//
// In host code `helix_noalloc_scratch` names a host-side stand-in, not device
// memory: only the address hipGetSymbolAddress returns for it, resolved once
// per device (on the entry point's first call there, with that device
// current), is ever passed to a kernel.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "helix/helix_host.h"
#include "helix_internal.h"

namespace {

static __device__ __align__(256) unsigned char helix_noalloc_scratch[HELIX_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

std::mutex g_mu;
void* g_ptr[kMaxDevices];          // device address of the array, per device
std::string g_err[kMaxDevices];    // why the address could not be resolved

}  // namespace

namespace helix::rt {

void* noalloc_scratch(int device, std::string* why) {
    if (device < 0 || device >= kMaxDevices) {
        *why = "device ordinal beyond the fixed scratch table";
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[device] && g_err[device].empty()) {
        // First call on this device: resolve the array's address there, with
        // the device current.
        int prev = -1;
        (void)hipGetDevice(&prev);
        if (prev != device && hipSetDevice(device) != hipSuccess) {
            (void)hipGetLastError();
            *why = "hipSetDevice failed";
            return nullptr;
        }
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(helix_noalloc_scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            g_err[device] = std::string("hipGetSymbolAddress of the fixed scratch failed: ") + hipGetErrorString(e);
        } else {
            g_ptr[device] = p;
        }
        if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
    }
    if (!g_ptr[device]) *why = g_err[device];
    return g_ptr[device];
}

}  // namespace helix::rt
