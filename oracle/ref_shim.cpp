// ref_shim.cpp -- extern "C" entry points over the REFERENCE's own CPU oracle.
// TEST INFRASTRUCTURE, built by oracle/Makefile into oracle/_ref/ only when the
// reference tree is present. It is compiled against the reference's headers
// (include/helix/reference.hpp, tests/harness.hpp) and linked with the
// reference's sources (src/reference/scan_ref.cpp, scan_chunked_ref.cpp,
// src/runtime/desc.cpp) where they lie; nothing of them is copied here.
#include <cstring>
#include <vector>

#include "harness.hpp"
#include "helix/helix.h"
#include "helix/reference.hpp"

extern "C" {

size_t ref_desc_size() { return sizeof(helix_scan_desc); }

void ref_desc_init(helix_scan_desc* d, int32_t L, int32_t S, int32_t H, int32_t P,
                   int32_t N, int32_t G) {
    helix_scan_desc_init(d, L, S, H, P, N, G);
}

void ref_scan(const helix_scan_desc* d, const float* s0, const float* x, const float* dt,
              const float* A, const float* B, const float* C, const int32_t* ids,
              float* y, float* s1) {
    helix::ref::scan(*d, s0, x, dt, A, B, C, ids, y, s1);
}

void ref_scan_chunked(const helix_scan_desc* d, const float* s0, const float* x,
                      const float* dt, const float* A, const float* B, const float* C,
                      const int32_t* ids, float* y, float* s1) {
    helix::ref::scan_chunked(*d, s0, x, dt, A, B, C, ids, y, s1);
}

// Flattens the per-chunk snapshot vectors into `out` (n_chunks * state elems).
void ref_scan_with_snapshots(const helix_scan_desc* d, const float* s0, const float* x,
                             const float* dt, const float* A, const float* B, const float* C,
                             const int32_t* ids, float* y, float* s1, int32_t chunk,
                             double* out) {
    std::vector<std::vector<double>> snaps;
    helix::ref::scan_with_snapshots(*d, s0, x, dt, A, B, C, ids, y, s1, chunk, &snaps);
    size_t off = 0;
    for (const auto& v : snaps) {
        std::memcpy(out + off, v.data(), v.size() * sizeof(double));
        off += v.size();
    }
}

// The harness generator, exactly as the reference's tests call it.
void ref_problem_make(int32_t L, int32_t S, int32_t H, int32_t P, int32_t N, int32_t G,
                      int32_t chunk, uint64_t seed, int memory,
                      float* s0, float* x, float* dt, float* A, float* B, float* C,
                      helix_scan_desc* d_out) {
    using helix::test::Memory;
    using helix::test::Problem;
    Problem p = Problem::make(L, S, H, P, N, G, chunk, seed,
                              memory ? Memory::LONG : Memory::SHORT);
    std::memcpy(s0, p.s0.data(), p.s0.size() * 4);
    std::memcpy(x, p.x.data(), p.x.size() * 4);
    std::memcpy(dt, p.dt.data(), p.dt.size() * 4);
    std::memcpy(A, p.A.data(), p.A.size() * 4);
    std::memcpy(B, p.B.data(), p.B.size() * 4);
    std::memcpy(C, p.C.data(), p.C.size() * 4);
    if (d_out) *d_out = p.d;
}

}  // extern "C"
