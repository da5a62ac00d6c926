// helix_common.h -- device helpers shared by the gfx950 HELIX kernels.
//
// Wave64 conventions used throughout:
//   lane = threadIdx.x & 63, wave = threadIdx.x >> 6 (4 waves per workgroup)
//   lo = lane & 31, hi = lane >> 5
//
// MFMA operand/result layouts (CDNA3/CDNA4 ISA):
//   v_mfma_f32_32x32x2_f32   A[i][k]: lane holds A[lo][hi]
//                            B[k][j]: lane holds B[hi][lo]
//                            D[i][j]: lane, reg r holds D[8*(r/4) + 4*hi + r%4][lo]
//   v_mfma_f32_32x32x16_bf16 A[i][k]: lane holds A[lo][8*hi + e], e = 0..7
//                            B[k][j]: lane holds B[8*hi + e][lo]
//                            D as above
// tests/test_gpu_mfma_layout.py checks these on the device.
#ifndef HELIX_COMMON_H
#define HELIX_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "helix_params.h"

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

#define HELIX_DEV static __device__ __forceinline__

HELIX_DEV int lane_id() { return threadIdx.x & 63; }
HELIX_DEV int wave_id() { return threadIdx.x >> 6; }

// softplus with the v > 20 shortcut the reference and ggml use
// (reference src/kernels/helix_common.h:14-16). log1p keeps full relative
// precision for the strongly negative dt of long-memory models.
HELIX_DEV float helix_softplus(float v) { return v > 20.0f ? v : log1pf(expf(v)); }

HELIX_DEV float helix_dt(const HelixScanParams& p, float raw) {
    return fminf(fmaxf(helix_softplus(raw), p.dt_min), p.dt_max);
}

// Inclusive prefix sum over the 64 lanes of a wave (Kogge-Stone, 6 steps),
// in fp64: the intra-chunk decays are exp(Lcum_t - Lcum_j), and with
// |A*dt| summing to a few hundred per chunk an fp32 prefix would lose the
// low digits that the difference of two nearby prefixes needs.
HELIX_DEV double wave_incl_sum(double v) {
    const int lane = lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const double n = __shfl_up(v, d, 64);
        if (lane >= d) v += n;
    }
    return v;
}

// Per-chunk decay preamble, computed redundantly by every wave so no LDS or
// barrier is needed: lane t owns token t of the chunk.
//   dtv  = clamp(softplus(dt_t))          (0 for t >= tlen)
//   lcum = sum_{j<=t} A_h * dtv_j         fp64; A_h*dtv is exact in fp64.
//                                         Constant past tlen since dtv = 0.
//   lend = lcum at the chunk's last token
// Padded rows therefore carry Lcum[tlen-1], which keeps every intra-chunk
// exponent Lcum_t - Lcum_j <= 0 for j <= t (reference helix_common.h:110-120).
struct ChunkDecay {
    float  dtv;
    double lcum;
    double lend;
};

HELIX_DEV ChunkDecay chunk_decay(const HelixScanParams& p, const float* __restrict__ dt_h,
                                 int t0, int tlen, float A_h) {
    const int lane = lane_id();
    ChunkDecay r;
    r.dtv = 0.0f;
    if (lane < tlen) r.dtv = helix_dt(p, dt_h[(long long)(t0 + lane) * p.s_dt[0]]);
    r.lcum = wave_incl_sum((double)A_h * (double)r.dtv);
    r.lend = __shfl(r.lcum, 63, 64);
    return r;
}

// exp of a (small, non-positive in practice) fp64 log-decay difference.
HELIX_DEV float exp_diff(double a, double b) { return expf((float)(a - b)); }

// MI355X hands the workgroups of a launch to its 8 XCDs round-robin (linear
// id i runs on XCD i % 8), and each XCD has its own L2. This maps the linear
// id to a logical id so that a contiguous run of logical ids shares one XCD:
// work items that read the same data (chunks of one segment, heads of one
// group) then share an L2 instead of each XCD fetching its own copy.
// A bijection on [0, total); the ragged tail past a multiple of 8 is kept.
HELIX_DEV unsigned xcd_logical_id(unsigned linear, unsigned total) {
    constexpr unsigned kXcd = 8;
    const unsigned per = total / kXcd;
    if (linear >= per * kXcd) return linear;
    return (linear % kXcd) * per + linear / kXcd;
}

// Wave-uniform broadcast of lane `src`'s value (src must be wave-uniform).
HELIX_DEV float bcast(float v, int src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}
HELIX_DEV double bcast(double v, int src) {
    const long long u = __builtin_bit_cast(long long, v);
    const int lo32 = __builtin_amdgcn_readlane((int)(u & 0xffffffffLL), src);
    const int hi32 = __builtin_amdgcn_readlane((int)(u >> 32), src);
    return __builtin_bit_cast(double, ((long long)hi32 << 32) | (unsigned int)lo32);
}

HELIX_DEV f32x16 mfma_f32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

HELIX_DEV f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Row of MFMA result register r for this lane (column is lo).
HELIX_DEV int acc_row(int r, int hi) { return 8 * (r >> 2) + 4 * hi + (r & 3); }

HELIX_DEV f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.0f;
    return z;
}

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
HELIX_DEV __bf16 to_bf16(float v) { return (__bf16)v; }

#endif  // HELIX_COMMON_H
