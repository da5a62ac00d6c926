// pass_b.hip -- Pass B: inter-segment state scan (HBM-bound).
//
// Reference counterpart: helix_state_scan_f32 (src/kernels/
// helix_scan_multipass.metal:154-220), a serial walk per (state, channel)
// slot over every chunk's (decay, dS) pair with the associative operator
// (a1, b1).(a2, b2) = (a1 a2, a2 b1 + b2) (multipass.metal:10-15).
//
// Pass A has already folded each segment's chunks into one (decay, D) pair,
// so this walk is seg_len times shorter than the reference's. One lane per
// state element of one (seq, head): the [P][N] element index is contiguous,
// so every segment row, s0 row and s1 row moves as full 256-byte wave
// transactions. The D loads of a block of segments are issued before the
// dependent FMA chain so the loads overlap.
//
//   carry = s0[ids[seq]] (first group) or s1[seq] (later groups)
//   for s: S_seg(s) = carry (in place over D_s); carry = exp(segld_s) carry + D_s
//   s1[seq] = carry
#include "helix_common.h"

extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_state_scan_f32(HelixScanParams p,
                                                                           HelixScanBuffers b) {
    constexpr int BLK = 8;
    const long long PN = (long long)p.head_dim * p.d_state;
    const long long e  = (long long)blockIdx.x * HELIX_WG + threadIdx.x;
    const int h   = blockIdx.y;
    const int seq = blockIdx.z;
    if (e >= PN) return;

    const int src = p.has_ids ? b.ids[seq] : seq;
    const long long s_out = seq * p.seq_s + h * p.s_s[0] + e;
    float carry = p.first_group ? b.s0[src * p.seq_s + h * p.s_s[0] + e] : b.s1[s_out];

    float* __restrict__ base = b.s_seg + seq * p.sg_seq + h * PN + e;
    const float* __restrict__ sd = b.segld + seq * p.sd_seq + h;

    for (int s0 = 0; s0 < p.n_seg; s0 += BLK) {
        const int nb = min(BLK, p.n_seg - s0);
        float d[BLK], a[BLK];
#pragma unroll
        for (int k = 0; k < BLK; ++k) {
            if (k < nb) {
                d[k] = base[(long long)(s0 + k) * p.sg_seg];
                a[k] = expf(sd[(long long)(s0 + k) * p.n_head]);
            }
        }
#pragma unroll
        for (int k = 0; k < BLK; ++k) {
            if (k < nb) {
                base[(long long)(s0 + k) * p.sg_seg] = carry;
                carry = a[k] * carry + d[k];
            }
        }
    }
    b.s1[s_out] = carry;
}
