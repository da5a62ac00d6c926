// pass_b.hip -- Pass B: inter-segment state scan (HBM-bound).
//
// Reference counterpart: helix_state_scan_f32 (src/kernels/
// helix_scan_multipass.metal:154-220), a serial walk per (state, channel)
// slot over every chunk's (decay, dS) pair with the associative operator
// (a1, b1).(a2, b2) = (a1 a2, a2 b1 + b2) (multipass.metal:10-15).
//
// Pass A has already folded each segment's chunks into one (decay, D) pair,
// so this walk is seg_len times shorter than the reference's. One thread per
// tile unit (four consecutive n of one p, helix_params.h layout) of one
// (seq, head): every segment row moves as 16-byte lane accesses, 1 KiB
// contiguous per wave. The D loads of a block of up to 16 segments are all
// issued before the dependent FMA chain, so a thread waits on memory once per
// block.
//
//   carry = s0[ids[seq]] (first group) or s1[seq] (later groups)
//   for s: S_seg(s) = carry (in place over D_s) if s starts a walk;
//          carry = exp(segld_s) carry + D_s
//   s1[seq] = carry
// Pass C starts a walk every walk_len / seg_len segments and reads the start
// states of those segments only; the others are not stored.
// YT: the single pass's form without scratch (HelixScanParams::ytile): the
// tiles and the log-decays are read from, and the start states written to, y
// (ytile_* in helix_common.h).
#include "helix_common.h"

template <bool YT>
__device__ __forceinline__ void state_scan_impl(const HelixScanParams& p, const HelixScanBuffers& b) {
    constexpr int BLK = 16;
    const int units_tile = 16 * p.np;                    // 64 * np / 4
    const int per_head = p.n_pslab * units_tile;
    const int u   = blockIdx.x * HELIX_WG + threadIdx.x; // unit within (seq, head)
    const int h   = blockIdx.y;
    const int seq = blockIdx.z;
    if (u >= per_head) return;

    // Unit -> (p, n..n+3).
    const int NT   = p.np / 32;
    const int slab = u / units_tile;
    const int q    = u % units_tile;
    const int lane = q & 63, r4 = (q >> 6) & 3, t = q >> 8;
    const int pr = slab * HELIX_HD + (t / NT) * 32 + (lane & 31);
    const int n  = (t % NT) * 32 + 8 * r4 + 4 * (lane >> 5);
    // Tile padding (p past head_dim, n past d_state) holds finite values that
    // no result depends on; it is scanned like the rest but never reaches s1.
    // d_state % 8 == 0, so n..n+3 are all valid or all padding.
    const bool valid = pr < p.head_dim && n < p.d_state;

    const int src = p.has_ids ? b.ids[seq] : seq;
    const long long soff = h * p.s_s[0] + (long long)pr * p.s_s[1] + n;
    f32x4 carry = {0.0f, 0.0f, 0.0f, 0.0f};
    if (valid) {
        const float* cs = p.first_group ? b.s0 + src * p.seq_s + soff : b.s1 + seq * p.seq_s + soff;
#pragma unroll
        for (int k = 0; k < 4; ++k) carry[k] = cs[k];
    }

    f32x4* __restrict__ base =
        YT ? nullptr : reinterpret_cast<f32x4*>(b.s_seg + seq * p.sg_seq + (long long)h * per_head * 4) + u;
    const long long seg_stride = p.sg_seg / 4;           // in units
    const float* __restrict__ sd = YT ? nullptr : b.segld + seq * p.sd_seq + h;
    const int ratio = p.walk_len / p.seg_len;            // segments per walk
    // YT: unit q of the slab's tile of segment s, and its log-decay, in y:
    // segment 0's addresses plus s segments of rows.
    const int pws = min(HELIX_HD, p.head_dim - slab * HELIX_HD);
    float* const yd0 = YT ? b.y + ytile_base(p, seq, h, slab, 0) + ytile_unit(p, q, pws) : nullptr;
    const float* const ya0 = YT ? b.y + ytile_segld(p, seq, h, 0) : nullptr;
    const long long yseg = (long long)p.seg_len * HELIX_CS * p.s_y[0];   // floats per segment of rows
    auto d_ptr = [&](long long s) -> f32x4* {
        if constexpr (YT) return reinterpret_cast<f32x4*>(yd0 + s * yseg);
        else return base + s * seg_stride;
    };
    auto a_ptr = [&](long long s) -> const float* {
        if constexpr (YT) return ya0 + s * yseg;
        else return sd + s * p.n_head;
    };

    // One block of up to K segments from s0: loads past the block's end
    // repeat its last segment, so there is no branch between the loads and
    // they all issue before the first wait.
    auto block = [&](auto kc, int s0) {
        constexpr int K = decltype(kc)::value;
        const int nb = min(K, p.n_seg - s0);
        f32x4 d[K];
        float a[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const long long sk = s0 + min(k, nb - 1);
            d[k] = *d_ptr(sk);
            a[k] = *a_ptr(sk);
        }
#pragma unroll
        for (int k = 0; k < K; ++k) a[k] = expf(a[k]);
#pragma unroll
        for (int k = 0; k < K; ++k) {
            if (k < nb) {
                if ((s0 + k) % ratio == 0) *d_ptr(s0 + k) = carry;
                carry = a[k] * carry + d[k];
            }
        }
    };
    // Blocks of 16 segments; a last block of at most 8 or 4 segments issues
    // 8 or 4 loads.
    for (int s0 = 0; s0 < p.n_seg; s0 += BLK) {
        const int left = p.n_seg - s0;
        if (left > 8) block(std::integral_constant<int, BLK>{}, s0);
        else if (left > 4) block(std::integral_constant<int, 8>{}, s0);
        else block(std::integral_constant<int, 4>{}, s0);
    }
    if (valid) {
        float* cs = b.s1 + seq * p.seq_s + soff;
#pragma unroll
        for (int k = 0; k < 4; ++k) cs[k] = carry[k];
    }
}

extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_state_scan_f32(HelixScanParams p, HelixScanBuffers b) {
    state_scan_impl<false>(p, b);
}

extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_state_scan_y_f32(HelixScanParams p, HelixScanBuffers b) {
    state_scan_impl<true>(p, b);
}
