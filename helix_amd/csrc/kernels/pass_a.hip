// pass_a.hip -- Pass A: chunk-state GEMM on fp32 MFMA, walked over a segment.
//
// Reference counterpart: helix_chunk_state_f32 (src/kernels/
// helix_scan_multipass.metal:51-149), which computes one chunk's
//     dS[n][c] = sum_j B[j][n] * exp(L_end - Lcum_j) * dt_j * x[j][c]
// per threadgroup and leaves the chunk-to-chunk recurrence to Pass B.
//
// Here one workgroup owns (seq, segment, head, 64-wide P slab) and walks the
// segment's chunks in order, keeping the running state in MFMA accumulators:
//     store R_c            (state entering chunk c from this segment; c > first)
//     R <- exp(L_end_c) R + B_c^T . (decay . dt . x)_c
// so the per-chunk states reach HBM once (s_local) instead of three times,
// and only the segment aggregates D_s go through Pass B.
//
// Tiling: the workgroup computes R[n][p] (N x 64) with v_mfma_f32_32x32x2_f32,
// M = n, N = p, K = token. Wave w owns P tile (w & 1) and N tiles
// (w >> 1) + 2i, so the dtXs operand is loaded once per K step and reused
// across its N tiles. Both operands come from LDS in their natural row-major
// staging (dtXs[j][p], B[j][n]); the result registers store as the scratch
// tile's units (four consecutive n of one p per lane).
#include "helix_common.h"

// Store this wave's accumulator tiles (R[n][p] tiles (nt0 + 2i, pt)) into a
// slab tile (helix_params.h layout): result registers 4 r4 .. 4 r4 + 3 are
// one unit, so each lane writes 16 (fp32) or 8 (bf16) bytes per four registers
// and a wave 1 KiB / 512 B contiguous. No guards: the whole padded tile is
// written (here the padding of a partial slab or of d_state < np holds zeros,
// because the matching dtXs columns and B columns were staged as zeros).
template <int NP, bool SBF>
__device__ __forceinline__ void store_state_tiles(const f32x16* acc, helix_rsrc dst, int pt, int nt0,
                                                  int lane) {
    constexpr int NT = NP / 32;
    constexpr int NTW = NP / 64;
#pragma unroll
    for (int i = 0; i < NTW; ++i) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int u = tile_unit(NT, pt, nt0 + 2 * i, r4, 0);
            const float v0 = acc[i][4 * r4], v1 = acc[i][4 * r4 + 1];
            const float v2 = acc[i][4 * r4 + 2], v3 = acc[i][4 * r4 + 3];
            if (SBF)
                buf_store_unit<__bf16>(dst, v0, v1, v2, v3, lane, u);
            else
                buf_store_unit<float>(dst, v0, v1, v2, v3, lane, u);
        }
    }
}

// Registers holding one chunk's global inputs for this thread, so the loads
// of chunk c+1 are in flight while chunk c runs on the MFMA pipe. Every load
// reads an in-bounds address (rows clamped to the last valid token, columns to
// the last valid index) and the tile masks are applied afterwards: a guarded
// load would compile to a branch and a wait per element.
template <int NP>
struct StageA {
    float dtraw;
    float x[16];
    float b[16][NP / 64];
};

template <int NP>
__device__ __forceinline__ void load_stage_a(StageA<NP>& st, const HelixScanParams& p,
                                             const float* __restrict__ dt_h,
                                             const float* __restrict__ x_h,
                                             const float* __restrict__ B_g, int c, int lane,
                                             int wave, int pw, int N) {
    const int t0   = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    // One buffer resource per tensor, based at the chunk's first token; the
    // host keeps a chunk's extent below 2 GiB so the offsets fit 32 bits.
    const int sdt = (int)p.s_dt[0], sx0 = (int)p.s_x[0], sx2 = (int)p.s_x[2], sb0 = (int)p.s_b[0];
    const helix_rsrc rdt = make_rsrc(dt_h + (long long)t0 * p.s_dt[0], ((tlen - 1) * sdt + 1) * 4u);
    const helix_rsrc rx  = make_rsrc(x_h + (long long)t0 * p.s_x[0], ((tlen - 1) * sx0 + (pw - 1) * sx2 + 1) * 4u);
    const helix_rsrc rb  = make_rsrc(B_g + (long long)t0 * p.s_b[0], ((tlen - 1) * sb0 + N) * 4u);
    st.dtraw = buf_elem<float>(rdt, min(lane, tlen - 1) * sdt, 0);
    const int xc = min(lane, pw - 1) * sx2;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int jr = min(wave + 4 * i, tlen - 1);
        st.x[i] = buf_elem<float>(rx, xc, jr * sx0);
#pragma unroll
        for (int m = 0; m < NP / 64; ++m) st.b[i][m] = buf_elem<float>(rb, min(lane + 64 * m, N - 1), jr * sb0);
    }
}

// MODE 0: store R_c as fp32 (fp32 path); 1: as bf16 (bf16 chunk-parallel
// Pass C); 2: store nothing per chunk, only the segment aggregate D_s (the
// chunk-walking Pass C recomputes R_c itself).
template <int NP, int MODE>
__device__ __forceinline__ void chunk_state_impl(const HelixScanParams& p, const HelixScanBuffers& b) {
    constexpr bool SBF = MODE == 1;
    constexpr int NTW = NP / 64;      // N tiles per wave (NP/32 tiles over 2 waves)
    constexpr int RSX = HELIX_HD;     // row stride of dtXs
    constexpr int RSB = NP;           // row stride of B
    __shared__ __attribute__((aligned(16))) float sX[HELIX_CS * RSX];
    __shared__ __attribute__((aligned(16))) float sB[HELIX_CS * RSB];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = wave_uniform(), lo = lane & 31, hi = lane >> 5;

    const int seg  = blockIdx.x;
    const int h    = blockIdx.y;
    const int slab = blockIdx.z % p.n_pslab;
    const int seq  = blockIdx.z / p.n_pslab;
    const int p0   = slab * HELIX_HD;
    const int pw   = min(HELIX_HD, p.head_dim - p0);
    const int N    = p.d_state;
    const int g    = h / p.heads_per_group;

    const int c_begin = seg * p.seg_len;
    const int c_end   = min(c_begin + p.seg_len, p.n_cg);
    if (c_begin >= c_end) return;

    const float A_h = b.A[(long long)h * p.s_a];
    const float* __restrict__ dt_h = b.dt + seq * p.seq_dt + h * p.s_dt[1];
    const float* __restrict__ x_h  = b.x + seq * p.seq_x + h * p.s_x[1] + p0 * p.s_x[2];
    const float* __restrict__ B_g  = b.B + seq * p.seq_b + g * p.s_b[1];

    const long long tile_off = state_tile_off(p, h, slab);
    const unsigned tile_elems = 64u * NP;

    const int pt  = wave & 1;
    const int nt0 = wave >> 1;

    f32x16 acc[NTW];
#pragma unroll
    for (int i = 0; i < NTW; ++i) acc[i] = zero16();
    float lam = 0.0f;  // log-decay accumulated over this segment before chunk c

    StageA<NP> st;
    load_stage_a<NP>(st, p, dt_h, x_h, B_g, c_begin, lane, wave, pw, N);

    for (int c = c_begin; c < c_end; ++c) {
        const int t0   = (p.chunk_base + c) * HELIX_CS;
        const int tlen = min(HELIX_CS, p.n_tok - t0);

        // Decay preamble from the staged dt (dtv = 0 past tlen).
        const float dtv = lane < tlen ? helix_dt(p, st.dtraw) : 0.0f;
        const double lcum = wave_incl_sum((double)A_h * (double)dtv);
        const double lend = __shfl(lcum, 63, 64);
        const float cf = (lane < tlen) ? exp_diff(lend, lcum) * dtv : 0.0f;
        if (MODE == 2 && b.pre && wave == 0 && slab == 0)
            store_decay_record(p, b, seq, c, h, lane, tlen, dtv, lcum, lend);

        // dtXs[j][p] = exp(L_end - Lcum_j) dt_j x[j][p] (cf_j = 0 past tlen);
        // B[j][n] zero past tlen and d_state.
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int j = wave + 4 * i;
            const float cj = bcast(cf, j);
            sX[j * RSX + lane] = lane < pw ? cj * st.x[i] : 0.0f;
#pragma unroll
            for (int m = 0; m < NP / 64; ++m) {
                const int n = lane + 64 * m;
                sB[j * RSB + n] = (j < tlen && n < N) ? st.b[i][m] : 0.0f;
            }
        }

        if (MODE != 2 && c > c_begin) {
            const long long off = seq * p.sl_seq + (long long)c * p.sl_cg + tile_off;
            const void* dst = SBF ? (const void*)(static_cast<const __bf16*>(b.s_local) + off)
                                  : (const void*)(static_cast<const float*>(b.s_local) + off);
            store_state_tiles<NP, SBF>(acc, make_rsrc(dst, tile_elems * (SBF ? 2u : 4u)), pt, nt0, lane);
        }
        if (slab == 0 && tid == 0) b.ld[seq * p.ld_seq + (long long)c * p.n_head + h] = lam;
        __syncthreads();

        // Next chunk's inputs travel while this chunk's GEMM runs.
        if (c + 1 < c_end) load_stage_a<NP>(st, p, dt_h, x_h, B_g, c + 1, lane, wave, pw, N);

        const float a_c = expf((float)lend);
#pragma unroll
        for (int i = 0; i < NTW; ++i) acc[i] *= a_c;

        // R[n][p] += sum_j B[j][n] dtXs[j][p]: A operand B (M = n), B operand
        // dtXs (N = p), K = token.
#pragma unroll 8
        for (int s = 0; s < HELIX_CS / 2; ++s) {
            const int j = 2 * s + hi;
            const float xv = sX[j * RSX + pt * 32 + lo];
#pragma unroll
            for (int i = 0; i < NTW; ++i) {
                const float bv = sB[j * RSB + (nt0 + 2 * i) * 32 + lo];
                acc[i] = mfma_f32(bv, xv, acc[i]);
            }
        }
        lam += (float)lend;
        __syncthreads();
    }

    const float* sg = b.s_seg + seq * p.sg_seq + (long long)seg * p.sg_seg + tile_off;
    store_state_tiles<NP, false>(acc, make_rsrc(sg, tile_elems * 4u), pt, nt0, lane);
    if (slab == 0 && tid == 0) b.segld[seq * p.sd_seq + (long long)seg * p.n_head + h] = lam;
}

#define HELIX_PASS_A(NP)                                                                        \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_state_f32_n##NP(          \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_state_impl<NP, 0>(p, b);                                                          \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_state_sbf_n##NP(          \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_state_impl<NP, 1>(p, b);                                                          \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_state_agg_n##NP(          \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_state_impl<NP, 2>(p, b);                                                          \
    }

HELIX_PASS_A(64)
HELIX_PASS_A(128)
HELIX_PASS_A(256)
