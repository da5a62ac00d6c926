// pass_c_f32.hip -- Pass C on fp32 MFMA (v_mfma_f32_32x32x2_f32).
//
// Reference counterpart: helix_chunk_out_f32 (src/kernels/
// helix_scan_multipass.metal:225-361):
//   G1  CB = C . B^T, causal tiles only, masked          (64 x 64, K = N)
//   G2  y_intra = (CB . exp(Lcum_t - Lcum_j)) . dtX      (64 x 64, K = 64)
//   G3  y_inter = C . S_init                             (64 x 64, K = N)
//   y   = y_intra + exp(Lcum_t) . y_inter
//
// MI355X layout: one workgroup per (seq, chunk, B/C group, head block). CB
// depends only on (seq, chunk, group), so G1 runs once and is reused by every
// head of the block instead of once per head. Then for each (head, P slab):
//   - S_init = R_c + exp(ld_c) S_seg(s) is assembled while staging (the two
//     halves of the two-level scan produced by Passes A and B),
//   - G3 accumulates straight into the output tile, the rows are scaled by
//     exp(Lcum_t), and G2 accumulates on top, so y leaves in one store.
// The chunk's C stays resident in LDS for every head; B is only needed for
// G1 and its LDS is recycled for S_init / dtX / M.
//
// Waves: wave w owns output tile (t block w >> 1, P block w & 1). G2 skips
// the all-zero upper tile (t block 0 only reads j < 32). Rows past tlen are
// zero in C and B and clamped in Lcum, so the ragged last chunk takes the
// same path (reference helix_pad.metal:1-46 does this with a padded copy;
// here the padding happens during staging).
#include "helix_common.h"

#include "pass_c_stage.h"

template <int NP>
__device__ __forceinline__ void chunk_out_f32_impl(const HelixScanParams& p, const HelixScanBuffers& b) {
    constexpr int KS  = NP > 128 ? 128 : NP;  // S_init staged in K blocks of KS
    constexpr int NKB = NP / KS;
    constexpr int RSC = NP + 1;               // odd strides: 32 rows x 1 column reads
    constexpr int RSS = KS + 1;
    constexpr int RSM = HELIX_CS + 1;
    constexpr int RSX = HELIX_HD;

    constexpr int SZ_C  = HELIX_CS * RSC;
    constexpr int SZ_B  = HELIX_CS * RSC;
    constexpr int SZ_S  = HELIX_HD * RSS;
    constexpr int SZ_X  = HELIX_CS * RSX;
    constexpr int SZ_M  = HELIX_CS * RSM;
    constexpr int SZ_R  = (SZ_B > SZ_S + SZ_X + SZ_M) ? SZ_B : (SZ_S + SZ_X + SZ_M);
    constexpr int OFF_R = SZ_C;
    constexpr int OFF_CB = OFF_R + SZ_R;
    constexpr int OFF_E  = OFF_CB + HELIX_CS * RSM;
    constexpr int TOTAL  = OFF_E + HELIX_CS;
    __shared__ __attribute__((aligned(16))) float lds[TOTAL];
    float* sC  = lds;
    float* sB  = lds + OFF_R;            // G1 only
    float* sS  = lds + OFF_R;            // S_init[p][k] block, after G1
    float* sX  = sS + SZ_S;              // dtX[j][p]
    float* sM  = sX + SZ_X;              // M[t][j] = CB[t][j] exp(Lcum_t - Lcum_j)
    float* sCB = lds + OFF_CB;           // masked CB[t][j]
    float* sE  = lds + OFF_E;            // exp(Lcum_t)

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = wave_uniform(), lo = lane & 31, hi = lane >> 5;

    // 1-D grid of n_cg * (n_group * n_hblk) * n_seq workgroups, chunk fastest
    // in the logical order so a segment's chunks (which share S_seg) and a
    // chunk's head blocks (which share B and C) stay on one XCD.
    const unsigned n_gh  = (unsigned)p.n_group * (unsigned)p.n_hblk;
    const unsigned total = (unsigned)p.n_cg * n_gh * (unsigned)p.n_seq;
    const unsigned wid   = xcd_logical_id(blockIdx.x, total);
    const int cg  = (int)(wid % (unsigned)p.n_cg);
    const int gh  = (int)((wid / (unsigned)p.n_cg) % n_gh);
    const int seq = (int)(wid / ((unsigned)p.n_cg * n_gh));
    const int g   = gh / p.n_hblk;
    const int hb  = gh % p.n_hblk;
    const int t0   = (p.chunk_base + cg) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const int N = p.d_state, P = p.head_dim;
    const int seg = cg / p.seg_len;
    const int cis = cg % p.seg_len;

    const int h_begin = g * p.heads_per_group + hb * p.hblk;
    const int h_end   = min(h_begin + p.hblk, (g + 1) * p.heads_per_group);
    if (h_begin >= h_end) return;

    // ---- stage C and B of this (seq, chunk, group) ---------------------------
    {
        float vc[16][NP / 64], vb[16][NP / 64];
        load_cb_rows<NP>(vc, vb, p, b, seq, g, t0, tlen, lane, wave);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int j = wave + 4 * i;
#pragma unroll
            for (int m = 0; m < NP / 64; ++m) {
                const int n = lane + 64 * m;
                const bool ok = j < tlen && n < N;
                sC[j * RSC + n] = ok ? vc[i][m] : 0.0f;
                sB[j * RSC + n] = ok ? vb[i][m] : 0.0f;
            }
        }
    }
    __syncthreads();

    // ---- G1: CB tiles (0,0), (1,0), (1,1) on waves 0..2 ----------------------
    if (wave < 3) {
        const int tb = wave == 0 ? 0 : 1;
        const int jb = wave == 2 ? 1 : 0;
        f32x16 acc = zero16();
#pragma unroll 8
        for (int s = 0; s < NP / 2; ++s) {
            const float av = sC[(tb * 32 + lo) * RSC + 2 * s + hi];
            const float bv = sB[(jb * 32 + lo) * RSC + 2 * s + hi];
            acc = mfma_f32(av, bv, acc);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = tb * 32 + acc_row(r, hi);
            const int j = jb * 32 + lo;
            sCB[t * RSM + j] = (j <= t) ? acc[r] : 0.0f;
        }
    }
    __syncthreads();

    const int tb = wave >> 1, pb = wave & 1;
    const float* __restrict__ x_s  = b.x + seq * p.seq_x;
    const float* __restrict__ dt_s = b.dt + seq * p.seq_dt;
    const float* __restrict__ sl_s = static_cast<const float*>(b.s_local) + seq * p.sl_seq + (long long)cg * p.sl_cg;
    const float* __restrict__ sg_s = b.s_seg + seq * p.sg_seq + (long long)seg * p.sg_seg;

    const int n_items = (h_end - h_begin) * p.n_pslab;
    StageC<NP, float> st;
    load_stage_c<NP, float>(st, p, b, x_s, dt_s, sl_s, sg_s, seq, cg, t0, tlen, cis, h_begin, 0,
                            lane, wave);

    for (int item = 0; item < n_items; ++item) {
        const int h    = h_begin + item / p.n_pslab;
        const int slab = item % p.n_pslab;
        const int p0 = slab * HELIX_HD;
        const int pw = min(HELIX_HD, P - p0);

        const float dtv = keep_if_lt(helix_dt(p, st.dtraw), lane, tlen);
        const double lcum = wave_incl_sum((double)st.A * (double)dtv);
        const float es = expf(st.ld);

        // dtX[j][p] (dtv_j = 0 past tlen)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int j = 16 * wave + i;
            sX[j * RSX + lane] = keep_if_lt(bcast(dtv, j) * st.x[i], lane, pw);
        }
        // M[t][j] for this head; lane = j, so Lcum_j is this lane's own.
#pragma unroll 4
        for (int i = 0; i < 16; ++i) {
            const int t = wave + 4 * i;
            const double lt = bcast(lcum, t);
            sM[t * RSM + lane] = keep_if_le(sCB[t * RSM + lane] * exp_diff(lt, lcum), lane, t);
        }
        if (wave == 0) sE[lane] = expf((float)lcum);

        f32x16 acc = zero16();
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            // S_init[p][k] = R_c + exp(ld_c) S_seg, zero past the slab and d_state.
#pragma unroll
            for (int pt = 0; pt < 2; ++pt) {
#pragma unroll
                for (int nt = kb * (KS / 32); nt < (kb + 1) * (KS / 32); ++nt) {
                    const int m  = pt * (NP / 32) + nt;
                    const int pr = pt * 32 + lo;
                    const int n  = nt * 32 + 8 * wave + 4 * hi;
                    const f32x4 g = unit_to_f32(st.sg[m]), l = unit_to_f32(st.sl[m]);
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        sS[pr * RSS + (n - kb * KS) + k] = keep_if_lt2(es * g[k] + l[k], pr, pw, n, N);
                }
            }
            __syncthreads();
            // The next item's inputs travel during the last block's GEMMs.
            if (kb + 1 == NKB && item + 1 < n_items) {
                const int hn = h_begin + (item + 1) / p.n_pslab;
                load_stage_c<NP, float>(st, p, b, x_s, dt_s, sl_s, sg_s, seq, cg, t0, tlen, cis, hn,
                                        (item + 1) % p.n_pslab, lane, wave);
            }
            // G3 partial: y += C[:, kblock] . S_init[kblock, :]
#pragma unroll 8
            for (int s = 0; s < KS / 2; ++s) {
                const float av = sC[(tb * 32 + lo) * RSC + kb * KS + 2 * s + hi];
                const float bv = sS[(pb * 32 + lo) * RSS + 2 * s + hi];
                acc = mfma_f32(av, bv, acc);
            }
            if (kb + 1 < NKB) __syncthreads();
        }

        // rows scaled by exp(Lcum_t), then G2 on top.
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] *= sE[tb * 32 + acc_row(r, hi)];
        const int ksteps = 16 * (tb + 1);
#pragma unroll 8
        for (int s = 0; s < ksteps; ++s) {
            const int j = 2 * s + hi;
            const float av = sM[(tb * 32 + lo) * RSM + j];
            const float bv = sX[j * RSX + pb * 32 + lo];
            acc = mfma_f32(av, bv, acc);
        }

        store_y_tile(acc, p, b, seq, h, t0, tlen, p0, pw, tb, pb, lo, hi);
        __syncthreads();
    }
}

#define HELIX_PASS_C_F32(NP)                                                                    \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_out_f32_n##NP(            \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_out_f32_impl<NP>(p, b);                                                           \
    }

// The fp32 path at d_state 256, where the bf16x6 Pass C does not fit its LDS.
HELIX_PASS_C_F32(256)
