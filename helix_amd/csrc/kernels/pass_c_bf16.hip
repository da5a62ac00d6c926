// pass_c_bf16.hip -- Pass C on bf16 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Reference counterpart: helix_chunk_out_mpp_impl<K> (src/kernels/mpp/
// helix_scan_mpp.metal:54-232): same G1/G2/G3 algebra as the fp32 Pass C with
// bf16 GEMM operands and fp32 accumulators; Lcum, exp, the carried state and
// the output stay fp32.
//
// The reference needs a separate cast pass (helix_cast.metal:19-46) to give
// MPP dense bf16 copies of B and C in device memory. Here B and C are read
// once in fp32 and rounded to bf16 (round-to-nearest-even) while they are
// staged into LDS, so the cast costs no extra HBM pass; rows past the end of
// the sequence are staged as zeros, which is what the cast pass's padding did.
//
// Every operand is stored k-contiguous in LDS so each lane fetches its eight
// bf16 K values with one 16-byte read:
//   C[t][n], B[j][n]   (K = n for G1 and G3)
//   M[t][j], dtX^T[p][j]  (K = j for G2)
//   S^T[p][n]          (K = n for G3; s_local is already [P][N])
#include "helix_common.h"

#include "pass_c_stage.h"

template <int NP>
__device__ __forceinline__ void chunk_out_bf16_impl(const HelixScanParams& p, const HelixScanBuffers& b) {
    constexpr int RS  = NP + 8;          // bf16 row stride of C, B, S^T (16-byte aligned rows)
    constexpr int RSJ = HELIX_CS + 8;    // bf16 row stride of M and dtX^T
    constexpr int RSCB = HELIX_CS + 1;   // fp32 row stride of CB

    __shared__ __attribute__((aligned(16))) __bf16 sC[HELIX_CS * RS];
    __shared__ __attribute__((aligned(16))) __bf16 sBS[HELIX_CS * RS];   // B for G1, then S^T
    __shared__ __attribute__((aligned(16))) __bf16 sM[HELIX_CS * RSJ];
    __shared__ __attribute__((aligned(16))) __bf16 sXt[HELIX_HD * RSJ];
    __shared__ __attribute__((aligned(16))) float sCB[HELIX_CS * RSCB];
    __shared__ __attribute__((aligned(16))) float sE[HELIX_CS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = wave_uniform(), lo = lane & 31, hi = lane >> 5;

    // 1-D grid of n_cg * (n_group * n_hblk) * n_seq workgroups, chunk fastest
    // in the logical order so a segment's chunks (which share S_seg) and a
    // chunk's head blocks (which share B and C) stay on one XCD.
    const unsigned n_gh  = (unsigned)(p.n_group * p.n_hblk);
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

    // ---- stage C and B as bf16 ----------------------------------------------
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
                sC[j * RS + n]  = to_bf16(ok ? vc[i][m] : 0.0f);
                sBS[j * RS + n] = to_bf16(ok ? vb[i][m] : 0.0f);
            }
        }
    }
    __syncthreads();

    // ---- G1: CB tiles (0,0), (1,0), (1,1) on waves 0..2 ----------------------
    if (wave < 3) {
        const int tb = wave == 0 ? 0 : 1;
        const int jb = wave == 2 ? 1 : 0;
        f32x16 acc = zero16();
#pragma unroll 4
        for (int s = 0; s < NP / 16; ++s) {
            const bf16x8 av = *reinterpret_cast<const bf16x8*>(&sC[(tb * 32 + lo) * RS + 16 * s + 8 * hi]);
            const bf16x8 bv = *reinterpret_cast<const bf16x8*>(&sBS[(jb * 32 + lo) * RS + 16 * s + 8 * hi]);
            acc = mfma_bf16(av, bv, acc);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = tb * 32 + acc_row(r, hi);
            const int j = jb * 32 + lo;
            sCB[t * RSCB + j] = (j <= t) ? acc[r] : 0.0f;
        }
    }
    __syncthreads();

    const int tb = wave >> 1, pb = wave & 1;
    const float* __restrict__ x_s  = b.x + seq * p.seq_x;
    const float* __restrict__ dt_s = b.dt + seq * p.seq_dt;
    const __bf16* __restrict__ sl_s = static_cast<const __bf16*>(b.s_local) + seq * p.sl_seq + (long long)cg * p.sl_cg;
    const float* __restrict__ sg_s = b.s_seg + seq * p.sg_seq + (long long)seg * p.sg_seg;

    const int n_items = (h_end - h_begin) * p.n_pslab;
    StageC<NP, __bf16> st;
    load_stage_c<NP, __bf16>(st, p, b, x_s, dt_s, sl_s, sg_s, seq, cg, t0, tlen, cis, h_begin, 0,
                             lane, wave);

    for (int item = 0; item < n_items; ++item) {
        const int h    = h_begin + item / p.n_pslab;
        const int slab = item % p.n_pslab;
        const int p0 = slab * HELIX_HD;
        const int pw = min(HELIX_HD, P - p0);

        const float dtv = keep_if_lt(helix_dt(p, st.dtraw), lane, tlen);
        const double lcum = wave_incl_sum((double)st.A * (double)dtv);
        const float es = expf(st.ld);

        // dtX^T[p][j] (bf16); dtv_j = 0 past tlen. Wave w holds tokens
        // 16w .. 16w+15 of its lane's channel: two 16-byte LDS writes.
        {
            bf16x8 v0, v1;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v0[i] = to_bf16(keep_if_lt(bcast(dtv, 16 * wave + i) * st.x[i], lane, pw));
                v1[i] = to_bf16(keep_if_lt(bcast(dtv, 16 * wave + 8 + i) * st.x[8 + i], lane, pw));
            }
            *reinterpret_cast<bf16x8*>(&sXt[lane * RSJ + 16 * wave]) = v0;
            *reinterpret_cast<bf16x8*>(&sXt[lane * RSJ + 16 * wave + 8]) = v1;
        }
        // M[t][j] = CB[t][j] exp(Lcum_t - Lcum_j) (bf16), zero above the
        // diagonal. Only the three causal 32 x 32 blocks are built, in 48 row
        // steps: steps 0..15 pair row s (lanes 0-31) with row s + 16 (lanes
        // 32-63) of block (0,0), columns j = lo; steps 16..47 are the full rows
        // t = s + 16 of blocks (1,0) and (1,1), j = lane. Wave w takes steps
        // w + 4k, so k < 4 are the paired steps for every wave.
        {
            const double l_lo = __shfl(lcum, lo, 64);    // Lcum of token lane % 32
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int s = wave + 4 * k;
                const int t = s + 16 * hi;
                const double lt = pick_hi(bcast(lcum, s), bcast(lcum, s + 16), hi);
                const float m = keep_if_le(sCB[t * RSCB + lo] * exp2_diff(lt, l_lo), lo, t);
                sM[t * RSJ + lo] = to_bf16(m);
            }
#pragma unroll 4
            for (int k = 4; k < 12; ++k) {
                const int t = wave + 4 * k + 16;
                const double lt = bcast(lcum, t);
                const float m = keep_if_le(sCB[t * RSCB + lane] * exp2_diff(lt, lcum), lane, t);
                sM[t * RSJ + lane] = to_bf16(m);
            }
        }
        if (wave == 0) sE[lane] = expf((float)lcum);
        // S^T[p][n] = R_c + exp(ld_c) S_seg, in fp32 then rounded to bf16: four
        // consecutive n per unit, one 8-byte LDS write.
#pragma unroll
        for (int m = 0; m < NP / 16; ++m) {
            const int pr = (m / (NP / 32)) * 32 + lo;
            const int n  = (m % (NP / 32)) * 32 + 8 * wave + 4 * hi;
            const f32x4 g = unit_to_f32(st.sg[m]), l = unit_to_f32(st.sl[m]);
            bf16x4 v;
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = to_bf16(keep_if_lt2(es * g[k] + l[k], pr, pw, n, N));
            *reinterpret_cast<bf16x4*>(&sBS[pr * RS + n]) = v;
        }
        __syncthreads();
        if (item + 1 < n_items) {
            const int hn = h_begin + (item + 1) / p.n_pslab;
            load_stage_c<NP, __bf16>(st, p, b, x_s, dt_s, sl_s, sg_s, seq, cg, t0, tlen, cis, hn,
                                     (item + 1) % p.n_pslab, lane, wave);
        }

        // G3, row scale, G2.
        f32x16 acc = zero16();
#pragma unroll 4
        for (int s = 0; s < NP / 16; ++s) {
            const bf16x8 av = *reinterpret_cast<const bf16x8*>(&sC[(tb * 32 + lo) * RS + 16 * s + 8 * hi]);
            const bf16x8 bv = *reinterpret_cast<const bf16x8*>(&sBS[(pb * 32 + lo) * RS + 16 * s + 8 * hi]);
            acc = mfma_bf16(av, bv, acc);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] *= sE[tb * 32 + acc_row(r, hi)];
        for (int s = 0; s < 2 * (tb + 1); ++s) {
            const bf16x8 av = *reinterpret_cast<const bf16x8*>(&sM[(tb * 32 + lo) * RSJ + 16 * s + 8 * hi]);
            const bf16x8 bv = *reinterpret_cast<const bf16x8*>(&sXt[(pb * 32 + lo) * RSJ + 16 * s + 8 * hi]);
            acc = mfma_bf16(av, bv, acc);
        }

        store_y_tile(acc, p, b, seq, h, t0, tlen, p0, pw, tb, pb, lo, hi);
        __syncthreads();
    }
}

#define HELIX_PASS_C_BF16(NP)                                                                   \
    extern "C" __global__ __launch_bounds__(HELIX_WG) __attribute__((amdgpu_waves_per_eu(2))) void helix_chunk_out_bf16_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_out_bf16_impl<NP>(p, b);                                                          \
    }

HELIX_PASS_C_BF16(64)
HELIX_PASS_C_BF16(128)
HELIX_PASS_C_BF16(256)
