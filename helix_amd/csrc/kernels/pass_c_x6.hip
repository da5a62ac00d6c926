// pass_c_x6.hip -- Pass C of the fp32 path on bf16x6 split products.
//
// Same computation as pass_c_f32.hip (reference helix_chunk_out_f32,
// src/kernels/helix_scan_multipass.metal:225-361):
//   G1  CB = C . B^T, causal tiles only, masked          (64 x 64, K = N)
//   G2  y_intra = (CB . exp(Lcum_t - Lcum_j)) . dtX      (64 x 64, K = 64)
//   G3  y_inter = C . S_init                             (64 x 64, K = N)
//   y   = y_intra + exp(Lcum_t) . y_inter
// with every GEMM on v_mfma_f32_32x32x16_bf16 over operands split into three
// bf16 parts (six products per fp32 product, helix_common.h), which keeps
// fp32 accuracy at 16x the fp32 matrix issue rate.
//
// Workgroup: (seq, chunk, B/C group, head block), as in pass_c_f32.hip; G1
// runs once and CB is reused by every head of the block. All split operands
// live in LDS k-contiguous (x6_off swizzle):
//   C planes     [3][64 t][NP n]    resident for the whole workgroup
//   B planes     [3][64 j][NP n]    G1 only; the region is then reused for
//   S^T planes   [3][64 p][NP n]    S_init of the current (head, slab) item
//   M planes     [3][64 t][64 j]    CB[t][j] exp(Lcum_t - Lcum_j), j <= t
//   dtX^T planes [3][64 p][64 j]
//   CB           fp32, the three causal 32 x 32 blocks
// At NP = 128 that is 158 KiB, one workgroup per CU. Wave w owns output tile
// (t block w >> 1, P block w & 1).
//
// Masks: C is zeroed past tlen and d_state, which is all G1 and G3 need (B
// rows past tlen then only meet dtX columns that are zero, as dt is; padding
// of S_init only meets zero columns of C). dtX is zero past tlen through
// dt. Channels past the slab only reach output columns that are not stored.
#include "helix_common.h"

#include "pass_c_stage.h"

template <int NP>
__device__ __forceinline__ void chunk_out_x6_impl(const HelixScanParams& p, const HelixScanBuffers& b) {
    constexpr int NCH = NP / 8;                      // 16-byte chunks per C / B / S^T row
    constexpr int SZ_C  = 3 * HELIX_CS * NP;         // bf16 elements
    constexpr int SZ_S  = 3 * HELIX_HD * NP;
    constexpr int SZ_M  = 3 * HELIX_CS * HELIX_CS;
    constexpr int SZ_X  = 3 * HELIX_HD * HELIX_CS;
    constexpr int CBS   = 32;                        // fp32 row stride of a CB block
    __shared__ __attribute__((aligned(16))) __bf16 sC[SZ_C];
    __shared__ __attribute__((aligned(16))) __bf16 sR[SZ_S + SZ_M + SZ_X];   // B planes during G1
    __shared__ __attribute__((aligned(16))) float sCB[3 * 32 * CBS];
    __shared__ __attribute__((aligned(16))) float sE[HELIX_CS];
    __shared__ __attribute__((aligned(16))) double sL[4][HELIX_CS];         // per-wave Lcum copy
    __bf16* const sB = sR;
    __bf16* const sS = sR;
    __bf16* const sM = sR + SZ_S;
    __bf16* const sX = sR + SZ_S + SZ_M;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = wave_uniform(), lo = lane & 31, hi = lane >> 5;

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

    // ---- stage C (masked) and B as split planes --------------------------------
    // Lane (q = lane % NCH, rr = lane / NCH) loads 32 bytes (state indices
    // 8q .. 8q+7) of rows 16 wave + (64/NCH) k + rr, one chunk per row.
    {
        constexpr int RPI = 64 / NCH;                // rows per wave instruction
        const int q = lane % NCH, rr = lane / NCH;
        const int sc0 = (int)p.s_c[0], sb0 = (int)p.s_b[0];
        const helix_rsrc rc = make_rsrc(b.C + seq * p.seq_c + g * p.s_c[1] + (long long)t0 * p.s_c[0],
                                        ((tlen - 1) * sc0 + N) * 4u);
        const helix_rsrc rb = make_rsrc(b.B + seq * p.seq_b + g * p.s_b[1] + (long long)t0 * p.s_b[0],
                                        ((tlen - 1) * sb0 + N) * 4u);
        const int n0 = min(8 * q, N - 8);            // d_state % 8 == 0: a run is all in or all out
        float vc[16 / RPI][8], vb[16 / RPI][8];
#pragma unroll
        for (int k = 0; k < 16 / RPI; ++k) {
            const int j = 16 * wave + RPI * k + rr;
            const int off = (n0 + min(j, tlen - 1) * sc0) * 4;
            const int offb = (n0 + min(j, tlen - 1) * sb0) * 4;
            const u32x4 c0 = __builtin_amdgcn_raw_buffer_load_b128(rc, off, 0, 0);
            const u32x4 c1 = __builtin_amdgcn_raw_buffer_load_b128(rc, off + 16, 0, 0);
            const u32x4 b0 = __builtin_amdgcn_raw_buffer_load_b128(rb, offb, 0, 0);
            const u32x4 b1 = __builtin_amdgcn_raw_buffer_load_b128(rb, offb + 16, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vc[k][e] = as_f32(c0[e]);
                vc[k][4 + e] = as_f32(c1[e]);
                vb[k][e] = as_f32(b0[e]);
                vb[k][4 + e] = as_f32(b1[e]);
            }
        }
#pragma unroll
        for (int k = 0; k < 16 / RPI; ++k) {
            const int j = 16 * wave + RPI * k + rr;
#pragma unroll
            for (int e = 0; e < 8; ++e) vc[k][e] = keep_if_lt2(vc[k][e], j, tlen, 8 * q, N);
            x6_write8<HELIX_CS, NCH>(sC, j, q, vc[k]);
            x6_write8<HELIX_CS, NCH>(sB, j, q, vb[k]);
        }
    }
    __syncthreads();

    // ---- G1: CB blocks (0,0), (1,0), (1,1) on waves 0..2 ------------------------
    if (wave < 3) {
        const int tb = wave == 0 ? 0 : 1;
        const int jb = wave == 2 ? 1 : 0;
        f32x16 acc = zero16();
#pragma unroll 2
        for (int s = 0; s < NP / 16; ++s) {
            bf16x8 av[3], bv[3];
            x6_read<HELIX_CS, NCH>(sC, tb * 32 + lo, 2 * s + hi, av);
            x6_read<HELIX_CS, NCH>(sB, jb * 32 + lo, 2 * s + hi, bv);
            acc = mfma_x6(av, bv, acc);
        }
        float* blk = sCB + wave * 32 * CBS;          // block index = wave
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int tt = acc_row(r, hi);
            const float v = acc[r];
            blk[tt * CBS + lo] = keep_if_le(v, jb * 32 + lo, tb * 32 + tt);
        }
    }
    __syncthreads();

    const int tb = wave >> 1, pb = wave & 1;
    const float* __restrict__ x_s  = b.x + seq * p.seq_x;
    const float* __restrict__ dt_s = b.dt + seq * p.seq_dt;
    const float* __restrict__ sl_s = static_cast<const float*>(b.s_local) + seq * p.sl_seq + (long long)cg * p.sl_cg;
    const float* __restrict__ sg_s = b.s_seg + seq * p.sg_seq + (long long)seg * p.sg_seg;

    const int n_items = (h_end - h_begin) * p.n_pslab;
    // Pass A's decay records replace the per-item softplus and fp64 scan.
    StageC<NP, float, true> st;
    load_stage_c<NP, float, true>(st, p, b, x_s, dt_s, sl_s, sg_s, seq, cg, t0, tlen, cis, h_begin, 0, lane, wave);

    for (int item = 0; item < n_items; ++item) {
        const int h    = h_begin + item / p.n_pslab;
        const int slab = item % p.n_pslab;
        const int p0 = slab * HELIX_HD;
        const int pw = min(HELIX_HD, P - p0);

        // Record of token lane: dt (0 past tlen), exp(Lcum), Lcum (fp64).
        const float dtv = as_f32(st.rec[0]);
        const double lcum = __builtin_bit_cast(double, (unsigned long long)st.rec[2] |
                                                           ((unsigned long long)st.rec[3] << 32));
        const float es = expf(st.ld);
        sL[wave][lane] = lcum;                       // this wave's own copy
        if (wave == 0) sE[lane] = as_f32(st.rec[1]);

        // dtX^T[p][j], row p = lane, tokens 16 wave .. 16 wave + 15.
        {
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = bcast(dtv, 16 * wave + i) * st.x[i];
            x6_write8<HELIX_HD, 8>(sX, lane, 2 * wave, v);
            x6_write8<HELIX_HD, 8>(sX, lane, 2 * wave + 1, v + 8);
        }
        // S_init^T[p][n] = R_c + exp(ld_c) S_seg, unit m of this wave: rows
        // p = (m / NT) 32 + lo, n = (m % NT) 32 + 8 wave + 4 hi + 0..3, i.e.
        // half `hi` of chunk (m % NT) 4 + wave. Two units (the two halves, from
        // lanes lo and lo + 32) are not in one lane, so each lane writes its
        // half of the three planes directly.
#pragma unroll
        for (int m = 0; m < NP / 16; ++m) {
            const int pr = (m / (NP / 32)) * 32 + lo;
            const int ch = (m % (NP / 32)) * 4 + wave;
            const f32x4 gv = unit_to_f32(st.sg[m]), lv = unit_to_f32(st.sl[m]);
            u32x2 q0, q1, q2;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                unsigned w0, w1, w2;
                split3_pair(es * gv[2 * e] + lv[2 * e], es * gv[2 * e + 1] + lv[2 * e + 1], w0, w1, w2);
                q0[e] = w0;
                q1[e] = w1;
                q2[e] = w2;
            }
            *reinterpret_cast<u32x2*>(&sS[x6_off<HELIX_HD, NCH>(0, pr, ch) + 4 * hi]) = q0;
            *reinterpret_cast<u32x2*>(&sS[x6_off<HELIX_HD, NCH>(1, pr, ch) + 4 * hi]) = q1;
            *reinterpret_cast<u32x2*>(&sS[x6_off<HELIX_HD, NCH>(2, pr, ch) + 4 * hi]) = q2;
        }
        // M[t][j] = CB[t][j] exp(Lcum_t - Lcum_j) for the chunks G2 reads:
        // rows 0..31 chunks 0..3 (jobs 0..127), rows 32..63 chunks 0..7 (jobs
        // 128..383); each job is eight consecutive j of one row.
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int job = tid + 256 * k;
            if (job < 384) {
                const int t  = job < 128 ? (job >> 2) : 32 + ((job - 128) >> 3);
                const int ch = job < 128 ? (job & 3) : ((job - 128) & 7);
                const int jb = ch >> 2;                      // CB block column
                const float* cbrow = sCB + ((t >= 32) + jb) * 32 * CBS + (t & 31) * CBS + 8 * (ch & 3);
                const f32x4 c0 = *reinterpret_cast<const f32x4*>(cbrow);
                const f32x4 c1 = *reinterpret_cast<const f32x4*>(cbrow + 4);
                const double lt = sL[wave][t];
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int j = 8 * ch + e;
                    const float cb = e < 4 ? c0[e] : c1[e - 4];
                    v[e] = keep_if_le(cb * exp2_diff(lt, sL[wave][j]), j, t);
                }
                x6_write8<HELIX_CS, 8>(sM, t, ch, v);
            }
        }
        __syncthreads();
        // The register stage is free: the next item's inputs travel during the GEMMs.
        if (item + 1 < n_items) {
            const int hn = h_begin + (item + 1) / p.n_pslab;
            load_stage_c<NP, float, true>(st, p, b, x_s, dt_s, sl_s, sg_s, seq, cg, t0, tlen, cis, hn,
                                    (item + 1) % p.n_pslab, lane, wave);
        }

        // G3, row scale, G2.
        f32x16 acc = zero16();
#pragma unroll 2
        for (int s = 0; s < NP / 16; ++s) {
            bf16x8 av[3], bv[3];
            x6_read<HELIX_CS, NCH>(sC, tb * 32 + lo, 2 * s + hi, av);
            x6_read<HELIX_HD, NCH>(sS, pb * 32 + lo, 2 * s + hi, bv);
            acc = mfma_x6(av, bv, acc);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] *= sE[tb * 32 + acc_row(r, hi)];
        for (int s = 0; s < 2 * (tb + 1); ++s) {
            bf16x8 av[3], bv[3];
            x6_read<HELIX_CS, 8>(sM, tb * 32 + lo, 2 * s + hi, av);
            x6_read<HELIX_HD, 8>(sX, pb * 32 + lo, 2 * s + hi, bv);
            acc = mfma_x6(av, bv, acc);
        }

        store_y_tile(acc, p, b, seq, h, t0, tlen, p0, pw, tb, pb, lo, hi);
        __syncthreads();
    }
}

#define HELIX_PASS_C_X6(NP)                                                                     \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_out_x6_n##NP(             \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_out_x6_impl<NP>(p, b);                                                            \
    }

HELIX_PASS_C_X6(64)
HELIX_PASS_C_X6(128)
