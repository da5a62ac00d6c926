// pass_c_walk.hip -- Pass C on bf16 MFMA, walking the chunks of a segment
// with the state held in registers.
//
// Reference counterpart: helix_chunk_out_mpp_impl<K> (src/kernels/mpp/
// helix_scan_mpp.metal:54-232), which reads each chunk's initial state as a
// bf16 copy that Pass B wrote (Sbf) and computes
//     y = tril(C B^T . decay) (dt x) + exp(Lcum) . (C S_init)
// with bf16 operands and fp32 accumulators.
//
// Here one workgroup owns (seq, segment, head, 64-wide P slab). It starts from
// the segment's initial state S_seg(s) (fp32, from Pass B) and walks the
// segment's chunks in order, so the per-chunk initial state never touches
// HBM: after producing y for chunk c it advances
//     R <- exp(L_end_c) R + B_c^T . (decay . dt . x)_c          (G4)
// in the same registers, on bf16 operands with fp32 accumulation. R only
// feeds y here; the fp32-exact carried state and s1 come from Passes A and B.
//
// Wave w owns output tile (t block tb = w >> 1, P block pb = w & 1) and keeps
// its own copy of R[:, pb block] (all N/32 state tiles) in MFMA result
// layout: lane (lo, hi), register r holds R[8(r/4) + 4hi + r%4 + 32nt][lo].
// That layout feeds G3 directly as the B operand: an MFMA's sixteen K slots
// may hold any sixteen state indices as long as the A operand (C) uses the
// same ones, and registers 0..7 of a tile give half hi the indices
// {0-3, 8-11} + 4hi, registers 8..15 the same plus 16. The G1 result is kept
// the same way (as C.B^T transposed, so the lane owns one output row t) and
// feeds G2's A operand without an LDS round trip.
#include "helix_common.h"

template <int NP>
struct StageW {
    float dtraw;
    float x[16];
    float b[16][NP / 64];
    float c[16][NP / 64];
};

template <int NP>
__device__ __forceinline__ void load_stage_w(StageW<NP>& st, const HelixScanParams& p,
                                             const float* __restrict__ dt_h,
                                             const float* __restrict__ x_h,
                                             const float* __restrict__ B_g,
                                             const float* __restrict__ C_g, int c, int lane,
                                             int wave, int pw, int N) {
    const int t0   = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    st.dtraw = dt_h[(long long)(t0 + min(lane, tlen - 1)) * p.s_dt[0]];
    const long long xc = (long long)min(lane, pw - 1) * p.s_x[2];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int jr = min(wave + 4 * i, tlen - 1);
        st.x[i] = x_h[(long long)(t0 + jr) * p.s_x[0] + xc];
        const float* brow = B_g + (long long)(t0 + jr) * p.s_b[0];
        const float* crow = C_g + (long long)(t0 + jr) * p.s_c[0];
#pragma unroll
        for (int m = 0; m < NP / 64; ++m) {
            const int nc = min(lane + 64 * m, N - 1);
            st.b[i][m] = brow[nc];
            st.c[i][m] = crow[nc];
        }
    }
}

// Eight bf16 K values from MFMA result registers r0..r0+7.
HELIX_DEV bf16x8 pack8(const f32x16& v, int r0) {
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = to_bf16(v[r0 + e]);
    return o;
}

// Two 4-element bf16 runs from an LDS row: columns [c0, c0+4) and [c0+8, c0+12).
HELIX_DEV bf16x8 lds_pair4(const __bf16* row, int c0) {
    const bf16x4 a = *reinterpret_cast<const bf16x4*>(row + c0);
    const bf16x4 b = *reinterpret_cast<const bf16x4*>(row + c0 + 8);
    bf16x8 o;
    o[0] = a[0]; o[1] = a[1]; o[2] = a[2]; o[3] = a[3];
    o[4] = b[0]; o[5] = b[1]; o[6] = b[2]; o[7] = b[3];
    return o;
}

template <int NP>
__device__ __forceinline__ void scan_walk_bf16_impl(const HelixScanParams& p, const HelixScanBuffers& b) {
    constexpr int NT  = NP / 32;          // state tiles per P block
    constexpr int RS  = NP + 8;           // bf16 row stride of C[t][n], B[j][n]
    constexpr int RSJ = HELIX_CS + 8;     // bf16 row stride of B^T[n][j], dtX^T[p][j], dtXs^T[p][j]

    __shared__ __attribute__((aligned(16))) __bf16 sC[HELIX_CS * RS];
    __shared__ __attribute__((aligned(16))) __bf16 sB[HELIX_CS * RS];
    __shared__ __attribute__((aligned(16))) __bf16 sBt[NP * RSJ];
    __shared__ __attribute__((aligned(16))) __bf16 sXt[HELIX_HD * RSJ];
    __shared__ __attribute__((aligned(16))) __bf16 sXst[HELIX_HD * RSJ];
    __shared__ __attribute__((aligned(16))) double sL[HELIX_CS];
    __shared__ __attribute__((aligned(16))) float sE[HELIX_CS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, lo = lane & 31, hi = lane >> 5;
    const int N = p.d_state, P = p.head_dim;
    const int hpg = p.heads_per_group;

    // 1-D grid, heads of one B/C group consecutive in the logical order so
    // they share an XCD (and the chunk's B and C in its L2).
    const unsigned total = (unsigned)(p.n_seg * p.n_head * p.n_pslab * p.n_seq);
    unsigned wid = xcd_logical_id(blockIdx.x, total);
    const int hig = (int)(wid % (unsigned)hpg);      wid /= (unsigned)hpg;
    const int seg = (int)(wid % (unsigned)p.n_seg);  wid /= (unsigned)p.n_seg;
    const int g   = (int)(wid % (unsigned)p.n_group); wid /= (unsigned)p.n_group;
    const int slab = (int)(wid % (unsigned)p.n_pslab);
    const int seq  = (int)(wid / (unsigned)p.n_pslab);
    const int h  = g * hpg + hig;
    const int p0 = slab * HELIX_HD;
    const int pw = min(HELIX_HD, P - p0);

    const int c_begin = seg * p.seg_len;
    const int c_end   = min(c_begin + p.seg_len, p.n_cg);
    if (c_begin >= c_end) return;

    const float A_h = b.A[(long long)h * p.s_a];
    const float* __restrict__ dt_h = b.dt + seq * p.seq_dt + h * p.s_dt[1];
    const float* __restrict__ x_h  = b.x + seq * p.seq_x + h * p.s_x[1] + p0 * p.s_x[2];
    const float* __restrict__ B_g  = b.B + seq * p.seq_b + g * p.s_b[1];
    const float* __restrict__ C_g  = b.C + seq * p.seq_c + g * p.s_c[1];

    const int tb = wave >> 1, pb = wave & 1;
    const int pp = pb * 32 + lo;                  // this lane's P column in the slab

    // R[n][p] for p in this wave's P block: the slab tile of S_seg(s) is
    // stored in exactly this register layout, so each group of four result
    // registers is one 16-byte unit load.
    f32x16 R[NT];
    {
        const float* sg = b.s_seg + seq * p.sg_seq + (long long)seg * p.sg_seg + state_tile_off(p, h, slab);
        const helix_rsrc rg = make_rsrc(sg, 64u * NP * sizeof(float));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const f32x4 v = buf_unit<float>(rg, lane, tile_unit(NT, pb, nt, r4, 0));
#pragma unroll
                for (int k = 0; k < 4; ++k) R[nt][4 * r4 + k] = v[k];
            }
    }

    StageW<NP> st;
    load_stage_w<NP>(st, p, dt_h, x_h, B_g, C_g, c_begin, lane, wave, pw, N);

    for (int c = c_begin; c < c_end; ++c) {
        const int t0   = (p.chunk_base + c) * HELIX_CS;
        const int tlen = min(HELIX_CS, p.n_tok - t0);

        const float dtv = lane < tlen ? helix_dt(p, st.dtraw) : 0.0f;
        const double lcum = wave_incl_sum((double)A_h * (double)dtv);
        const double lend = __shfl(lcum, 63, 64);
        const float sdec = lane < tlen ? exp_diff(lend, lcum) : 0.0f;

        // ---- stage this chunk into LDS (bf16 operands) ----------------------
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int j = wave + 4 * i;
            const float dj = bcast(dtv, j);
            const float sj = bcast(sdec, j);
            const float xv = lane < pw ? st.x[i] : 0.0f;
            sXt[lane * RSJ + j]  = to_bf16(dj * xv);
            sXst[lane * RSJ + j] = to_bf16(sj * dj * xv);
#pragma unroll
            for (int m = 0; m < NP / 64; ++m) {
                const int n = lane + 64 * m;
                const bool ok = j < tlen && n < N;
                const __bf16 bv = to_bf16(ok ? st.b[i][m] : 0.0f);
                sB[j * RS + n]   = bv;
                sBt[n * RSJ + j] = bv;
                sC[j * RS + n]   = to_bf16(ok ? st.c[i][m] : 0.0f);
            }
        }
        if (wave == 0) {
            sL[lane] = lcum;
            sE[lane] = expf((float)lcum);
        }
        __syncthreads();

        if (c + 1 < c_end) load_stage_w<NP>(st, p, dt_h, x_h, B_g, C_g, c + 1, lane, wave, pw, N);

        // ---- G1: CB^T tiles (jb, tb) for jb <= tb, kept as M^T -------------
        // D'[j][t] = sum_n B[j][n] C[t][n]; lane owns column t = tb*32 + lo.
        const int t_own = tb * 32 + lo;
        const double l_t = sL[t_own];
        bf16x8 mA[2][2];                        // [jb][half] A operands of G2
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
            if (jb > tb) break;
            f32x16 d = zero16();
#pragma unroll 4
            for (int s = 0; s < NP / 16; ++s) {
                const bf16x8 av = *reinterpret_cast<const bf16x8*>(&sB[(jb * 32 + lo) * RS + 16 * s + 8 * hi]);
                const bf16x8 bv = *reinterpret_cast<const bf16x8*>(&sC[t_own * RS + 16 * s + 8 * hi]);
                d = mfma_bf16(av, bv, d);
            }
            // M[t][j] = CB[t][j] exp(Lcum_t - Lcum_j), zero above the diagonal.
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int j = jb * 32 + acc_row(r, hi);
                d[r] = (j <= t_own) ? d[r] * expf((float)(l_t - sL[j])) : 0.0f;
            }
            mA[jb][0] = pack8(d, 0);
            mA[jb][1] = pack8(d, 8);
        }

        // ---- G3: y = C . R (state before this chunk), row scale, G2 --------
        f32x16 acc = zero16();
        const __bf16* crow = &sC[t_own * RS];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const bf16x8 av = lds_pair4(crow, nt * 32 + 16 * half + 4 * hi);
                acc = mfma_bf16(av, pack8(R[nt], 8 * half), acc);
            }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] *= sE[tb * 32 + acc_row(r, hi)];
        const __bf16* xrow = &sXt[pp * RSJ];
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
            if (jb > tb) break;
#pragma unroll
            for (int half = 0; half < 2; ++half)
                acc = mfma_bf16(mA[jb][half], lds_pair4(xrow, jb * 32 + 16 * half + 4 * hi), acc);
        }
        float* yh = b.y + seq * p.seq_y + h * p.s_y[1] + p0 * p.s_y[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = tb * 32 + acc_row(r, hi);
            if (t < tlen && pp < pw) yh[(long long)(t0 + t) * p.s_y[0] + pp * p.s_y[2]] = acc[r];
        }

        // ---- G4: R <- exp(L_end) R + B^T . dtXs ----------------------------
        const float a_c = expf((float)lend);
        const __bf16* xsrow = &sXst[pp * RSJ];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            R[nt] *= a_c;
#pragma unroll
            for (int s = 0; s < HELIX_CS / 16; ++s) {
                const bf16x8 av = *reinterpret_cast<const bf16x8*>(&sBt[(nt * 32 + lo) * RSJ + 16 * s + 8 * hi]);
                const bf16x8 bv = *reinterpret_cast<const bf16x8*>(&xsrow[16 * s + 8 * hi]);
                R[nt] = mfma_bf16(av, bv, R[nt]);
            }
        }
        __syncthreads();
    }
}

#define HELIX_PASS_C_WALK(NP)                                                                   \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_scan_walk_bf16_n##NP(           \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk_bf16_impl<NP>(p, b);                                                          \
    }

HELIX_PASS_C_WALK(64)
HELIX_PASS_C_WALK(128)
HELIX_PASS_C_WALK(256)
