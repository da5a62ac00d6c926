// pass_single.hip -- the single-pass scan (multipass = false): one launch, no
// scratch.
//
// Reference counterpart: helix_scan_sgmma_f32 (src/kernels/
// helix_scan_sgmma.metal:32-249). One workgroup per (16-channel block, head,
// seq) walks every chunk of the sequence in order:
//   y_t = sum_{j<=t} (C_t . B_j) exp(Lcum_t - Lcum_j) dt_j x_j     (G1, G2)
//       + exp(Lcum_t) C_t . S                                     (G3)
//   S  <- exp(L_end) S + sum_j B_j^T exp(L_end - Lcum_j) dt_j x_j   (G4)
// The reference parks S in the caller's s1 buffer between chunks (a device
// round trip per chunk). Here the state stays in the workgroup's MFMA
// registers for the whole sequence: s0 is read once at the start and s1
// written once at the end.
//
// MI355X layout: one workgroup per (seq, head, 16-channel block of a P slab).
// Four blocks per slab give four times the workgroups of a slab-wide walk
// (256 at 64 heads), so a single sequence fills the chip. Two forms:
//   - d_state <= 128 with fp32 storage (X6): eight waves in two roles (y
//     waves and state waves, see scan_1pass_impl), every product on six
//     v_mfma_f32_16x16x32_bf16 of three bf16 split planes (fp32 accuracy),
//     C, B, the state and M^T shared as planes in LDS, two barriers per
//     chunk. 150.5 KiB of LDS at d_state 128.
//   - otherwise (d_state 256, 16-bit storage, diagonal A):
//     v_mfma_f32_16x16x4_f32, fp32 throughout. With four waves, wave w
//     produces y's t block w (all 16 channels) and advances state tiles
//     NT/4 w .. NT/4 (w + 1) - 1; the state is shared through LDS (sR,
//     16 x d_state fp32) once per chunk for every wave's G3; G1 (C B^T,
//     shared by the block's channels) is split over the waves by tile; M
//     reuses B's rows once G1 and G4 are done with them. 150 KiB of LDS at
//     d_state 256.
//   16x16x4 layouts: A[i][k]: lane holds A[lane%16][lane/16];
//                    B[k][j]: lane holds B[lane/16][lane%16];
//                    D[i][j]: lane, reg r holds D[4*(lane/16) + r][lane%16].
// The state tile nt is R[n][p] for n = 16 nt .. 16 nt + 15 (M = n, N = p).
// K order (fp32 MFMA): G1 and G3 step s of a 16-wide K block takes
// k = 4*(lane/16) + s, so the A operand's four k of a block are one 16-byte
// LDS read, and so are G3's four state values (sR row p); G2 and G4 take
// token j = 4 s + lane/16. Both operands of a product use the same order.
#include "helix_common.h"

#include "pass_c_stage.h"

HELIX_DEV f32x4 mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Six 16 x 16 x 32 products of split operands a[3] x b[3], smallest terms first.
HELIX_DEV f32x4 mfma16_x6(const bf16x8 (&a)[3], const bf16x8 (&b)[3], f32x4 acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], b[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[0], acc, 0, 0, 0);
    return acc;
}

HELIX_DEV f32x4 zero4() {
    f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    return z;
}

// One chunk's global inputs for this thread, loaded for chunk c+1 while chunk
// c runs: dt of token `lane`, x of tokens tid / 16 + 4 NWV i at channel tid % 16
// of the block, and the wave's C and B rows wave + NWV r (NWV waves). Every
// address is clamped in bounds; the masks are applied when the registers are
// staged into LDS (fp32 storage: C and B rows read 0 there instead, through
// the range check). With fp32 storage a lane loads four consecutive state
// indices per row at a time (16-byte loads, a quarter of the instructions):
// load i covers rows r = i RPI + lane / LPR, indices 4 (lane % LPR) .. +3;
// with 16-bit storage, one index per row: columns lane + 64 m.
template <int NP, typename IO, int NWV>
struct StageS {
    typedef typename IoWord<IO>::type W;    // x, C, B in storage form
    static constexpr bool WIDE = sizeof(IO) == 4;
    static constexpr int RPW = HELIX_CS / NWV;   // rows per wave
    static constexpr int LPR = NP / 4;      // lanes per row (WIDE)
    static constexpr int RPI = 64 / LPR;    // rows per load (WIDE)
    static constexpr int NW = WIDE ? RPW / RPI : 1;
    static constexpr int NN = WIDE ? 1 : RPW;
    static constexpr int NX = 16 / NWV;     // x values per thread
    float dtraw;
    W x[NX];
    u32x4 cw[NW], bw[NW];
    W c[NN][NP / 64];
    W b[NN][NP / 64];
};

template <int NP, typename IO, int NWV>
__device__ __forceinline__ void load_stage_s(StageS<NP, IO, NWV>& st, const HelixScanParams& p,
                                             const HelixScanBuffers& b, const float* __restrict__ dt_h,
                                             const IO* __restrict__ x_h, int seq, int g, int t0,
                                             int tlen, int pw, int lane, int wave) {
    const int sdt = (int)p.s_dt[0], sx0 = sgpr_fresh((int)p.s_x[0]), sx2 = (int)p.s_x[2];
    const helix_rsrc rdt = make_rsrc(dt_h + (long long)t0 * p.s_dt[0], ((tlen - 1) * sdt + 1) * 4u);
    const helix_rsrc rx = make_rsrc(x_h + (long long)t0 * p.s_x[0],
                                    ((tlen - 1) * sx0 + (pw - 1) * sx2 + 1) * (unsigned)sizeof(IO));
    st.dtraw = buf_elem<float>(rdt, min(lane, tlen - 1) * sdt, 0);
    const int tid = 64 * wave + lane;
    const int xc = min(tid & 15, pw - 1) * sx2;
#pragma unroll
    for (int i = 0; i < StageS<NP, IO, NWV>::NX; ++i) {
        const int jr = min((tid >> 4) + 4 * NWV * i, tlen - 1);
        st.x[i] = io_load_word<IO>(rx, xc + jr * sx0, 0);   // lane-varying row: all in the VGPR offset
    }
    if constexpr (StageS<NP, IO, NWV>::WIDE) {
        constexpr int LPR = StageS<NP, IO, NWV>::LPR, RPI = StageS<NP, IO, NWV>::RPI;
        const int N = p.d_state;
        const int sc0 = (int)p.s_c[0], sb0 = (int)p.s_b[0];
        const helix_rsrc rc = make_rsrc(b.C + seq * p.seq_c + g * p.s_c[1] + (long long)t0 * p.s_c[0],
                                        ((tlen - 1) * sc0 + N) * 4u);
        const helix_rsrc rb = make_rsrc(b.B + seq * p.seq_b + g * p.s_b[1] + (long long)t0 * p.s_b[0],
                                        ((tlen - 1) * sb0 + N) * 4u);
        // Rows past tlen and indices past d_state (d_state % 8 == 0: four
        // indices all in or all out) take an offset past the range: they read 0.
        const int n0 = 4 * (lane % LPR);
#pragma unroll
        for (int i = 0; i < StageS<NP, IO, NWV>::NW; ++i) {
            const int j = wave + NWV * (i * RPI + lane / LPR);
            st.cw[i] = __builtin_amdgcn_raw_buffer_load_b128(rc, store_off_if_lt((n0 + j * sc0) * 4, j, tlen, n0, N), 0, 0);
            st.bw[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, store_off_if_lt((n0 + j * sb0) * 4, j, tlen, n0, N), 0, 0);
        }
    } else {
        load_cb_rows<NP, IO, NWV>(st.c, st.b, p, b, seq, g, t0, tlen, lane, wave);
    }
}

// G1 tile idx (0..9) of the causal 4 x 4 grid of 16 x 16 tiles, row-major
// over the lower triangle: (0,0) (1,0) (1,1) (2,0) ... (3,3).
HELIX_DEV int tri_tb(int idx) { return (idx >= 1) + (idx >= 3) + (idx >= 6); }
HELIX_DEV int tri_jb(int idx) {
    const int tb = tri_tb(idx);
    return idx - tb * (tb + 1) / 2;
}

// DIAG: A is one decay per (head, state index), A[h][n] (reference
// scan_ref.cpp:26-29). Then M[t][j] = sum_n C_t[n] B_j[n] exp(A_n (cs_t -
// cs_j)), with cs the chunk-local prefix of dt, is no longer a product of
// matrices; it is summed on the VALU (exp2 of a pre-scaled A), and the rest
// stays on MFMA after folding every other decay into factors that never
// exceed 1: C rows by exp(A_n cs_t) (G3), B rows by exp(A_n (cs_end - cs_j))
// (G4), and the carried state by exp(A_n cs_end) per state index.
// IO: the caller's storage type of x, B, C and y (dt, A and the states are fp32).
//
// NWV = 8 waves (d_state <= 128, scalar A): waves 0..3 produce y (G3 and G2 of
// t block `wave`), waves 4..7 carry the state (G4 on tiles NTW sw .. +NTW-1,
// sw = wave - 4), and G1's ten blocks go one to each state wave and the other
// six to the y waves (two to waves 0 and 1), whose G3 and G2 are the lighter
// part (per-phase cycle counts).
// Two waves per SIMD hide each other's staging, preamble and load latencies.
// NWV = 4 (diagonal A, d_state 256): every wave does all four parts.
// YACC: a block of state indices after the first (fp32 storage, p.y_acc): each
// y wave loads y of its rows at the top of the chunk and adds it at the store.
template <int NP, bool DIAG, typename IO = float, int NWV = 4, bool YACC = false>
__device__ __forceinline__ void scan_1pass_impl(const HelixScanParams& p, const HelixScanBuffers& b) {
    static_assert(!YACC || sizeof(IO) == 4, "y accumulates in fp32 storage only");
    static_assert(NWV == 4 || (NWV == 8 && !DIAG), "eight waves on the scalar-A path only");
    constexpr int NT  = NP / 16;           // 16-row state tiles
    constexpr int NTW = NT / 4;            // state tiles state wave sw advances: NTW sw .. NTW sw + NTW - 1
    constexpr int RSC = NP + 4;            // C and B rows
    constexpr int RSM = HELIX_CS + 4;      // M rows: in B's region after G4 (scalar A), own rows (DIAG)
    constexpr int RSR = NP + 4;            // state rows, one per channel of the block
    static_assert(HELIX_CS * RSM <= HELIX_CS * RSC, "M fits in the B rows");
    // X6 (fp32 storage, scalar A, d_state <= 128): all four products on
    // bf16x6 16x16x32 MFMA, from C and B staged as three bf16 planes each
    // (G4 reads B's planes transposed), the state shared as planes, and M
    // stored as planes of M^T (G2 reads them transposed); no fp32 rows.
    constexpr bool X6 = !DIAG && NP <= 128 && sizeof(IO) == 4;
    constexpr int NCH = NP / 8;            // 16-byte chunks per plane row (X6)
    constexpr int PLC = X6 ? 3 * HELIX_CS * NP : 8;   // C or B planes, bf16 elements
    constexpr int PLR = X6 ? 3 * 16 * NP : 8;         // state planes
    __shared__ __attribute__((aligned(16))) float sC[X6 ? 4 : HELIX_CS * RSC];
    __shared__ __attribute__((aligned(16))) float sB[X6 ? 4 : HELIX_CS * RSC];   // B rows, then M
    __shared__ __attribute__((aligned(16))) float sX[HELIX_CS * 16];   // dtX[token][channel]
    __shared__ __attribute__((aligned(16))) float sR[X6 ? 4 : 16 * RSR];   // S[channel][state index]
    __shared__ __attribute__((aligned(16))) __bf16 sCp[PLC];          // C[t][n] planes (X6)
    __shared__ __attribute__((aligned(16))) __bf16 sBp[PLC];          // B[j][n] planes (X6)
    __shared__ __attribute__((aligned(16))) __bf16 sRp[2 * PLR];      // S[p][n] planes, two chunks (X6)
    __shared__ __attribute__((aligned(16))) __bf16 sMt[X6 ? 3 * HELIX_CS * HELIX_CS : 8];   // M[t][j] as M^T[j][t] planes (X6)
    // PRE (eight waves): the chunk preamble (dt, Lcum and its exponentials)
    // is formed once, by wave PW during the previous chunk, into the other
    // half of two-chunk buffers, instead of by every wave at the chunk's start.
    constexpr bool PRE = NWV == 8;
    constexpr int PW = 3;                  // a y wave with one G1 block
    constexpr int NB = PRE ? 2 : 1;
    __shared__ double sLb[NB * HELIX_CS];  // Lcum_t (scalar A) or cs_t (DIAG), fp64
    __shared__ float sCsb[NB * HELIX_CS];  // exp(L_end - Lcum_j)
    __shared__ float sEb[NB * HELIX_CS];   // exp(Lcum_t)
    __shared__ float sDtb[PRE ? 2 * HELIX_CS : 4];   // dt_t (PRE)
    __shared__ double sA2[DIAG ? NP : 2];        // A_n log2(e) in fp64, 0 past d_state
    __shared__ __attribute__((aligned(16))) float sMd[DIAG ? HELIX_CS * RSM : 4];
    float* const sM = DIAG ? sMd : sB;

    const int lane = threadIdx.x & 63, wave = wave_uniform();
    const int l16 = lane & 15, g4 = lane >> 4;
    const int tid = (int)threadIdx.x;
    const bool ywave = wave < 4;           // produces y (G3, G2)
    const bool swave = wave >= NWV - 4;    // carries state tiles (G4)
    const int sw = wave - (NWV - 4);       // its state-wave index
    // G1 block q of this wave (wave-uniform), or -1.
    auto g1_idx = [&](int q) -> int {
        if constexpr (NWV == 4) {
            const int idx = wave + 4 * q;
            return idx < 10 ? idx : -1;
        } else {
            if (swave) return q == 0 ? sw : -1;                  // blocks 0..3
            if (q == 0) return 4 + wave;                         // blocks 4..7
            return (q == 1 && wave < 2) ? 8 + wave : -1;         // blocks 8, 9
        }
    };

    // 1-D grid over (seq, head, P slab, 16-channel block), block fastest in
    // the logical order, so a head's blocks and a group's heads (which read
    // the same B and C rows) run on one XCD.
    const unsigned total = (unsigned)p.n_seq * (unsigned)p.n_head * (unsigned)p.n_pslab * 4u;
    unsigned wid = xcd_logical_id(blockIdx.x, total);
    const int pb   = (int)(wid % 4u);                wid /= 4u;
    const int slab = (int)(wid % (unsigned)p.n_pslab); wid /= (unsigned)p.n_pslab;
    const int h    = (int)(wid % (unsigned)p.n_head);
    const int seq  = (int)(wid / (unsigned)p.n_head);
    const int g  = h / p.heads_per_group;
    const int N  = p.d_state;
    const int p0 = slab * HELIX_HD + 16 * pb;          // the block's first channel
    const int pw = min(16, p.head_dim - p0);           // its channels
    if (pw <= 0) return;   // a block past a short last slab: uniform, before any barrier
    const int tb = wave & 3;   // the t block of y this wave produces (y waves)

    const float A_h = DIAG ? 0.0f : b.A[(long long)h * p.s_a];
    if constexpr (DIAG) {
        for (int n = tid; n < NP; n += 64 * NWV)
            sA2[n] = n < N ? (double)b.A[(long long)h * p.s_a + n] * 1.4426950408889634074 : 0.0;
    }
    const float* __restrict__ dt_h = b.dt + seq * p.seq_dt + h * p.s_dt[1];
    const IO* __restrict__ x_h = reinterpret_cast<const IO*>(b.x) + seq * p.seq_x + h * p.s_x[1] +
                                 (long long)p0 * p.s_x[2];

    // State entering the sequence, s0[ids[seq]] in the caller's [P][N] rows
    // of s_s[1] elements (d_state, or more when this launch serves a block of
    // the state indices): register r of tile i holds n = 16 (NTW sw + i) +
    // 4 g4 + r at channel p0 + l16. Channels past the block read 0 through the
    // range check; n past d_state is masked (its index is clamped into the
    // row). Waves that carry no state load an empty range.
    const int src = p.has_ids ? b.ids[seq] : seq;
    const int sN = (int)p.s_s[1];    // d_state, or the whole row for a block of state indices
    const unsigned srow_bytes = (unsigned)((pw - 1) * sN + N) * 4u;
    f32x4 R[NTW];
    {
        const helix_rsrc rs = make_rsrc(b.s0 + src * p.seq_s + h * p.s_s[0] + (long long)p0 * sN,
                                        swave ? srow_bytes : 0u);
#pragma unroll
        for (int i = 0; i < NTW; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = 16 * (NTW * max(sw, 0) + i) + 4 * g4 + r;
                R[i][r] = keep_if_lt(buf_f32(rs, (l16 * sN + min(n, N - 1)) * 4, 0), n, N);
            }
    }
    // Every wave's G3 reads the whole state: it is shared through sR, written
    // by the wave that advances each tile. X6: planes in half `half` of sRp,
    // the one chunk `half` (mod 2) reads.
    auto publish_state = [&](int half) {
        if (swave) {
#pragma unroll
            for (int i = 0; i < NTW; ++i) {
                const int n = 16 * (NTW * sw + i) + 4 * g4;
                if constexpr (X6) {
                    unsigned w[2][3];
#pragma unroll
                    for (int e = 0; e < 2; ++e) split3_pair(R[i][2 * e], R[i][2 * e + 1], w[e][0], w[e][1], w[e][2]);
#pragma unroll
                    for (int pl = 0; pl < 3; ++pl)
                        *reinterpret_cast<u32x2*>(&sRp[half * PLR + x6_off<16, NCH>(pl, l16, n >> 3) + (n & 7)]) =
                            u32x2{w[0][pl], w[1][pl]};
                } else {
                    *reinterpret_cast<f32x4*>(&sR[l16 * RSR + n]) = R[i];
                }
            }
        }
    };
    publish_state(0);

    if constexpr (X6) {
        // M^T blocks above the diagonal that G2's 32-token steps cover, rows
        // j 16..31 at t 0..15 and rows 48..63 at t 32..47: zero for good (no
        // chunk writes them). 2 blocks x 16 rows x 2 chunks x 3 planes.
        for (int e = tid; e < 192; e += 64 * NWV) {
            const int pl = e % 3, c = (e / 3) & 1, row = (e / 6) & 15, blk = e / 96;
            *reinterpret_cast<u32x4*>(&sMt[x6_off<HELIX_CS, 8>(pl, 16 + 32 * blk + row, 4 * blk + c)]) =
                u32x4{0u, 0u, 0u, 0u};
        }
    }
    const int n_ch = (p.n_tok + HELIX_CS - 1) / HELIX_CS;
    const int sy0 = (int)p.s_y[0], sy2 = (int)p.s_y[2];
    StageS<NP, IO, NWV> st;
    load_stage_s<NP, IO, NWV>(st, p, b, dt_h, x_h, seq, g, 0, min(HELIX_CS, p.n_tok), pw, lane, wave);

    // Chunk cc's preamble from its raw dt (one wave, lane = token), into
    // buffer half cc & 1. dt = 0 past the chunk's length, so Lcum stays at
    // Lcum[tlen-1] there and dtX rows past tlen are zero.
    auto preamble = [&](int cc, float dtraw) {
        const int tl = min(HELIX_CS, p.n_tok - cc * HELIX_CS);
        const float d = keep_if_lt(helix_dt(p, dtraw), lane, tl);
        const double lc = wave_incl_sum((double)A_h * (double)d);
        const double le = bcast(lc, 63);
        const int o = (cc & 1) * HELIX_CS;
        sDtb[o + lane] = d;
        sLb[o + lane]  = lc;
        sCsb[o + lane] = exp_diff(le, lc);
        sEb[o + lane]  = expf((float)lc);
    };
    if constexpr (PRE) {
        if (wave == PW) preamble(0, st.dtraw);
        __syncthreads();
    }

    for (int c = 0; c < n_ch; ++c) {
        const int t0   = c * HELIX_CS;
        const int tlen = min(HELIX_CS, p.n_tok - t0);
        f32x4 yprev = zero4();
        if constexpr (YACC) {
            if (ywave) {
                const helix_rsrc ryp = make_rsrc(b.y + seq * p.seq_y + h * p.s_y[1] + (long long)t0 * p.s_y[0] +
                                                     (long long)p0 * p.s_y[2],
                                                 ((tlen - 1) * sy0 + (pw - 1) * sy2 + 1) * 4u);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 16 * tb + 4 * g4 + r;
                    yprev[r] = buf_f32(ryp, store_off_if_lt((t * sy0 + l16 * sy2) * 4, t, tlen, l16, pw), 0);
                }
            }
        }

        // ---- chunk preamble and staging ------------------------------------
        // dt = 0 past tlen, so Lcum stays at Lcum[tlen-1] there and dtX rows
        // past tlen are zero.
        const int cbo = PRE ? (c & 1) * HELIX_CS : 0;
        double* const sL = sLb + cbo;
        float* const sCs = sCsb + cbo;
        float* const sE  = sEb + cbo;
        float dtv = 0.0f;
        double lend;
        if constexpr (PRE) {
            lend = sL[HELIX_CS - 1];
        } else {
            dtv = keep_if_lt(helix_dt(p, st.dtraw), lane, tlen);
            const double lcum = wave_incl_sum(DIAG ? (double)dtv : (double)A_h * (double)dtv);
            lend = bcast(lcum, 63);
            if (wave == 0) {
                sL[lane] = lcum;
                if constexpr (!DIAG) {
                    sCs[lane] = exp_diff(lend, lcum);
                    sE[lane]  = expf((float)lcum);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < StageS<NP, IO, NWV>::NX; ++i) {
            const int j = (tid >> 4) + 4 * NWV * i;
            const float dj = PRE ? sDtb[cbo + j] : __shfl(dtv, j, 64);
            sX[j * 16 + (tid & 15)] = keep_if_lt(dj * io_widen<IO>(st.x[i]), tid & 15, pw);
        }
        if constexpr (StageS<NP, IO, NWV>::WIDE) {
            constexpr int LPR = StageS<NP, IO, NWV>::LPR, RPI = StageS<NP, IO, NWV>::RPI;
            const int n = 4 * (lane % LPR);
#pragma unroll
            for (int i = 0; i < StageS<NP, IO, NWV>::NW; ++i) {
                const int j = wave + NWV * (i * RPI + lane / LPR);
                f32x4 cv, bv;   // zero past tlen and d_state (range check)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    cv[e] = as_f32(st.cw[i][e]);
                    bv[e] = as_f32(st.bw[i][e]);
                }
                if constexpr (X6) {
                    unsigned wc[2][3], wb[2][3];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        split3_pair(cv[2 * e], cv[2 * e + 1], wc[e][0], wc[e][1], wc[e][2]);
                        split3_pair(bv[2 * e], bv[2 * e + 1], wb[e][0], wb[e][1], wb[e][2]);
                    }
#pragma unroll
                    for (int pl = 0; pl < 3; ++pl) {
                        const int off = x6_off<HELIX_CS, NCH>(pl, j, n >> 3) + (n & 7);
                        *reinterpret_cast<u32x2*>(&sCp[off]) = u32x2{wc[0][pl], wc[1][pl]};
                        *reinterpret_cast<u32x2*>(&sBp[off]) = u32x2{wb[0][pl], wb[1][pl]};
                    }
                } else {
                    *reinterpret_cast<f32x4*>(&sB[j * RSC + n]) = bv;
                    *reinterpret_cast<f32x4*>(&sC[j * RSC + n]) = cv;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < StageS<NP, IO, NWV>::RPW; ++i) {
                const int j = wave + NWV * i;
#pragma unroll
                for (int m = 0; m < NP / 64; ++m) {
                    const int n = lane + 64 * m;
                    sC[j * RSC + n] = keep_if_lt2(io_widen<IO>(st.c[i][m]), j, tlen, n, N);
                    sB[j * RSC + n] = keep_if_lt2(io_widen<IO>(st.b[i][m]), j, tlen, n, N);
                }
            }
        }
        __syncthreads();

        // The next chunk's inputs travel while this one runs on the MFMA pipe.
        // With eight waves the state waves issue theirs later (after G1, or
        // inside G4 with bf16x6 products), so the two halves do not queue for
        // the texture units at the same time.
        const bool early_pf = NWV == 4 || ywave;
        if (c + 1 < n_ch && early_pf)
            load_stage_s<NP, IO, NWV>(st, p, b, dt_h, x_h, seq, g, t0 + HELIX_CS,
                                 min(HELIX_CS, p.n_tok - t0 - HELIX_CS), pw, lane, wave);

        // B operands of G2 (dtX) and G4 (dtX scaled by exp(L_end - Lcum_j); with
        // DIAG that decay goes into the B rows instead).
        float xb[16], xs[16];
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int j = 4 * s + g4;
            xb[s] = sX[j * 16 + l16];
            xs[s] = DIAG ? xb[s] : xb[s] * sCs[j];
        }

        // ---- G1: M = tril(C B^T) . exp(Lcum_t - Lcum_j), tiles wave + 4 q ----
        f32x4 mt[3];
        if constexpr (DIAG) {
            // M on the VALU. Thread: row t = tid / 4, columns j = 16 q + i
            // (q = tid % 4); a group wholly above the diagonal skips the sum.
            // Past d_state C and B are zero, so n runs to d_state only. Each
            // exponent is formed in fp64 and rounded once, as the scalar
            // path's exp(Lcum_t - Lcum_j) is.
            const int t = tid >> 2, q = tid & 3;
            const double ct = sL[t];
            double dcs[16];
            float acc[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                dcs[i] = ct - sL[16 * q + i];
                acc[i] = 0.0f;
            }
            if (16 * q <= t) {
                for (int n = 0; n < N; n += 4) {
                    const f32x4 c4 = *reinterpret_cast<const f32x4*>(&sC[t * RSC + n]);
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const double a = sA2[n + k];
#pragma unroll
                        for (int i = 0; i < 16; ++i)
                            acc[i] = fmaf(c4[k] * __builtin_amdgcn_exp2f((float)(a * dcs[i])),
                                          sB[(16 * q + i) * RSC + n + k], acc[i]);
                    }
                }
            }
            // j > t: the exponent is positive and may overflow; the bitwise
            // mask clears whatever the sum holds.
#pragma unroll
            for (int i = 0; i < 16; ++i) sM[t * RSM + 16 * q + i] = keep_if_le(acc[i], 16 * q + i, t);
            __syncthreads();   // M is summed from the unscaled rows
            // C rows by exp(A_n cs_t), B rows by exp(A_n (cs_end - cs_j)).
#pragma unroll 4
            for (int i = 0; i < HELIX_CS * NP / HELIX_WG; ++i) {
                const int idx = tid + HELIX_WG * i;
                const int row = idx / NP, n = idx % NP;
                const double cr = sL[row];
                const double a = sA2[n];
                sC[row * RSC + n] *= __builtin_amdgcn_exp2f((float)(a * cr));
                sB[row * RSC + n] *= __builtin_amdgcn_exp2f((float)(a * (lend - cr)));
            }
            __syncthreads();
        }
#pragma unroll
        for (int q = 0; q < 3; ++q) {
            mt[q] = zero4();
            const int idx = g1_idx(q);
            if (!DIAG && idx >= 0) {
                const int gtb = tri_tb(idx), jb = tri_jb(idx);
                f32x4 acc = zero4();
                if constexpr (X6) {
#pragma unroll
                    for (int s = 0; s < NP / 32; ++s) {
                        bf16x8 av[3], bv[3];
                        x6_read<HELIX_CS, NCH>(sCp, 16 * gtb + l16, 4 * s + g4, av);
                        x6_read<HELIX_CS, NCH>(sBp, 16 * jb + l16, 4 * s + g4, bv);
                        acc = mfma16_x6(av, bv, acc);
                    }
                } else {
#pragma unroll 4
                for (int kb = 0; kb < NP / 16; ++kb) {
                    const f32x4 a4 = *reinterpret_cast<const f32x4*>(&sC[(16 * gtb + l16) * RSC + 16 * kb + 4 * g4]);
                    const f32x4 b4 = *reinterpret_cast<const f32x4*>(&sB[(16 * jb + l16) * RSC + 16 * kb + 4 * g4]);
#pragma unroll
                    for (int s = 0; s < 4; ++s) acc = mfma16(a4[s], b4[s], acc);
                }
                }
                const int j = 16 * jb + l16;
                const double lj = sL[j];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 16 * gtb + 4 * g4 + r;
                    // j > t: exp of a positive difference may overflow; the
                    // bitwise mask clears the product whatever it is.
                    mt[q][r] = keep_if_le(acc[r] * exp_diff(sL[t], lj), j, t);
                }
                if constexpr (X6) {
                    // Planes of M^T: row j, t = 16 gtb + 4 g4 .. + 3 (8 bytes a
                    // plane). The previous chunk's G2 is behind the last barrier.
                    unsigned w[2][3];
#pragma unroll
                    for (int e = 0; e < 2; ++e) split3_pair(mt[q][2 * e], mt[q][2 * e + 1], w[e][0], w[e][1], w[e][2]);
                    const int t = 16 * gtb + 4 * g4;
#pragma unroll
                    for (int pl = 0; pl < 3; ++pl)
                        *reinterpret_cast<u32x2*>(&sMt[x6_off<HELIX_CS, 8>(pl, j, t >> 3) + (t & 7)]) =
                            u32x2{w[0][pl], w[1][pl]};
                }
            }
        }

        // With bf16x6 products the state waves issue theirs inside G4, behind
        // its first product, so a stall at the texture units does not hold
        // back MFMAs that are already queued.
        if (!X6 && c + 1 < n_ch && !early_pf)
            load_stage_s<NP, IO, NWV>(st, p, b, dt_h, x_h, seq, g, t0 + HELIX_CS,
                                 min(HELIX_CS, p.n_tok - t0 - HELIX_CS), pw, lane, wave);

        // ---- G3: y = exp(Lcum_t) . (C S) for this wave's t block; S from sR --
        f32x4 ya = zero4();
        if (ywave) {
        if constexpr (X6) {
#pragma unroll
            for (int s = 0; s < NP / 32; ++s) {
                bf16x8 av[3], rv[3];
                x6_read<HELIX_CS, NCH>(sCp, 16 * tb + l16, 4 * s + g4, av);
                x6_read<16, NCH>(sRp + (c & 1) * PLR, l16, 4 * s + g4, rv);
                ya = mfma16_x6(av, rv, ya);
            }
        } else {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const f32x4 a4 = *reinterpret_cast<const f32x4*>(&sC[(16 * tb + l16) * RSC + 16 * nt + 4 * g4]);
            const f32x4 r4 = *reinterpret_cast<const f32x4*>(&sR[l16 * RSR + 16 * nt + 4 * g4]);
#pragma unroll
            for (int s = 0; s < 4; ++s) ya = mfma16(a4[s], r4[s], ya);
        }
        }
        if constexpr (!DIAG) {
#pragma unroll
            for (int r = 0; r < 4; ++r) ya[r] *= sE[16 * tb + 4 * g4 + r];
        }
        }
        // The next chunk's preamble (its dt arrived with this chunk's prefetch;
        // its buffer half was last read before the previous chunk's end).
        if constexpr (PRE) {
            if (wave == PW && c + 1 < n_ch) preamble(c + 1, st.dtraw);
        }

        // ---- G4: S <- exp(L_end) S + B^T (exp(L_end - Lcum) dt x), own tiles --
        if (swave) {
        if constexpr (DIAG) {
#pragma unroll
            for (int i = 0; i < NTW; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    R[i][r] *= __builtin_amdgcn_exp2f((float)(sA2[16 * (NTW * sw + i) + 4 * g4 + r] * lend));
        } else {
            const float a_c = expf((float)lend);
#pragma unroll
            for (int i = 0; i < NTW; ++i) R[i] *= a_c;
        }
        if constexpr (X6) {
            // K slot 4 h + r of lane group g4 in step S is token
            // j = 32 S + 16 h + 4 r + g4, the token of xs[8 S + 4 h + r], so
            // the x operand is xs split in registers; the B^T operand comes
            // from B's planes by transpose reads (lane 4 r + q names row j,
            // state indices n0 + 4 q .. + 3).
            const int rr = l16 >> 2, qq = l16 & 3;
#pragma unroll
            for (int S = 0; S < HELIX_CS / 32; ++S) {
                float xv8[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) xv8[i] = xs[8 * S + i];
                bf16x8 xp[3];
                x6_split8(xv8, xp);
#pragma unroll
                for (int i = 0; i < NTW; ++i) {
                    const int n = 16 * (NTW * sw + i) + 4 * qq;
                    bf16x8 bt[3];
#pragma unroll
                    for (int pl = 0; pl < 3; ++pl) {
                        const u32x2 lo = lds_read_tr16(&sBp[x6_off<HELIX_CS, NCH>(pl, 32 * S + 4 * rr + g4, n >> 3) + (n & 7)]);
                        const u32x2 hi = lds_read_tr16(&sBp[x6_off<HELIX_CS, NCH>(pl, 32 * S + 16 + 4 * rr + g4, n >> 3) + (n & 7)]);
                        bt[pl] = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
                    }
                    R[i] = mfma16_x6(bt, xp, R[i]);
                    if (S == 0 && i == 0) {
                        __builtin_amdgcn_sched_barrier(0);
                        if (c + 1 < n_ch)
                            load_stage_s<NP, IO, NWV>(st, p, b, dt_h, x_h, seq, g, t0 + HELIX_CS,
                                                      min(HELIX_CS, p.n_tok - t0 - HELIX_CS), pw, lane, wave);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
        } else {
#pragma unroll 4
        for (int s = 0; s < 16; ++s) {
            const int j = 4 * s + g4;
#pragma unroll
            for (int i = 0; i < NTW; ++i)
                R[i] = mfma16(sB[j * RSC + 16 * (NTW * sw + i) + l16], xs[s], R[i]);
        }
        }
        }
        // X6: the advanced state goes to the other half of sRp (the one chunk
        // c + 1 reads; chunk c - 1's readers are behind the last barrier), and
        // M^T is complete once every wave is past this barrier. Otherwise
        // every wave is done with the B rows and with sR here: M takes over
        // B's rows, and the advanced state replaces the old one.
        if constexpr (X6) publish_state((c + 1) & 1);
        __syncthreads();
        if constexpr (!X6) {
        if constexpr (!DIAG) {
#pragma unroll
            for (int q = 0; q < 3; ++q) {
                const int idx = g1_idx(q);
                if (idx >= 0) {
                    const int gtb = tri_tb(idx), jb = tri_jb(idx);
#pragma unroll
                    for (int r = 0; r < 4; ++r) sM[(16 * gtb + 4 * g4 + r) * RSM + 16 * jb + l16] = mt[q][r];
                }
            }
        }
        publish_state(0);
        __syncthreads();
        }

        // ---- G2: y += M dtX over the causal K range of this t block --------
        if (ywave) {
        if constexpr (X6) {
            // K slot 4 h + r of lane group g4 in step S is token
            // j = 32 S + 16 h + 4 r + g4 (xb[8 S + 4 h + r]); lane 4 r + q
            // names row j of M^T, t = 16 tb + 4 q .. + 3. Steps past the t
            // block's causal range are skipped; the blocks above the diagonal
            // inside a step, (0,1) and (2,3), hold zeros.
            const int rr = l16 >> 2, qq = l16 & 3;
            const int t = 16 * tb + 4 * qq;
#pragma unroll
            for (int S = 0; S < HELIX_CS / 32; ++S) {
                if (S > (tb >> 1)) break;
                float xv8[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) xv8[i] = xb[8 * S + i];
                bf16x8 xp[3], mv[3];
                x6_split8(xv8, xp);
#pragma unroll
                for (int pl = 0; pl < 3; ++pl) {
                    const u32x2 lo = lds_read_tr16(&sMt[x6_off<HELIX_CS, 8>(pl, 32 * S + 4 * rr + g4, t >> 3) + (t & 7)]);
                    const u32x2 hi = lds_read_tr16(&sMt[x6_off<HELIX_CS, 8>(pl, 32 * S + 16 + 4 * rr + g4, t >> 3) + (t & 7)]);
                    mv[pl] = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
                }
                ya = mfma16_x6(mv, xp, ya);
            }
        } else {
        for (int s = 0; s < 4 * (tb + 1); ++s)
            ya = mfma16(sM[(16 * tb + l16) * RSM + 4 * s + g4], xb[s], ya);
        }

        // ---- y rows t < tlen, channels < pw ---------------------------------
        {
            constexpr int ES = (int)sizeof(IO);
            const unsigned bytes = ((tlen - 1) * sy0 + (pw - 1) * sy2 + 1) * (unsigned)ES;
            const helix_rsrc ry = make_rsrc(reinterpret_cast<IO*>(b.y) + seq * p.seq_y + h * p.s_y[1] +
                                                (long long)t0 * p.s_y[0] + (long long)p0 * p.s_y[2],
                                            bytes);
            auto put = [&](auto acc_on) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 16 * tb + 4 * g4 + r;
                    y_store<IO, decltype(acc_on)::value>(
                        ry, ya[r], store_off_if_lt((t * sy0 + l16 * sy2) * ES, t, tlen, l16, pw), 0);
                }
            };
            if constexpr (YACC) {
#pragma unroll
                for (int r = 0; r < 4; ++r) ya[r] += yprev[r];
                put(std::false_type{});
            } else {
                with_y_acc(p, put);
            }
        }
        }
        // The next chunk's staging overwrites C, B/M and dtX. X6 needs no
        // barrier here: G2 reads only M^T (rewritten after the next chunk's
        // first barrier) and registers, and every reader of C, B, dtX and
        // the state planes is behind the barrier above; the state waves stage
        // the next chunk while the y waves finish G2.
        if constexpr (!X6) __syncthreads();
    }

    // Final state to s1[seq], same register layout as the s0 read (the state
    // waves; the others store to an empty range).
    const helix_rsrc ro = make_rsrc(b.s1 + seq * p.seq_s + h * p.s_s[0] + (long long)p0 * sN,
                                    swave ? srow_bytes : 0u);
#pragma unroll
    for (int i = 0; i < NTW; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int n = 16 * (NTW * max(sw, 0) + i) + 4 * g4 + r;
            __builtin_amdgcn_raw_buffer_store_b32(as_u32(R[i][r]), ro,
                                                  store_off_if_lt((l16 * sN + n) * 4, n, N, l16, pw), 0, 0);
        }
}

#define HELIX_SCAN_1PASS(NP)                                                                    \
    extern "C" __global__ __launch_bounds__(64 * HELIX_1PASS_WAVES(NP)) void helix_scan_1pass_f32_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_1pass_impl<NP, false, float, HELIX_1PASS_WAVES(NP)>(p, b);                         \
    }

// 16-bit storage of x, B, C and y (io_dtype BF16 / F16), fp32 compute.
#define HELIX_SCAN_1PASS_IO(NP)                                                                 \
    extern "C" __global__ __launch_bounds__(64 * HELIX_1PASS_WAVES(NP)) void helix_scan_1pass_bf16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_1pass_impl<NP, false, __bf16, HELIX_1PASS_WAVES(NP)>(p, b);                        \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(64 * HELIX_1PASS_WAVES(NP)) void helix_scan_1pass_f16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_1pass_impl<NP, false, _Float16, HELIX_1PASS_WAVES(NP)>(p, b);                      \
    }

#define HELIX_SCAN_1PASS_DIAG(NP)                                                               \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_scan_1pass_diag_f32_n##NP(      \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_1pass_impl<NP, true>(p, b);                                                        \
    }

// The one-launch kernel of the second and later blocks of state indices
// (at most HELIX_N_BLOCK = 128 wide).
#define HELIX_SCAN_1PASS_ACC(NP)                                                                \
    extern "C" __global__ __launch_bounds__(64 * HELIX_1PASS_WAVES(NP)) void helix_scan_1pass_f32_acc_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_1pass_impl<NP, false, float, HELIX_1PASS_WAVES(NP), true>(p, b);                   \
    }

HELIX_SCAN_1PASS(64)
HELIX_SCAN_1PASS(128)
HELIX_SCAN_1PASS(256)
HELIX_SCAN_1PASS_ACC(64)
HELIX_SCAN_1PASS_ACC(128)
HELIX_SCAN_1PASS_IO(64)
HELIX_SCAN_1PASS_IO(128)
HELIX_SCAN_1PASS_IO(256)
// d_state <= 128: the diagonal form keeps M in rows of its own.
HELIX_SCAN_1PASS_DIAG(64)
HELIX_SCAN_1PASS_DIAG(128)
