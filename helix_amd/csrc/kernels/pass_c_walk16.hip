// pass_c_walk16.hip -- the chunk-walking bf16 Pass C on 16 x 16 x 32 MFMA tiles.
//
// One workgroup owns (seq, walk segment of walk_len chunks, HELIX_WALK_HPW
// heads of one B/C group, 64-wide P slab), starts each head from S_seg (fp32:
// from Pass B at the Pass A segment the walk segment starts at, or, with
// p.fuse_b, scanned here from s0 and Pass A's segment aggregates) and walks
// the segment's chunks,
// producing per chunk
//     y = tril(C B^T . decay) (dt x) + exp(Lcum) . (C R)        (G1, G2, G3)
//     R <- exp(L_end) R + B^T . (decay . dt . x)                  (G4)
// on bf16 operands with fp32 accumulation (reference counterpart:
// helix_chunk_out_mpp_impl, src/kernels/mpp/helix_scan_mpp.metal:54-232).
//
// Work split. The four waves of a head each own a 16-column P block
// (p = 16 w4 + lane%16) for all 64 tokens, so no product is computed twice:
//   - R[n][p] for the wave's 16 columns lives in registers, NP/16 result tiles
//     of v_mfma_f32_16x16x32_bf16: register r of tile nb holds
//     R[16 nb + 4 (lane/16) + r][p];
//   - G3 (C R) and G4 (B^T dtXs) run on those tiles; G2 (M dtX) on the
//     wave's columns;
//   - G1 (C B^T and its decay mask) is split over the head's waves by 16 x 16
//     block (ten blocks on or below the diagonal) and shared through LDS as
//     M[t][j] in bf16.
// An MFMA's 32 K slots may hold any 32 indices as long as both operands use
// the same ones. A lane of the 16x16x32 layout supplies K slots 8 (lane/16)
// .. +7; R's result registers give lane q state rows 4q .. 4q+3 of two
// consecutive tiles, so within each group of 32 state indices, index
// 16 h + 4 q + r sits at K position 8 q + 4 h + r (perm32) in every
// n-contiguous operand (C and B rows in LDS), and R feeds G3 straight from
// its registers.
//
// LDS (bf16, rows padded by 16): C[t][n], B[j][n] (perm32 order), B^T[n][j],
// and per head dtX^T[p][j] (two buffers, by chunk parity), dtXs^T[p][j] and
// M[t][j] (natural j order).
#include "helix_common.h"

#include "pass_c_stage.h"

HELIX_DEV f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// K position of state index i inside its group of 32: 16 h + 4 q + r -> 8 q + 4 h + r.
HELIX_DEV int perm32(int i) {
    return (i & ~31) | (8 * ((i >> 2) & 3) + 4 * ((i >> 4) & 1) + (i & 3));
}

// G1 block idx (0..9) of the lower triangle of the 4 x 4 grid of 16 x 16
// blocks, in the order (jb, tb) = (0,0) (0,1) (1,1) (0,2) (1,2) (2,2) (0,3) ...
HELIX_DEV int g1_tb(int idx) { return (idx >= 1) + (idx >= 3) + (idx >= 6); }
HELIX_DEV int g1_jb(int idx) {
    const int tb = g1_tb(idx);
    return idx - tb * (tb + 1) / 2;
}

// x of tokens 16 wave + i at channel p = lane and the decay record of token
// lane (Pass A's store_decay_record: dt, Lcum log2(e)), prefetched a chunk
// ahead in storage form.
template <typename IO>
struct StageW16 {
    u32x2 rec;
    typename IoWord<IO>::type x[16];
};

template <typename IO>
__device__ __forceinline__ void load_stage_w16(StageW16<IO>& st, const HelixScanParams& p,
                                               const float* __restrict__ rec_h,
                                               const IO* __restrict__ x_h, int c, int lane,
                                               int wave, int pw) {
    const int t0   = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const int sx0 = sgpr_fresh((int)p.s_x[0]), sx2 = (int)p.s_x[2];
    const helix_rsrc rr = make_rsrc(reinterpret_cast<const char*>(rec_h) + (long long)c * p.n_head * (HELIX_CS * HELIX_REC_WALK_BYTES),
                                    HELIX_CS * HELIX_REC_WALK_BYTES);
    const helix_rsrc rx  = make_rsrc(x_h + (long long)t0 * p.s_x[0],
                                     ((tlen - 1) * sx0 + (pw - 1) * sx2 + 1) * (unsigned)sizeof(IO));
    st.rec = __builtin_amdgcn_raw_buffer_load_b64(rr, lane * HELIX_REC_WALK_BYTES, 0, 0);
    const int xc = min(lane, pw - 1) * sx2;
#pragma unroll
    for (int i = 0; i < 16; ++i) st.x[i] = io_load_word<IO>(rx, xc, min(16 * wave + i, tlen - 1) * sx0);
}

// This lane's B and C runs of one chunk, as loaded: the run of eight state
// indices 8u .. 8u+7 of KQ rows jrow + RPI k, two 16-byte words each in fp32
// storage, one in 16-bit.
template <int KQ, typename IO>
struct RunsW16 {
    static constexpr int WPR = sizeof(IO) == 4 ? 2 : 1;
    u32x4 b[KQ][WPR], c[KQ][WPR];
};

template <int KQ, int RPI, typename IO>
__device__ __forceinline__ void load_runs_w16(RunsW16<KQ, IO>& r, const HelixScanParams& p,
                                              const IO* __restrict__ B_g, const IO* __restrict__ C_g,
                                              int c, int N, int jrow, int u) {
    constexpr int ES = (int)sizeof(IO);
    const int t0   = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const int sb0 = sgpr_fresh((int)p.s_b[0]), sc0 = sgpr_fresh((int)p.s_c[0]);
    const helix_rsrc rb = make_rsrc(B_g + (long long)t0 * p.s_b[0], ((tlen - 1) * sb0 + N) * (unsigned)ES);
    const helix_rsrc rc = make_rsrc(C_g + (long long)t0 * p.s_c[0], ((tlen - 1) * sc0 + N) * (unsigned)ES);
    const int n0 = min(8 * u, N - 8);   // d_state % 8 == 0: a run is all in or out
#pragma unroll
    for (int k = 0; k < KQ; ++k) {
        const int jr = min(jrow + RPI * k, tlen - 1);
#pragma unroll
        for (int w = 0; w < RunsW16<KQ, IO>::WPR; ++w) {
            r.b[k][w] = __builtin_amdgcn_raw_buffer_load_b128(rb, (n0 + jr * sb0) * ES + 16 * w, 0, 0);
            r.c[k][w] = __builtin_amdgcn_raw_buffer_load_b128(rc, (n0 + jr * sc0) * ES + 16 * w, 0, 0);
        }
    }
}

// Element e (0..7) of a run, widened to fp32.
template <typename IO, int WPR>
HELIX_DEV float run16_elem(const u32x4 (&w)[WPR], int e) {
    if constexpr (sizeof(IO) == 4) {
        return as_f32(w[e >> 2][e & 3]);
    } else {
        const unsigned v = w[0][e >> 1];
        return io_f32<IO>((unsigned short)((e & 1) ? (v >> 16) : (v & 0xffffu)));
    }
}

// Element offset of column col of row `row` in a bf16 LDS buffer of row
// stride RSX: the 16-byte chunk index is XOR-ed with (row / 4) % 8. Every
// operand read takes 16 consecutive rows of one chunk per 16 lanes; with the
// swizzle those take 4 cycles per 16-byte read instruction instead of 5.8 on
// gfx950 (measured), and the 8- and 16-byte staging writes of M and dtX^T
// 8 and 7.5 instead of 16 and 10. The chunk index stays in its group of 8.
template <int RSX>
HELIX_DEV int swz_off(int row, int col) {
    return row * RSX + ((((col >> 3) ^ ((row >> 2) & 7))) << 3) + (col & 7);
}

// Sixteen consecutive tokens' values of one row, in natural order: columns
// col0 .. col0 + 15 of row `row` (col0 a multiple of 8).
template <int RSX>
HELIX_DEV void store16_nat(__bf16* buf, int row, int col0, const float (&v)[16]) {
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = to_bf16(v[e]);
        b[e] = to_bf16(v[8 + e]);
    }
    *reinterpret_cast<bf16x8*>(&buf[swz_off<RSX>(row, col0)]) = a;
    *reinterpret_cast<bf16x8*>(&buf[swz_off<RSX>(row, col0 + 8)]) = b;
}

// IO: the caller's storage type of x, B, C and y (dt, A and the states are
// fp32). BIO: the type B and C are read in; __bf16 with fp32 storage when
// they come from Pass A's bf16 copies (the host points B and C there).
// YACC: the kernel of a block of state indices after the first (fp32
// storage, p.y_acc): y of each chunk is loaded with the next chunk's inputs
// and added to the chunk's result.
template <int NP, int HPW, typename IO = float, typename BIO = IO, bool YACC = false>
__device__ __forceinline__ void scan_walk16_impl(const HelixScanParams& p, const HelixScanBuffers& b) {
    static_assert(!YACC || sizeof(IO) == 4, "y accumulates in fp32 storage only");
    constexpr int NW  = 4 * HPW;              // HPW heads per workgroup, four waves each
    constexpr int NB  = NP / 16;              // 16-row state tiles of R
    constexpr int KS  = NP / 32;              // K steps over the state
    constexpr int NT32 = NP / 32;             // 32 x 32 tiles of the slab tile layout
    // Row strides (bf16) of C[t][n], B[j][n] and of B^T, dtX^T, dtXs^T, M. Every
    // operand read takes 16 rows (lane % 16) x four 16-byte chunks (lane / 16);
    // measured on gfx950 (SQ_LDS_BANK_CONFLICT), that is conflict-free when
    // the row stride in dwords is 8 mod 16 and about 17% conflicted at the
    // 4 mod 16 of an 8-element pad. Padding 16 elements gives NP/2 + 8 and 40.
    constexpr int RS  = NP + 16;
    constexpr int RSJ = HELIX_CS + 16;
    constexpr int NCH = NP / 8;               // 8-element runs per C / B row
    // B^T[n][j] sits at row n, 16-byte chunk (j / 8) ^ ((n / 16) % 8). The
    // staging writes are a transpose: one instruction writes column j of rows
    // 8 u + e for eight u, which without the swizzle share one bank row
    // (8-way conflicts); G4's 16-byte reads take 16 consecutive rows of one
    // chunk, which the swizzle leaves in distinct banks.
    auto bt_off = [](int n, int j) { return n * RSJ + (((j >> 3) ^ ((n >> 4) & 7)) << 3) + (j & 7); };

    // M takes the place of B's rows when they fit (B is dead once G1 has read
    // it): G1 then keeps its blocks in registers until every wave is past
    // its B reads.
    constexpr bool M_IN_B = HPW * HELIX_CS * RSJ <= HELIX_CS * RS;
    constexpr int MB = M_IN_B ? 0 : HPW * HELIX_CS * RSJ;
    __shared__ __attribute__((aligned(16))) __bf16 sC[HELIX_CS * RS];
    __shared__ __attribute__((aligned(16))) __bf16 sB[HELIX_CS * RS];
    __shared__ __attribute__((aligned(16))) __bf16 sBt[NP * RSJ];
    __shared__ __attribute__((aligned(16))) __bf16 sXt[2][HPW][HELIX_HD * RSJ];   // by chunk parity
    __shared__ __attribute__((aligned(16))) __bf16 sXst[HPW][HELIX_HD * RSJ];
    __shared__ __attribute__((aligned(16))) __bf16 sMown[MB > 0 ? MB : 8];
    __bf16* const sM = M_IN_B ? sB : sMown;      // head slot hw at sM + hw * HELIX_CS * RSJ
    __shared__ __attribute__((aligned(16))) float sL2[HPW][HELIX_CS];   // Lcum_t log2(e)
    __shared__ __attribute__((aligned(16))) float sE[HPW][HELIX_CS];    // exp(Lcum_t)
    __shared__ __attribute__((aligned(16))) float sDt[NW][2][HELIX_CS];  // per wave: dt_j, decay_j

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = wave_uniform();
    const int c16 = lane & 15, q = lane >> 4;
    const int hw = wave >> 2, w4 = wave & 3;      // head slot in the workgroup, P block within it
    const int N = p.d_state, P = p.head_dim;
    const int hpg = p.heads_per_group;
    const int npair = (hpg + HPW - 1) / HPW;

    // 1-D grid in the logical order (head block, group, slab, walk segment,
    // sequence). An XCD's share of the logical ids then covers whole walk
    // segments over every group: a group's head blocks share the XCD (and the
    // chunk's B and C in its L2), and the XCD's x reads and y writes are whole
    // token rows of one stretch of a sequence. With the walk segment as the
    // fastest index after the group (an XCD per group, 2 KiB of every 16 KiB
    // token row at config 2) the walk took 66-78 us depending on where y lay
    // in memory; in this order 65-67 us wherever it lies. The walk segment
    // sits below the sequence because with the sequence below it an XCD's
    // share spans every sequence of a batch at one stretch of positions: at
    // 8 x 4096 tokens x 80 heads that walk took 377 us, 346 us in this order.
    const unsigned total = (unsigned)p.n_walk * (unsigned)p.n_group * (unsigned)npair *
                           (unsigned)p.n_pslab * (unsigned)p.n_seq;
    unsigned wid = xcd_logical_id(blockIdx.x, total);
    const int pair = (int)(wid % (unsigned)npair);    wid /= (unsigned)npair;
    const int g    = (int)(wid % (unsigned)p.n_group); wid /= (unsigned)p.n_group;
    const int slab = (int)(wid % (unsigned)p.n_pslab); wid /= (unsigned)p.n_pslab;
    const int seg  = (int)(wid % (unsigned)p.n_walk); wid /= (unsigned)p.n_walk;
    const int seq  = (int)wid;
    // A workgroup of the last block may have fewer heads than HPW: its spare
    // waves walk the block's last head again and store nothing.
    const int hslot = HPW * pair + hw;
    const bool head_ok = hslot < hpg;
    const int h  = g * hpg + min(hslot, hpg - 1);
    const int p0 = slab * HELIX_HD;
    const int pw = min(HELIX_HD, P - p0);

    const int c_begin = seg * p.walk_len;
    const int c_end   = min(c_begin + p.walk_len, p.n_cg);
    if (c_begin >= c_end) return;

    // Decay records of this head, chunk stride n_head * 64 records.
    const float* __restrict__ rec_h = reinterpret_cast<const float*>(
        reinterpret_cast<const char*>(b.pre) + ((long long)seq * p.cpg * p.n_head + h) * (HELIX_CS * HELIX_REC_WALK_BYTES));
    const IO* __restrict__ x_h = reinterpret_cast<const IO*>(b.x) + seq * p.seq_x + h * p.s_x[1] + p0 * p.s_x[2];
    const BIO* __restrict__ B_g = reinterpret_cast<const BIO*>(b.B) + seq * p.seq_b + g * p.s_b[1];
    const BIO* __restrict__ C_g = reinterpret_cast<const BIO*>(b.C) + seq * p.seq_c + g * p.s_c[1];

    const int pp = 16 * w4 + c16;                 // this lane's P column in the slab

    __bf16* const sMh = sM + hw * (HELIX_CS * RSJ);
    // M blocks (jb, tb) = (1, 0) and (3, 2) lie above the diagonal but inside
    // the 32-wide K steps G2 reads: zero. Written once, or with every chunk's
    // M when M shares B's rows.
    const int zoff = [&] {
        const int e2 = 2 * (64 * w4 + lane);      // 0 .. 510: 32 rows x 16 columns
        const int row = e2 >> 4, col = e2 & 15;
        const int t = row < 16 ? row : row + 16;
        const int j = row < 16 ? 16 + col : 48 + col;
        return swz_off<RSJ>(t, j);
    }();
    if constexpr (!M_IN_B) *reinterpret_cast<unsigned*>(&sMh[zoff]) = 0u;

    // B and C are staged once for the workgroup's heads. All NW waves share
    // the 64 rows, RPW each. An instruction covers RPI whole rows, NCH lanes
    // per row: lane holds state indices 8u .. 8u+7, u = lane % NCH, of rows
    // RPW wave + lane / NCH + RPI k. (With lanes spread over eight rows and
    // eight runs instead, the 8-byte LDS writes measured 19 cycles each
    // against 8; the global loads are whole rows too.)
    constexpr int RPW = HELIX_CS / NW;
    constexpr int RPI = 64 / NCH;                 // rows per wave instruction
    constexpr int KQ  = RPW / RPI;
    static_assert(RPI * NCH == 64 && KQ * RPI == RPW, "whole rows per instruction");
    const int ur = lane % NCH;
    const int jrow = RPW * wave + lane / NCH;

    // Issued in the loop's order (runs, then x and dt): the counter state at
    // the loop head is then the same on entry as around the loop, and the
    // wait for the runs never covers the previous chunk's y stores.
    RunsW16<KQ, BIO> runs;
    load_runs_w16<KQ, RPI, BIO>(runs, p, B_g, C_g, c_begin, N, jrow, ur);
    StageW16<IO> st;
    load_stage_w16<IO>(st, p, rec_h, x_h, c_begin, lane, w4, pw);

    // The segment's start state, after the first chunk's loads are issued so
    // that their latency overlaps the prologue's tile loads.
    f32x4 R[NB];
    walk_start_state<NP>(R, p, b, seq, h, slab, seg, p0, pw, pp, q, w4, c16, head_ok);

    // Two barriers per chunk: (1) after staging, (2) after G1 has written M.
    // Whatever a wave stages for chunk c+1 was last read before barrier (2)
    // of chunk c, except dtX^T, which G2 reads after it: dtX^T alternates
    // between two buffers. (With M in B's rows, B's staging must also wait
    // for G2: a third barrier ends the chunk.)
    for (int c = c_begin; c < c_end; ++c) {
        const int t0   = (p.chunk_base + c) * HELIX_CS;
        const int tlen = min(HELIX_CS, p.n_tok - t0);
        const int par  = (c - c_begin) & 1;
        // The next chunk's inputs are loaded as soon as this chunk's copy is
        // consumed; on the last chunk the same chunk is loaded again, so the
        // loop has no branch.
        const int cn = min(c + 1, c_end - 1);

        // ---- B and C of this chunk (loaded during the previous one) -------
        {
            // C is zeroed past tlen and d_state; that is all G1 and G3 need
            // (B rows past tlen only meet zero dtXs columns in G4). With bf16
            // storage a run's elements are already MFMA operands.
            constexpr bool RAW = __is_same(BIO, __bf16);
#pragma unroll
            for (int k = 0; k < KQ; ++k) {
                const int u = ur;
                const int cpos = perm32(8 * u);           // elements 8u+4 .. 8u+7 sit 8 further
                const int j = jrow + RPI * k;
                const unsigned keep = ~(unsigned)(((tlen - 1 - j) | (N - 1 - 8 * u)) >> 31);
                bf16x4 b_lo, b_hi, c_lo, c_hi;
                if constexpr (RAW) {
                    b_lo = __builtin_bit_cast(bf16x4, u32x2{runs.b[k][0][0], runs.b[k][0][1]});
                    b_hi = __builtin_bit_cast(bf16x4, u32x2{runs.b[k][0][2], runs.b[k][0][3]});
                    c_lo = __builtin_bit_cast(bf16x4, u32x2{runs.c[k][0][0] & keep, runs.c[k][0][1] & keep});
                    c_hi = __builtin_bit_cast(bf16x4, u32x2{runs.c[k][0][2] & keep, runs.c[k][0][3] & keep});
                } else {
                    constexpr int WPR = RunsW16<KQ, BIO>::WPR;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        b_lo[e] = to_bf16(run16_elem<BIO, WPR>(runs.b[k], e));
                        b_hi[e] = to_bf16(run16_elem<BIO, WPR>(runs.b[k], 4 + e));
                        c_lo[e] = to_bf16(as_f32(as_u32(run16_elem<BIO, WPR>(runs.c[k], e)) & keep));
                        c_hi[e] = to_bf16(as_f32(as_u32(run16_elem<BIO, WPR>(runs.c[k], 4 + e)) & keep));
                    }
                }
                *reinterpret_cast<bf16x4*>(&sB[swz_off<RS>(j, cpos)]) = b_lo;
                *reinterpret_cast<bf16x4*>(&sB[swz_off<RS>(j, cpos + 8)]) = b_hi;
                *reinterpret_cast<bf16x4*>(&sC[swz_off<RS>(j, cpos)]) = c_lo;
                *reinterpret_cast<bf16x4*>(&sC[swz_off<RS>(j, cpos + 8)]) = c_hi;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sBt[bt_off(8 * u + e, j)] = b_lo[e];
                    sBt[bt_off(8 * u + 4 + e, j)] = b_hi[e];
                }
            }
        }
        load_runs_w16<KQ, RPI, BIO>(runs, p, B_g, C_g, cn, N, jrow, ur);

        // ---- decay record, dtX^T and dtXs^T --------------------------------
        // Pass A's record of token lane: dt (0 past tlen) and Lcum log2(e);
        // L_end is token 63's. exp(L_end - Lcum) weights G4's dtXs (its
        // tokens past tlen have dt 0), exp(Lcum) G3's rows.
        const float dtv = as_f32(st.rec[0]);
        const float l2 = as_f32(st.rec[1]);
        const float l2_end = __builtin_bit_cast(float, __builtin_amdgcn_readlane((int)st.rec[1], 63));
        const float sdec = __builtin_amdgcn_exp2f(l2_end - l2);
        const float a_c = __builtin_amdgcn_exp2f(l2_end);
        {
            // dt and the decay of this wave's 16 tokens, through the wave's own
            // LDS row (one write, four broadcast reads each).
            sDt[wave][0][lane] = dtv;
            sDt[wave][1][lane] = sdec;
            float vx[16], vs[16];
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sDt[wave][0][16 * w4 + 4 * i4]);
                const f32x4 s4 = *reinterpret_cast<const f32x4*>(&sDt[wave][1][16 * w4 + 4 * i4]);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float dx = d4[k] * io_widen<IO>(st.x[4 * i4 + k]);
                    vx[4 * i4 + k] = dx;
                    vs[4 * i4 + k] = s4[k] * dx;
                }
            }
            store16_nat<RSJ>(sXt[par][hw], lane, 16 * w4, vx);
            store16_nat<RSJ>(sXst[hw], lane, 16 * w4, vs);
        }
        if (w4 == 0) {
            sL2[hw][lane] = l2;
            sE[hw][lane] = __builtin_amdgcn_exp2f(l2);
        }
        load_stage_w16<IO>(st, p, rec_h, x_h, cn, lane, w4, pw);
        f32x4 yprev[4];
        if constexpr (YACC) load_y16(yprev, p, b, seq, h, t0, head_ok ? tlen : 0, p0, pw, pp, q);
        __syncthreads();

        // ---- G1: C B^T once for the workgroup's heads (they share B and C);
        // wave w takes blocks idx = w + NW i and writes every head's M^T =
        // (B C^T) . decay block from its registers into that head's M[t][j].
        // Block idx: D[j = 16 jb + 4 q + r][t = 16 tb + c16].
        {
            constexpr int NBLK = (10 + NW - 1) / NW;
            f32x4 d[NBLK];
#pragma unroll
            for (int i = 0; i < NBLK; ++i) {
                const int idx = wave + NW * i;
                if (idx >= 10) break;
                const int tb = g1_tb(idx), jb = g1_jb(idx);
                const int ar = 16 * jb + c16, br = 16 * tb + c16;
                d[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int s = 0; s < KS; ++s)
                    d[i] = mfma16(*reinterpret_cast<const bf16x8*>(&sB[swz_off<RS>(ar, 32 * s + 8 * q)]),
                                  *reinterpret_cast<const bf16x8*>(&sC[swz_off<RS>(br, 32 * s + 8 * q)]), d[i]);
            }
            if constexpr (M_IN_B) {
                __syncthreads();   // every wave's B reads are done
                *reinterpret_cast<unsigned*>(&sMh[zoff]) = 0u;
            }
#pragma unroll
            for (int i = 0; i < NBLK; ++i) {
                const int idx = wave + NW * i;
                if (idx >= 10) break;
                const int tb = g1_tb(idx), jb = g1_jb(idx);
                const int t = 16 * tb + c16;
                const int j0 = 16 * jb + 4 * q;
#pragma unroll
                for (int hh = 0; hh < HPW; ++hh) {
                    const float l_t = sL2[hh][t];
                    const f32x4 lj = *reinterpret_cast<const f32x4*>(&sL2[hh][j0]);
                    bf16x4 m;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        m[r] = to_bf16(keep_if_le(d[i][r] * __builtin_amdgcn_exp2f(l_t - lj[r]), j0 + r, t));
                    *reinterpret_cast<bf16x4*>(&sM[hh * (HELIX_CS * RSJ) + swz_off<RSJ>(t, j0)]) = m;
                }
            }
        }

        // ---- G3: y = exp(Lcum_t) . (C R), R the state before this chunk -----
        f32x4 acc[4];
        {
            bf16x8 rb[KS];
#pragma unroll
            for (int s = 0; s < KS; ++s)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    rb[s][e] = to_bf16(R[2 * s][e]);
                    rb[s][4 + e] = to_bf16(R[2 * s + 1][e]);
                }
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                acc[tb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                const int cr = 16 * tb + c16;
#pragma unroll
                for (int s = 0; s < KS; ++s)
                    acc[tb] = mfma16(*reinterpret_cast<const bf16x8*>(&sC[swz_off<RS>(cr, 32 * s + 8 * q)]), rb[s], acc[tb]);
                const f32x4 e4 = *reinterpret_cast<const f32x4*>(&sE[hw][16 * tb + 4 * q]);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[tb][r] *= e4[r];
            }
        }
        // ---- G4: R <- exp(L_end) R + B^T . dtXs (after G3 has used R) -------
        {
            bf16x8 xs[2];
#pragma unroll
            for (int s = 0; s < 2; ++s) xs[s] = *reinterpret_cast<const bf16x8*>(&sXst[hw][swz_off<RSJ>(pp, 32 * s + 8 * q)]);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                f32x4 rn = R[nb] * a_c;
#pragma unroll
                for (int s = 0; s < 2; ++s)
                    rn = mfma16(*reinterpret_cast<const bf16x8*>(&sBt[bt_off(16 * nb + c16, 32 * s + 8 * q)]), xs[s], rn);
                R[nb] = rn;
            }
        }
        __syncthreads();   // M complete

        // ---- G2: y += M . dtX (causal: t block tb needs j < 16 (tb + 1)) ----
        {
            bf16x8 xb[2];
#pragma unroll
            for (int s = 0; s < 2; ++s) xb[s] = *reinterpret_cast<const bf16x8*>(&sXt[par][hw][swz_off<RSJ>(pp, 32 * s + 8 * q)]);
#pragma unroll
            for (int tb = 0; tb < 4; ++tb)
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    if (s == 1 && tb < 2) continue;
                    const bf16x8 ma = *reinterpret_cast<const bf16x8*>(&sMh[swz_off<RSJ>(16 * tb + c16, 32 * s + 8 * q)]);
                    acc[tb] = mfma16(ma, xb[s], acc[tb]);
                }
        }
        // Reading Pass A's bf16 copies (fp32 storage, BIO bf16): nt alone.
        constexpr int YAUX = sizeof(IO) == 4 && __is_same(BIO, __bf16) ? HELIX_NT_L2 : HELIX_NT;
        if constexpr (YACC) {
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) acc[tb] += yprev[tb];
            store_y16<IO, YAUX, false>(acc, p, b, seq, h, t0, head_ok ? tlen : 0, p0, pw, pp, q);
        } else {
            store_y16<IO, YAUX>(acc, p, b, seq, h, t0, head_ok ? tlen : 0, p0, pw, pp, q);
        }

        if constexpr (M_IN_B) __syncthreads();
    }
}

#define HELIX_PASS_C_WALK16(NP)                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_WG * HELIX_WALK16_HPW(NP)) void helix_scan_walk16_bf16_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk16_impl<NP, HELIX_WALK16_HPW(NP)>(p, b);                                       \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG * HELIX_WALK16_HPW(NP)) void helix_scan_walk16_bf16_bc_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk16_impl<NP, HELIX_WALK16_HPW(NP), float, __bf16>(p, b);                        \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG * HELIX_WALK16_HPW(NP)) void helix_scan_walk16_bf16_bf16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk16_impl<NP, HELIX_WALK16_HPW(NP), __bf16>(p, b);                               \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG * HELIX_WALK16_HPW(NP)) void helix_scan_walk16_bf16_f16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk16_impl<NP, HELIX_WALK16_HPW(NP), _Float16>(p, b);                             \
    }

HELIX_PASS_C_WALK16(64)
HELIX_PASS_C_WALK16(128)
HELIX_PASS_C_WALK16(256)

// The walks of the second and later blocks of state indices (blocks are at
// most HELIX_N_BLOCK = 128 wide): y of each chunk loaded ahead and added.
#define HELIX_PASS_C_WALK16_ACC(NP)                                                             \
    extern "C" __global__ __launch_bounds__(HELIX_WG * HELIX_WALK16_HPW(NP)) void helix_scan_walk16_bf16_acc_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk16_impl<NP, HELIX_WALK16_HPW(NP), float, float, true>(p, b);                   \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG * HELIX_WALK16_HPW(NP)) void helix_scan_walk16_bf16_bc_acc_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk16_impl<NP, HELIX_WALK16_HPW(NP), float, __bf16, true>(p, b);                  \
    }

HELIX_PASS_C_WALK16_ACC(64)
HELIX_PASS_C_WALK16_ACC(128)
