// pass_c_walk.hip -- Pass C on bf16 MFMA, walking the chunks of a segment
// with the state held in registers.
//
// Reference counterpart: helix_chunk_out_mpp_impl<K> (src/kernels/mpp/
// helix_scan_mpp.metal:54-232), which reads each chunk's initial state as a
// bf16 copy that Pass B wrote (Sbf) and computes
//     y = tril(C B^T . decay) (dt x) + exp(Lcum) . (C S_init)
// with bf16 operands and fp32 accumulators.
//
// Here one workgroup owns (seq, segment, HELIX_WALK_HPW heads of one B/C
// group, 64-wide P slab); the heads share the staging of B and C, four waves
// per head. Each head starts from the segment's initial state S_seg(s)
// (fp32, from Pass B) and walks the
// segment's chunks in order, so the per-chunk initial state never touches
// HBM: after producing y for chunk c it advances
//     R <- exp(L_end_c) R + B_c^T . (decay . dt . x)_c          (G4)
// in the same registers, on bf16 operands with fp32 accumulation. R only
// feeds y here; the fp32-accurate carried state and s1 come from Passes A
// and B (Pass A runs its aggregate-only variant).
//
// Wave w owns output tile (t block tb = w >> 1, P block pb = w & 1) and keeps
// its own copy of R[:, pb block] (all N/32 state tiles) in MFMA result
// layout: lane (lo, hi), register r holds R[32nt + 8(r/4) + 4hi + r%4][lo].
// Registers 8q .. 8q+7 of a tile therefore hold, for half hi, the state
// indices 32nt + 16q + {0-3, 8-11} + 4hi. An MFMA's sixteen K slots may hold
// any sixteen indices as long as both operands use the same ones, so every
// k-contiguous operand in LDS is stored in that order: within each group of
// 16, index i sits at position perm16(i) (bits 2 and 3 swapped), and a lane's
// eight K values are one 16-byte read. R feeds G3 straight from registers;
// the G1 result (C.B^T, kept transposed so the lane owns one output row t)
// feeds G2 the same way.
//
// LDS (bf16, k-contiguous, perm16 order): C[t][n] and B[j][n] (G1, G3),
// B^T[n][j] (G4), dtX^T[p][j] (G2) and dtXs^T[p][j] (G4); rows padded by 8.
#include "helix_common.h"

#include "pass_c_stage.h"

// Position of index i inside its group of 16 (bits 2 and 3 swapped).
HELIX_DEV int perm16(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }

// Per-chunk inputs prefetched a chunk ahead: dt for token `lane`, and x for
// tokens 16 wave + i at channel p = lane.
template <typename IO>
struct StageW {
    float dtraw;
    typename IoWord<IO>::type x[16];    // storage form
};

template <typename IO>
__device__ __forceinline__ void load_stage_w(StageW<IO>& st, const HelixScanParams& p,
                                             const float* __restrict__ dt_h,
                                             const IO* __restrict__ x_h, int c, int lane,
                                             int wave, int pw) {
    const int t0   = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const int sdt = (int)p.s_dt[0], sx0 = sgpr_fresh((int)p.s_x[0]), sx2 = (int)p.s_x[2];
    const helix_rsrc rdt = make_rsrc(dt_h + (long long)t0 * p.s_dt[0], ((tlen - 1) * sdt + 1) * 4u);
    const helix_rsrc rx  = make_rsrc(x_h + (long long)t0 * p.s_x[0],
                                     ((tlen - 1) * sx0 + (pw - 1) * sx2 + 1) * (unsigned)sizeof(IO));
    st.dtraw = buf_elem<float>(rdt, min(lane, tlen - 1) * sdt, 0);
    const int xc = min(lane, pw - 1) * sx2;
#pragma unroll
    for (int i = 0; i < 16; ++i) st.x[i] = io_load_word<IO>(rx, xc, min(16 * wave + i, tlen - 1) * sx0);
}

// This lane's B and C runs of one chunk, as loaded: KQ runs of eight state
// indices of row jrow, each two 16-byte words in fp32 storage or one in
// 16-bit storage. Loaded a chunk ahead and widened only when staged.
template <int KQ, typename IO>
struct RunsW {
    static constexpr int WPR = sizeof(IO) == 4 ? 2 : 1;
    u32x4 b[KQ][WPR], c[KQ][WPR];
};

template <int KQ, int QPI, typename IO>
__device__ __forceinline__ void load_runs_w(RunsW<KQ, IO>& r, const HelixScanParams& p,
                                            const IO* __restrict__ B_g, const IO* __restrict__ C_g,
                                            int c, int N, int jrow, int qq) {
    constexpr int ES = (int)sizeof(IO);
    const int t0   = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const int sb0 = sgpr_fresh((int)p.s_b[0]), sc0 = sgpr_fresh((int)p.s_c[0]);
    const helix_rsrc rb = make_rsrc(B_g + (long long)t0 * p.s_b[0], ((tlen - 1) * sb0 + N) * (unsigned)ES);
    const helix_rsrc rc = make_rsrc(C_g + (long long)t0 * p.s_c[0], ((tlen - 1) * sc0 + N) * (unsigned)ES);
    const int jr = min(jrow, tlen - 1);
#pragma unroll
    for (int k = 0; k < KQ; ++k) {
        const int n0 = min(8 * (qq + QPI * k), N - 8);   // d_state % 8 == 0: a run is all in or out
#pragma unroll
        for (int w = 0; w < RunsW<KQ, IO>::WPR; ++w) {
            r.b[k][w] = __builtin_amdgcn_raw_buffer_load_b128(rb, (n0 + jr * sb0) * ES + 16 * w, 0, 0);
            r.c[k][w] = __builtin_amdgcn_raw_buffer_load_b128(rc, (n0 + jr * sc0) * ES + 16 * w, 0, 0);
        }
    }
}

// Element e (0..7) of a run, widened to fp32.
template <typename IO, int WPR>
HELIX_DEV float run_elem(const u32x4 (&w)[WPR], int e) {
    if constexpr (sizeof(IO) == 4) {
        return as_f32(w[e >> 2][e & 3]);
    } else {
        const unsigned v = w[0][e >> 1];
        return io_f32<IO>((unsigned short)((e & 1) ? (v >> 16) : (v & 0xffffu)));
    }
}

// Eight bf16 K values from MFMA result registers r0 .. r0+7.
HELIX_DEV bf16x8 pack8(const f32x16& v, int r0) {
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float f = v[r0 + e];
        o[e] = to_bf16(f);
    }
    return o;
}

// Sixteen consecutive tokens' values written as one perm16-ordered group.
HELIX_DEV void store16_perm(__bf16* row, const float (&v)[16]) {
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        a[e] = to_bf16(v[e]);          // positions 0..3   <- 0..3
        a[4 + e] = to_bf16(v[8 + e]);  // positions 4..7   <- 8..11
        b[e] = to_bf16(v[4 + e]);      // positions 8..11  <- 4..7
        b[4 + e] = to_bf16(v[12 + e]); // positions 12..15 <- 12..15
    }
    *reinterpret_cast<bf16x8*>(row) = a;
    *reinterpret_cast<bf16x8*>(row + 8) = b;
}

// IO: the caller's storage type of x, B, C and y (dt, A and the states are fp32).
template <int NP, typename IO = float>
__device__ __forceinline__ void scan_walk_bf16_impl(const HelixScanParams& p, const HelixScanBuffers& b) {
    constexpr int HPW = HELIX_WALK_HPW(NP);   // heads per workgroup, four waves each
    constexpr int NW  = 4 * HPW;          // waves per workgroup
    constexpr int NT  = NP / 32;          // state tiles per P block
    constexpr int RS  = NP + 8;           // bf16 row stride of C[t][n], B[j][n]
    constexpr int RSJ = HELIX_CS + 8;     // bf16 row stride of B^T[n][j], dtX^T[p][j], dtXs^T[p][j]
    constexpr int NCH = NP / 8;           // 8-element runs per C / B row

    __shared__ __attribute__((aligned(16))) __bf16 sC[HELIX_CS * RS];
    __shared__ __attribute__((aligned(16))) __bf16 sB[HELIX_CS * RS];
    __shared__ __attribute__((aligned(16))) __bf16 sBt[NP * RSJ];
    __shared__ __attribute__((aligned(16))) __bf16 sXt[HPW][HELIX_HD * RSJ];
    __shared__ __attribute__((aligned(16))) __bf16 sXst[HPW][HELIX_HD * RSJ];
    __shared__ __attribute__((aligned(16))) float sL2[HPW][HELIX_CS];   // Lcum_t log2(e), fp32
    __shared__ __attribute__((aligned(16))) float sE[HPW][HELIX_CS];
    __shared__ __attribute__((aligned(16))) float sDt[NW][2][HELIX_CS];  // per wave: dt_j, decay_j

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = wave_uniform(), lo = lane & 31, hi = lane >> 5;
    const int hw = wave >> 2, w4 = wave & 3;      // head slot in the workgroup, role within it
    const int N = p.d_state, P = p.head_dim;
    const int hpg = p.heads_per_group;
    const int npair = (hpg + HPW - 1) / HPW;

    // 1-D grid, a group's head blocks consecutive in the logical order so they
    // share an XCD (and the chunk's B and C in its L2).
    const unsigned total = (unsigned)(p.n_seg * p.n_group * npair * p.n_pslab * p.n_seq);
    unsigned wid = xcd_logical_id(blockIdx.x, total);
    const int pair = (int)(wid % (unsigned)npair);   wid /= (unsigned)npair;
    const int seg  = (int)(wid % (unsigned)p.n_seg); wid /= (unsigned)p.n_seg;
    const int g    = (int)(wid % (unsigned)p.n_group); wid /= (unsigned)p.n_group;
    const int slab = (int)(wid % (unsigned)p.n_pslab);
    const int seq  = (int)(wid / (unsigned)p.n_pslab);
    // A workgroup of the last block may have fewer heads than HPW: its spare
    // waves walk the block's last head again and store nothing.
    const int hslot = HPW * pair + hw;
    const bool head_ok = hslot < hpg;
    const int h  = g * hpg + min(hslot, hpg - 1);
    const int p0 = slab * HELIX_HD;
    const int pw = min(HELIX_HD, P - p0);

    const int c_begin = seg * p.seg_len;
    const int c_end   = min(c_begin + p.seg_len, p.n_cg);
    if (c_begin >= c_end) return;

    const float A_h = b.A[(long long)h * p.s_a];
    const float* __restrict__ dt_h = b.dt + seq * p.seq_dt + h * p.s_dt[1];
    constexpr int ES = (int)sizeof(IO);
    const IO* __restrict__ x_h = reinterpret_cast<const IO*>(b.x) + seq * p.seq_x + h * p.s_x[1] + p0 * p.s_x[2];
    const IO* __restrict__ B_g = reinterpret_cast<const IO*>(b.B) + seq * p.seq_b + g * p.s_b[1];
    const IO* __restrict__ C_g = reinterpret_cast<const IO*>(b.C) + seq * p.seq_c + g * p.s_c[1];

    const int tb = w4 >> 1, pb = w4 & 1;
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

    // B and C are staged once for the workgroup's heads. All NW waves share
    // the 64 rows, RPW each: lane (jj = lane % RPW, qq = lane / RPW) holds
    // state indices 8q .. 8q+7, q = qq + (64/RPW) k, of row RPW wave + jj;
    // RPW consecutive rows per lane group keep the B^T writes contiguous.
    constexpr int RPW = HELIX_CS / NW;
    constexpr int QPI = 64 / RPW;                 // runs per wave instruction
    constexpr int KQ  = NCH / QPI;
    const int jj = lane % RPW, qq = lane / RPW;
    const int jrow = RPW * wave + jj;
    const int jp = perm16(jrow);

    StageW<IO> st;
    load_stage_w<IO>(st, p, dt_h, x_h, c_begin, lane, w4, pw);
    RunsW<KQ, IO> runs;
    load_runs_w<KQ, QPI, IO>(runs, p, B_g, C_g, c_begin, N, jrow, qq);

    // The output tile of chunk c is stored after chunk c+1's B and C loads are
    // issued: the vmcnt counter completes in order and counts stores, so a
    // store issued first would be waited on together with those loads.
    f32x16 y_prev = zero16();

    for (int c = c_begin; c < c_end; ++c) {
        const int t0   = (p.chunk_base + c) * HELIX_CS;
        const int tlen = min(HELIX_CS, p.n_tok - t0);

        // ---- B and C of this chunk, loaded during the previous one ---------
        {
            // Chunk c-1's tile (a full chunk: only the sequence's last chunk is
            // ragged). Unconditional, so every path has the same counter
            // state; on the first chunk no row is valid and the range check
            // drops the stores. The runs were loaded before these stores, so
            // waiting for them does not wait for the stores.
            const bool have_prev = c > c_begin;
            store_y_tile<IO>(y_prev, p, b, seq, h, have_prev ? t0 - HELIX_CS : t0,
                         (have_prev && head_ok) ? HELIX_CS : 0, p0, pw, tb, pb, lo, hi);
            // C is zeroed past tlen and d_state; that is all G1 and G3 need
            // (B rows past tlen only meet zero dtXs columns in G4). With bf16
            // storage a run's elements are already MFMA operands.
            constexpr bool RAW = __is_same(IO, __bf16);
#pragma unroll
            for (int k = 0; k < KQ; ++k) {
                const int q = qq + QPI * k;
                const int cpos = 16 * (q >> 1) + 4 * (q & 1);   // perm16 position of 8q; 8q+4 sits 8 further
                const int j = jrow;
                const unsigned keep = ~(unsigned)(((tlen - 1 - j) | (N - 1 - 8 * q)) >> 31);
                bf16x4 b_lo, b_hi, c_lo, c_hi;
                if constexpr (RAW) {
                    b_lo = __builtin_bit_cast(bf16x4, u32x2{runs.b[k][0][0], runs.b[k][0][1]});
                    b_hi = __builtin_bit_cast(bf16x4, u32x2{runs.b[k][0][2], runs.b[k][0][3]});
                    c_lo = __builtin_bit_cast(bf16x4, u32x2{runs.c[k][0][0] & keep, runs.c[k][0][1] & keep});
                    c_hi = __builtin_bit_cast(bf16x4, u32x2{runs.c[k][0][2] & keep, runs.c[k][0][3] & keep});
                } else {
                    constexpr int WPR = RunsW<KQ, IO>::WPR;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        b_lo[e] = to_bf16(run_elem<IO, WPR>(runs.b[k], e));
                        b_hi[e] = to_bf16(run_elem<IO, WPR>(runs.b[k], 4 + e));
                        c_lo[e] = to_bf16(as_f32(as_u32(run_elem<IO, WPR>(runs.c[k], e)) & keep));
                        c_hi[e] = to_bf16(as_f32(as_u32(run_elem<IO, WPR>(runs.c[k], 4 + e)) & keep));
                    }
                }
                *reinterpret_cast<bf16x4*>(&sB[j * RS + cpos]) = b_lo;
                *reinterpret_cast<bf16x4*>(&sB[j * RS + cpos + 8]) = b_hi;
                *reinterpret_cast<bf16x4*>(&sC[j * RS + cpos]) = c_lo;
                *reinterpret_cast<bf16x4*>(&sC[j * RS + cpos + 8]) = c_hi;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sBt[(8 * q + e) * RSJ + jp] = b_lo[e];
                    sBt[(8 * q + 4 + e) * RSJ + jp] = b_hi[e];
                }
            }
        }

        // ---- decay preamble, dtX^T and dtXs^T -----------------------------------
        // The prefix itself is summed in fp64; the decays that only feed bf16
        // operands (M, dtXs) are formed in fp32 from Lcum log2(e): an fp32
        // difference of two prefixes is good to ~2^-24 of their magnitude,
        // far inside the 2^-9 of a bf16 operand.
        const float dtv = keep_if_lt(helix_dt(p, st.dtraw), lane, tlen);
        const double lcum = wave_incl_sum((double)A_h * (double)dtv);
        const double lend = __shfl(lcum, 63, 64);
        const float sdec = keep_if_lt(exp2_diff(lend, lcum), lane, tlen);
        {
            // dt and the decay of this wave's 16 tokens, through the wave's own
            // LDS row (one write, four broadcast reads each; the wave's LDS
            // accesses complete in order).
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
            store16_perm(&sXt[hw][lane * RSJ + 16 * w4], vx);
            store16_perm(&sXst[hw][lane * RSJ + 16 * w4], vs);
        }
        if (w4 == 0) {
            sL2[hw][lane] = (float)(lcum * 1.4426950408889634074);
            sE[hw][lane] = expf((float)lcum);
        }
        __syncthreads();

        // The next chunk's inputs travel while this one computes. On the last
        // chunk the same chunk is loaded again, so the loop has no branch.
        {
            const int cn = min(c + 1, c_end - 1);
            load_stage_w<IO>(st, p, dt_h, x_h, cn, lane, w4, pw);
            load_runs_w<KQ, QPI, IO>(runs, p, B_g, C_g, cn, N, jrow, qq);
        }

        // ---- G1: CB^T tiles (jb, tb) for jb <= tb, kept as M^T ---------------
        // D'[j][t] = sum_n B[j][n] C[t][n]; lane owns column t = tb*32 + lo,
        // register r holds j = 32 jb + acc_row(r, hi).
        const int t_own = tb * 32 + lo;
        const float l_t = sL2[hw][t_own];
        bf16x8 mA[2][2];                        // [jb][half] A operands of G2
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
            if (jb > tb) break;
            f32x16 d = zero16();
            // Operands of step s+1 are read before step s's MFMA issues.
            const __bf16* arow = &sB[(jb * 32 + lo) * RS + 8 * hi];
            const __bf16* brow = &sC[t_own * RS + 8 * hi];
            bf16x8 av = *reinterpret_cast<const bf16x8*>(arow);
            bf16x8 bv = *reinterpret_cast<const bf16x8*>(brow);
#pragma unroll
            for (int s = 0; s < NP / 16; ++s) {
                bf16x8 an = av, bn = bv;
                if (s + 1 < NP / 16) {
                    an = *reinterpret_cast<const bf16x8*>(arow + 16 * (s + 1));
                    bn = *reinterpret_cast<const bf16x8*>(brow + 16 * (s + 1));
                }
                d = mfma_bf16(av, bv, d);
                av = an;
                bv = bn;
            }
            // M[t][j] = CB[t][j] exp(Lcum_t - Lcum_j), zero above the diagonal;
            // registers 4q .. 4q+3 are rows j0 .. j0+3, one 16-byte read.
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int j0 = jb * 32 + 8 * q + 4 * hi;
                const f32x4 lj = *reinterpret_cast<const f32x4*>(&sL2[hw][j0]);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float v = d[4 * q + k];
                    d[4 * q + k] = keep_if_le(v * __builtin_amdgcn_exp2f(l_t - lj[k]), j0 + k, t_own);
                }
            }
            mA[jb][0] = pack8(d, 0);
            mA[jb][1] = pack8(d, 8);
        }

        // ---- G3: y = C . R (state before this chunk), row scale, G2. The
        // tile is stored as coalesced 4-byte writes (a wave covers two
        // 128-byte row runs per store); a transposed tile stored as 16-byte
        // writes scatters each store over 64 rows and measured 3x slower. ----
        f32x16 acc = zero16();
        {
            // All of this lane's C row operands first (NT x 2 reads), then the MFMAs.
            bf16x8 ca[NT][2];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int half = 0; half < 2; ++half)
                    ca[nt][half] = *reinterpret_cast<const bf16x8*>(&sC[t_own * RS + nt * 32 + 16 * half + 8 * hi]);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int half = 0; half < 2; ++half) acc = mfma_bf16(ca[nt][half], pack8(R[nt], 8 * half), acc);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] *= sE[hw][tb * 32 + acc_row(r, hi)];
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
            if (jb > tb) break;
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const bf16x8 bv = *reinterpret_cast<const bf16x8*>(&sXt[hw][pp * RSJ + jb * 32 + 16 * half + 8 * hi]);
                acc = mfma_bf16(mA[jb][half], bv, acc);
            }
        }
        y_prev = acc;

        // ---- G4: R <- exp(L_end) R + B^T . dtXs --------------------------------
        const float a_c = expf((float)lend);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) R[nt] *= a_c;
        {
            // K step outermost: the NT tiles' MFMAs are independent, so each
            // step's reads are issued while the previous step's MFMAs run.
            bf16x8 xs = *reinterpret_cast<const bf16x8*>(&sXst[hw][pp * RSJ + 8 * hi]);
            bf16x8 bt[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) bt[nt] = *reinterpret_cast<const bf16x8*>(&sBt[(nt * 32 + lo) * RSJ + 8 * hi]);
#pragma unroll
            for (int s = 0; s < HELIX_CS / 16; ++s) {
                bf16x8 xn = xs, bn[NT];
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) bn[nt] = bt[nt];
                if (s + 1 < HELIX_CS / 16) {
                    xn = *reinterpret_cast<const bf16x8*>(&sXst[hw][pp * RSJ + 16 * (s + 1) + 8 * hi]);
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
                        bn[nt] = *reinterpret_cast<const bf16x8*>(&sBt[(nt * 32 + lo) * RSJ + 16 * (s + 1) + 8 * hi]);
                }
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) R[nt] = mfma_bf16(bt[nt], xs, R[nt]);
                xs = xn;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) bt[nt] = bn[nt];
            }
        }
        __syncthreads();
    }
    {
        const int tl0  = (p.chunk_base + c_end - 1) * HELIX_CS;
        store_y_tile<IO>(y_prev, p, b, seq, h, tl0, head_ok ? min(HELIX_CS, p.n_tok - tl0) : 0, p0, pw, tb, pb,
                         lo, hi);
    }
}

#define HELIX_PASS_C_WALK(NP)                                                                   \
    extern "C" __global__ __launch_bounds__(HELIX_WG * HELIX_WALK_HPW(NP)) void helix_scan_walk_bf16_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk_bf16_impl<NP>(p, b);                                                          \
    }

// 16-bit storage of x, B, C and y (io_dtype BF16 / F16).
#define HELIX_PASS_C_WALK_IO(NP)                                                                \
    extern "C" __global__ __launch_bounds__(HELIX_WG * HELIX_WALK_HPW(NP)) void helix_scan_walk_bf16_bf16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk_bf16_impl<NP, __bf16>(p, b);                                                  \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG * HELIX_WALK_HPW(NP)) void helix_scan_walk_bf16_f16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk_bf16_impl<NP, _Float16>(p, b);                                                \
    }

HELIX_PASS_C_WALK(64)
HELIX_PASS_C_WALK(128)
HELIX_PASS_C_WALK(256)
HELIX_PASS_C_WALK_IO(64)
HELIX_PASS_C_WALK_IO(128)
HELIX_PASS_C_WALK_IO(256)
