// pass_c_walk_x6.hip -- the fp32 path's Pass C: the chunk walk on bf16x6 products.
//
// Reference counterpart: helix_chunk_out_f32 (src/kernels/
// helix_scan_multipass.metal:225-361). Like the bf16 path's walk
// (pass_c_walk16.hip), one workgroup walks a segment of chunks from the
// segment's start state S_seg (Pass B) and forms every chunk's own start
// state R on the way, producing per chunk
//     y = tril(C B^T . decay) (dt x) + exp(Lcum) . (C R)        (G1, G2, G3)
//     R <- exp(L_end) R + B^T . (decay . dt . x)                  (G4)
// Here every product keeps fp32 accuracy: v_mfma_f32_16x16x32_bf16 over
// operands split into three bf16 parts (six products, fp32 accumulation),
// and R stays in fp32 registers. Against the chunk-parallel bf16x6 Pass C
// (pass_c_x6.hip), whose per-chunk start states Pass A writes and Pass C
// reads back, the walk moves half the bytes.
//
// Workgroup: (seq, walk segment, two heads of one B/C group, 64-wide P slab),
// eight waves; wave (hw, w4) owns P columns 16 w4 .. 16 w4 + 15 of head hw:
//   - R[n][p] for its 16 columns: NP/16 result tiles, register r of tile nb
//     holding R[16 nb + 4 (lane/16) + r][p];
//   - G3 and G4 on those tiles, G2 on its columns;
//   - G1 (C B^T, the same for both heads) split over the eight waves by
//     16 x 16 block; each head's M = C B^T . decay shared through LDS.
// K order: within each group of 32 state indices, index 16 h + 4 q + r sits at
// K position 8 q + 4 h + r (perm32) in the C and B rows, so R's registers are
// G3's operand as they stand (the layout of the bf16 walk).
//
// LDS, three bf16 planes per operand in the x6_off layout (no padding):
//   C    [64 t][NP n]   perm32 n order             G1, G3
//   B    [64 j][NP n]   perm32 n order             G1; afterwards the region
//   M    [64 t][64 j]   one per head               holds the heads' M (G2)
//   B^T  [NP n][64 j]   natural n order            G4
// and the heads' decay records: 145 KiB at d_state 128 (one workgroup per
// CU), 98 KiB at d_state 64.
// The B operands of G2 and G4 (dt x and decay dt x at the lane's own column
// and K tokens) and of G3 (R) are split in registers.
#include "helix_common.h"

#include "pass_c_stage.h"

// Six 16 x 16 x 32 products of split operands a[3] x b[3], smallest terms first.
HELIX_DEV f32x4 wx6_mfma(const bf16x8 (&a)[3], const bf16x8 (&b)[3], f32x4 acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], b[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[0], acc, 0, 0, 0);
    return acc;
}

// v, opaque to the optimizer (it stays in a VGPR and is not known to be
// loop-invariant).
HELIX_DEV int vgpr_opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// K position of state index i inside its group of 32: 16 h + 4 q + r -> 8 q + 4 h + r.
HELIX_DEV int wx6_perm32(int i) {
    return (i & ~31) | (8 * ((i >> 2) & 3) + 4 * ((i >> 4) & 1) + (i & 3));
}

// G1 block idx (0..9) of the lower triangle of the 4 x 4 grid of 16 x 16
// blocks: (tb, jb) = (0,0) (1,0) (1,1) (2,0) (2,1) (2,2) (3,0) ...
HELIX_DEV int wx6_tb(int idx) { return (idx >= 1) + (idx >= 3) + (idx >= 6); }
HELIX_DEV int wx6_jb(int idx) {
    const int tb = wx6_tb(idx);
    return idx - tb * (tb + 1) / 2;
}

// This lane's B and C runs of one chunk (fp32) of rows j0 and j0 + 1: NH
// 16-byte words per row, state indices 8u + 4 hh .. + 3 for hh = 0 .. NH - 1
// (d_state 128: NH = 2, the whole run 8u .. 8u + 7) or for hh = hf alone
// (d_state 64: NH = 1, lanes 8 apart take the run's two halves).
template <int NH>
struct RunsWX6 {
    u32x4 b[2][NH], c[2][NH];
};

template <int NH>
__device__ __forceinline__ void load_runs_x6(RunsWX6<NH>& r, const HelixScanParams& p, const float* __restrict__ B_g,
                                             const float* __restrict__ C_g, int c, int N, int j0, int u, int hf) {
    const int t0   = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const int sb0 = sgpr_fresh((int)p.s_b[0]), sc0 = sgpr_fresh((int)p.s_c[0]);
    const helix_rsrc rb = make_rsrc(B_g + (long long)t0 * p.s_b[0], ((tlen - 1) * sb0 + N) * 4u);
    const helix_rsrc rc = make_rsrc(C_g + (long long)t0 * p.s_c[0], ((tlen - 1) * sc0 + N) * 4u);
    const int n0 = min(8 * u, N - 8);   // d_state % 8 == 0: a run is all in or out
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int jr = min(j0 + k, tlen - 1);
#pragma unroll
        for (int w = 0; w < NH; ++w) {
            const int hh = NH == 2 ? w : hf;
            r.b[k][w] = __builtin_amdgcn_raw_buffer_load_b128(rb, (n0 + jr * sb0) * 4 + 16 * hh, 0, 0);
            r.c[k][w] = __builtin_amdgcn_raw_buffer_load_b128(rc, (n0 + jr * sc0) * 4 + 16 * hh, 0, 0);
        }
    }
}

// The decay record of token lane (store_decay_record64: dt, exp(Lcum), Lcum
// in fp64) and x at this lane's P column for its K tokens j = 32 s + 8 q + e
// (s = 0, 1; e = 0..7), prefetched a chunk ahead. YT (no records): the raw dt
// of token lane instead.
struct StageWX6 {
    u32x4 rec;
    float dtraw;
    float x[16];
};

template <bool YT>
__device__ __forceinline__ void load_stage_x6(StageWX6& st, const HelixScanParams& p, const float* __restrict__ rec_h,
                                              const float* __restrict__ dt_h, const float* __restrict__ x_h, int c,
                                              int lane, int q, int pp, int pw) {
    const int t0   = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const int sx0 = sgpr_fresh((int)p.s_x[0]), sx2 = (int)p.s_x[2];
    const helix_rsrc rx = make_rsrc(x_h + (long long)t0 * p.s_x[0], ((tlen - 1) * sx0 + (pw - 1) * sx2 + 1) * 4u);
    if constexpr (YT) {
        const int sdt = (int)p.s_dt[0];
        const helix_rsrc rdt = make_rsrc(dt_h + (long long)t0 * p.s_dt[0], ((tlen - 1) * sdt + 1) * 4u);
        st.dtraw = buf_f32(rdt, min(lane, tlen - 1) * sdt * 4, 0);
    } else {
        const helix_rsrc rr = make_rsrc(rec_h + (long long)c * p.n_head * (HELIX_CS * 4), HELIX_CS * 16u);
        st.rec = __builtin_amdgcn_raw_buffer_load_b128(rr, lane * 16, 0, 0);
    }
    // Rows past tlen read 0 (past the resource's range) or, with strides under
    // which a token row is shorter than the slab, another element of the
    // chunk: dt is 0 for them either way.
    const int xv = min(pp, pw - 1) * sx2 + 8 * q * sx0;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) st.x[8 * s + e] = buf_elem<float>(rx, xv, (32 * s + e) * sx0);
}

// YT: the single pass run as the three passes without scratch
// (HelixScanParams::ytile): the start state comes from y (walk_start_state)
// and the decay preamble is formed here from dt, as Pass A forms its records
// (softplus, fp64 wave scan), since there are no records.
// YACC: the walk of a block of state indices after the first (p.y_acc): y of
// each chunk is loaded with the next chunk's inputs and added to the chunk's
// result.
template <int NP, bool YT = false, bool YACC = false>
__device__ __forceinline__ void scan_walk_x6_impl(const HelixScanParams& p, const HelixScanBuffers& b) {
    static_assert(NP == 64 || NP == 128, "d_state 64 or 128");
    // Staging lanes: 16 per pair of rows; a run of eight state indices per
    // lane at d_state 128 (NH = 2 words per row), half a run at 64 (NH = 1).
    constexpr int NH = NP / 64;
    constexpr int HPW = 2;                     // heads per workgroup, four waves each
    constexpr int NB  = NP / 16;               // 16-row state tiles of R
    constexpr int KS  = NP / 32;               // K steps over the state
    constexpr int NT32 = NP / 32;              // 32 x 32 tiles of the slab tile layout
    constexpr int NCH = NP / 8;                // 16-byte chunks per C / B row
    constexpr int PL_CB = 3 * HELIX_CS * NP;   // C (or B) planes, elements
    constexpr int PL_M  = 3 * HELIX_CS * HELIX_CS;
    constexpr int PF = 2;                      // products an operand read runs ahead
    __shared__ __attribute__((aligned(16))) __bf16 sC[PL_CB];
    __shared__ __attribute__((aligned(16))) __bf16 sBt[3 * NP * HELIX_CS];   // B^T[n][j] planes
    __shared__ __attribute__((aligned(16))) __bf16 sM[HPW * PL_M];     // each head's M[t][j] planes
    __shared__ __attribute__((aligned(16))) float sDt[HPW][HELIX_CS];    // dt_j (0 past tlen)
    __shared__ __attribute__((aligned(16))) float sSd[HPW][HELIX_CS];    // exp(L_end - Lcum_j)
    __shared__ __attribute__((aligned(16))) float sE[HPW][HELIX_CS];     // exp(Lcum_t)
    __shared__ __attribute__((aligned(16))) double sL[HPW][HELIX_CS];    // Lcum_t

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = wave_uniform();
    const int hw = wave >> 2, w4 = wave & 3;   // head slot, P block within it
    const int N = p.d_state, P = p.head_dim;
    const int hpg = p.heads_per_group;
    const int npair = (hpg + HPW - 1) / HPW;

    // 1-D grid in the logical order (head block, group, slab, walk segment,
    // sequence). An XCD's share of the logical ids then covers whole walk
    // segments over every group: a group's head blocks share the XCD (and the
    // chunk's B and C in its L2), and the XCD's x reads and y writes are whole
    // token rows of one stretch of a sequence. With the walk segment as the
    // fastest index after the group (an XCD per group, 2 KiB of every 16 KiB
    // token row at config 2) the fp32 path took 212-215 us; 207-210 us in this
    // order. The walk segment sits below the sequence, as in the bf16 walk,
    // so that an XCD's share stays within one sequence of a batch.
    const unsigned total = (unsigned)p.n_walk * (unsigned)p.n_group * (unsigned)npair *
                           (unsigned)p.n_pslab * (unsigned)p.n_seq;
    unsigned wid = xcd_logical_id(blockIdx.x, total);
    const int pair = (int)(wid % (unsigned)npair);    wid /= (unsigned)npair;
    const int g    = (int)(wid % (unsigned)p.n_group); wid /= (unsigned)p.n_group;
    const int slab = (int)(wid % (unsigned)p.n_pslab); wid /= (unsigned)p.n_pslab;
    const int seg  = (int)(wid % (unsigned)p.n_walk); wid /= (unsigned)p.n_walk;
    const int seq  = (int)wid;
    // A workgroup of the last pair may have one head: its spare waves walk
    // that head again and store nothing.
    const int hslot = HPW * pair + hw;
    const bool head_ok = hslot < hpg;
    const int h  = g * hpg + min(hslot, hpg - 1);
    const int p0 = slab * HELIX_HD;
    const int pw = min(HELIX_HD, P - p0);

    const int c_begin = seg * p.walk_len;
    const int c_end   = min(c_begin + p.walk_len, p.n_cg);
    if (c_begin >= c_end) return;

    const float* __restrict__ rec_h = YT ? nullptr : b.pre + ((long long)seq * p.cpg * p.n_head + h) * (HELIX_CS * 4);
    const float* __restrict__ dt_h = b.dt + seq * p.seq_dt + h * p.s_dt[1];
    const float A_h = YT ? b.A[(long long)h * p.s_a] : 0.0f;
    const float* __restrict__ x_h = b.x + seq * p.seq_x + h * p.s_x[1] + p0 * p.s_x[2];
    const float* __restrict__ B_g = b.B + seq * p.seq_b + g * p.s_b[1];
    const float* __restrict__ C_g = b.C + seq * p.seq_c + g * p.s_c[1];

    // Staging: lane (c16, rr) holds its run's state indices (RunsWX6) of rows
    // j0 and j0 + 1 (the wave's eight rows, 16 lanes per pair). A chunk's planes are staged
    // while the previous chunk's products run: C once G1 and G3 are done with
    // it, B once G4 is. C is zeroed past tlen and d_state, which is all G1 and
    // G3 need; B rows past tlen only meet dt = 0 columns in G4.
    // Word w of a run holds state indices 8u + 4 hh .. + 3, at K position
    // cpos + 8 hh (perm32 keeps each group of four together).
    auto half_of = [&](int w, int hf) { return NH == 2 ? w : hf; };
    auto stage_c = [&](const RunsWX6<NH>& rn, int tl, int j0, int u, int hf, int cpos) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int j = j0 + k;
            const unsigned keep = ~(unsigned)(((tl - 1 - j) | (N - 1 - 8 * u)) >> 31);
#pragma unroll
            for (int w = 0; w < NH; ++w) {
                u32x2 cq[3];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    unsigned c0, c1, c2;
                    split3_pair(as_f32(rn.c[k][w][2 * e] & keep), as_f32(rn.c[k][w][2 * e + 1] & keep), c0, c1, c2);
                    cq[0][e] = c0;
                    cq[1][e] = c1;
                    cq[2][e] = c2;
                }
                const int pos = cpos + 8 * half_of(w, hf);
#pragma unroll
                for (int pl = 0; pl < 3; ++pl)
                    *reinterpret_cast<u32x2*>(&sC[x6_off<HELIX_CS, NCH>(pl, j, pos >> 3) + (pos & 7)]) = cq[pl];
            }
        }
    };
    // B's split planes, bw[row k][plane][pair e] (state indices 8u + 4 hh +
    // 2 (e % 2), +1 for word w = e / 2).
    auto split_b = [&](const RunsWX6<NH>& rn, unsigned (&bw)[2][3][2 * NH]) {
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
            for (int e = 0; e < 2 * NH; ++e)
                split3_pair(as_f32(rn.b[k][e >> 1][2 * (e & 1)]), as_f32(rn.b[k][e >> 1][2 * (e & 1) + 1]),
                            bw[k][0][e], bw[k][1][e], bw[k][2][e]);
    };
    // B^T[n][j0 .. j0 + 1] (natural n order): the halves of rows j0 and
    // j0 + 1 as one 4-byte store.
    auto write_bt = [&](const unsigned (&bw)[2][3][2 * NH], int j0, int u, int hf) {
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
#pragma unroll
            for (int e = 0; e < 4 * NH; ++e) {
                const unsigned wa = bw[0][pl][e >> 1], wb = bw[1][pl][e >> 1];
                const unsigned v = (e & 1) ? ((wa >> 16) | (wb & 0xffff0000u)) : ((wa & 0xffffu) | (wb << 16));
                const int n = 8 * u + 4 * half_of(e >> 2, hf) + (e & 3);
                *reinterpret_cast<unsigned*>(&sBt[x6_off<NP, 8>(pl, n, j0 >> 3) + (j0 & 7)]) = v;
            }
    };
    auto tlen_of = [&](int c) { return min(HELIX_CS, p.n_tok - (p.chunk_base + c) * HELIX_CS); };

    RunsWX6<NH> runs;
    unsigned bw[2][3][2 * NH];
    StageWX6 st;
    {
        const int c16 = lane & 15, rr = lane >> 4, j0 = 8 * wave + 2 * rr;
        const int u = NH == 2 ? c16 : (c16 & 7), hf = NH == 2 ? 0 : (c16 >> 3);
        load_runs_x6<NH>(runs, p, B_g, C_g, c_begin, N, j0, u, hf);
        load_stage_x6<YT>(st, p, rec_h, dt_h, x_h, c_begin, lane, rr, 16 * w4 + c16, pw);
        stage_c(runs, tlen_of(c_begin), j0, u, hf, wx6_perm32(8 * u));
        split_b(runs, bw);
        load_runs_x6<NH>(runs, p, B_g, C_g, min(c_begin + 1, c_end - 1), N, j0, u, hf);
    }

    // The segment's start state: S_seg from Pass B, or Pass B's recurrence
    // over Pass A's aggregates run here (p.fuse_b).
    f32x4 R[NB];
    {
        const int q = lane >> 4, c16 = lane & 15;
        walk_start_state<NP, YT>(R, p, b, seq, h, slab, seg, p0, pw, 16 * w4 + c16, q, w4, c16, head_ok);
        if constexpr (YT) {
            // The start state lies in y's rows that this workgroup's waves
            // overwrite from the first chunk on: every wave has it in
            // registers before the first barrier, which comes before any y
            // store.
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                asm volatile("" ::"v"(R[nb][0]), "v"(R[nb][1]), "v"(R[nb][2]), "v"(R[nb][3]));
        }
    }

    __bf16* const sMh = sM + hw * PL_M;

    // Three barriers per chunk: (1) the chunk's planes and records are staged;
    // (2) M is written and G1 and G3 are done with C (the next chunk's C
    // planes are staged behind it); (3) G1 and G4 are done with B^T (the next
    // chunk's B^T planes are written at the top of the loop). G2 reads M after
    // (2); the next chunk writes M only after its (1).
    for (int c = c_begin; c < c_end; ++c) {
        const int t0   = (p.chunk_base + c) * HELIX_CS;
        const int tlen = tlen_of(c);
        // On the last chunk the next chunk is this one again: no branch.
        const int cn = min(c + 1, c_end - 1);
        // Lane-derived indices, formed anew in every chunk: hoisted out of the
        // loop, the LDS addresses made from them would not fit the registers.
        const int ln = vgpr_opaque(lane);
        const int c16 = ln & 15, q = ln >> 4;  // MFMA operand row, K slot group
        const int u = NH == 2 ? c16 : (c16 & 7), hf = NH == 2 ? 0 : (c16 >> 3);   // staging run, its half
        const int rr = q;                      // staging row pair
        const int j0 = 8 * wave + 2 * rr;
        const int cpos = wx6_perm32(8 * u);    // K position of 8u; 8u + 4 sits 8 further
        const int pp = 16 * w4 + c16;          // this lane's P column in the slab

        write_bt(bw, j0, u, hf);

        // ---- decay records of the two heads --------------------------------
        float a_c = 0.0f;
        if constexpr (YT) {
            // dt (0 past tlen), Lcum in fp64 and its exponentials, as Pass A's
            // hb_preamble forms the records, by one wave of each head: wave
            // w4 == hw, so the two heads' preambles run on different SIMDs.
            // The others read exp(L_end) (token 63's exp(Lcum)) from sE after
            // the barrier below.
            if (w4 == hw) {
                const float dtv = keep_if_lt(helix_dt(p, st.dtraw), lane, tlen);
                const double lcum = wave_incl_sum((double)A_h * (double)dtv);
                const double lend = bcast(lcum, 63);
                sDt[hw][lane] = dtv;
                sE[hw][lane] = expf((float)lcum);
                sSd[hw][lane] = exp2_diff(lend, lcum);
                sL[hw][lane] = lcum;
            }
        } else {
            if (w4 == 0) {
                const double lcum = __builtin_bit_cast(double, (unsigned long long)st.rec[2] |
                                                                   ((unsigned long long)st.rec[3] << 32));
                const double lend = __builtin_bit_cast(
                    double, (unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)st.rec[2], 63) |
                                ((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)st.rec[3], 63) << 32));
                sDt[hw][lane] = as_f32(st.rec[0]);
                sE[hw][lane] = as_f32(st.rec[1]);
                sSd[hw][lane] = exp2_diff(lend, lcum);
                sL[hw][lane] = lcum;
            }
            // exp(L_end) = exp(Lcum) of token 63.
            a_c = __builtin_bit_cast(float, __builtin_amdgcn_readlane((int)st.rec[1], 63));
        }
        __syncthreads();   // (1)
        if constexpr (YT) a_c = sE[hw][HELIX_CS - 1];

        // dt x at (K token j = 32 s + 8 q + e, column pp); G4 scales it by the
        // decay when it needs it.
        float xb[2][8];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int h4 = 0; h4 < 2; ++h4) {
                const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sDt[hw][32 * s + 8 * q + 4 * h4]);
#pragma unroll
                for (int k = 0; k < 4; ++k) xb[s][4 * h4 + k] = d4[k] * st.x[8 * s + 4 * h4 + k];
            }
        // The scheduling fences keep each prefetch's loads after the last use
        // of the registers they fill, and each staging step after the barrier
        // that frees its LDS: hoisted, they wait on loads still in flight.
        __builtin_amdgcn_sched_barrier(0);
        load_stage_x6<YT>(st, p, rec_h, dt_h, x_h, cn, lane, q, pp, pw);
        f32x4 yprev[4];
        if constexpr (YACC) load_y16(yprev, p, b, seq, h, t0, head_ok ? tlen : 0, p0, pw, pp, q);

        // ---- G1: D[j][t] = (B C^T) of blocks idx = wave, wave + 8 -----------
        // Block idx: D[j = 16 jb + 4 q + r][t = 16 tb + c16].
        f32x4 d[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = wave + 8 * i;
            d[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if (idx < 10) {
                const int tb = wx6_tb(idx), jb = wx6_jb(idx);
#pragma unroll
                for (int s = 0; s < KS; ++s) {
                    // B rows j = 16 jb + c16 by transpose reads of B^T: K slot
                    // 4 h + r of lane group q is C's column 32 s + 8 q + 4 h + r,
                    // state index 32 s + 16 h + 4 q + r (perm32); lane 4 r + v
                    // names that row of B^T and tokens 16 jb + 4 v .. + 3.
                    bf16x8 av[3], bv[3];
                    {
                        const int jc = 16 * jb + 4 * (c16 & 3);
                        const int nr = 32 * s + 4 * q + (c16 >> 2);
#pragma unroll
                        for (int pl = 0; pl < 3; ++pl) {
                            const u32x2 lo = lds_read_tr16(&sBt[x6_off<NP, 8>(pl, nr, jc >> 3) + (jc & 7)]);
                            const u32x2 hi = lds_read_tr16(&sBt[x6_off<NP, 8>(pl, nr + 16, jc >> 3) + (jc & 7)]);
                            av[pl] = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
                        }
                    }
                    x6_read<HELIX_CS, NCH>(sC, 16 * tb + c16, 4 * s + q, bv);
                    d[i] = wx6_mfma(av, bv, d[i]);
                }
            }
        }

        // ---- M[t][j] = (C B^T)[t][j] exp(Lcum_t - Lcum_j), j <= t, per head --
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = wave + 8 * i;
            if (idx < 10) {
                const int tb = wx6_tb(idx), jb = wx6_jb(idx);
                const int t = 16 * tb + c16;
                const int jq = 16 * jb + 4 * q;
#pragma unroll
                for (int hh = 0; hh < HPW; ++hh) {
                    const double lt = sL[hh][t];
                    float m[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        m[r] = keep_if_le(d[i][r] * exp2_diff(lt, sL[hh][jq + r]), jq + r, t);
                    u32x2 mq[3];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        unsigned w0, w1, w2;
                        split3_pair(m[2 * e], m[2 * e + 1], w0, w1, w2);
                        mq[0][e] = w0;
                        mq[1][e] = w1;
                        mq[2][e] = w2;
                    }
#pragma unroll
                    for (int pl = 0; pl < 3; ++pl)
                        *reinterpret_cast<u32x2*>(&sM[hh * PL_M + x6_off<HELIX_CS, 8>(pl, t, jq >> 3) + (jq & 7)]) =
                            mq[pl];
                }
            }
        }

        // ---- G3: y = exp(Lcum_t) . (C R), R the state before this chunk -----
        // Products (s, tb) in order; the C planes of a product are read PF
        // products ahead, and R's split for the next K step during this one.
        f32x4 acc[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) acc[tb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        {
            auto split_r = [&](int s, bf16x8 (&rp)[3]) {
                float rv[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    rv[e] = R[2 * s][e];
                    rv[4 + e] = R[2 * s + 1][e];
                }
                x6_split8(rv, rp);
            };
            constexpr int NI = 4 * KS;
            bf16x8 cv[PF + 1][3], rp[2][3];
#pragma unroll
            for (int k = 0; k < PF; ++k) x6_read<HELIX_CS, NCH>(sC, 16 * (k % 4) + c16, 4 * (k / 4) + q, cv[k]);
            split_r(0, rp[0]);
#pragma unroll
            for (int it = 0; it < NI; ++it) {
                const int s = it / 4, tb = it % 4;
                const int nx = it + PF;
                if (nx < NI) x6_read<HELIX_CS, NCH>(sC, 16 * (nx % 4) + c16, 4 * (nx / 4) + q, cv[nx % (PF + 1)]);
                if (tb == 1 && s + 1 < KS) split_r(s + 1, rp[(s + 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);
                acc[tb] = wx6_mfma(cv[it % (PF + 1)], rp[s & 1], acc[tb]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            const f32x4 e4 = *reinterpret_cast<const f32x4*>(&sE[hw][16 * tb + 4 * q]);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[tb][r] *= e4[r];
        }
        __syncthreads();   // (2)

        __builtin_amdgcn_sched_barrier(0);
        stage_c(runs, tlen_of(cn), j0, u, hf, cpos);

        // ---- G4: R <- exp(L_end) R + B^T . (decay dt x) (after G3 used R) ---
        // Products (s, nb) in order, B^T's planes read PF products ahead.
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) R[nb] *= a_c;
        {
            auto split_x = [&](int s, bf16x8 (&xp)[3]) {
                float xs[8];
#pragma unroll
                for (int h4 = 0; h4 < 2; ++h4) {
                    const f32x4 s4 = *reinterpret_cast<const f32x4*>(&sSd[hw][32 * s + 8 * q + 4 * h4]);
#pragma unroll
                    for (int k = 0; k < 4; ++k) xs[4 * h4 + k] = s4[k] * xb[s][4 * h4 + k];
                }
                x6_split8(xs, xp);
            };
            auto read_bt = [&](int s, int nb, bf16x8 (&bt)[3]) {
                x6_read<NP, 8>(sBt, 16 * nb + c16, 4 * s + q, bt);
            };
            constexpr int NI = 2 * NB;
            bf16x8 bt[PF + 1][3], xp[2][3];
#pragma unroll
            for (int k = 0; k < PF; ++k) read_bt(k / NB, k % NB, bt[k]);
            split_x(0, xp[0]);
#pragma unroll
            for (int it = 0; it < NI; ++it) {
                const int s = it / NB, nb = it % NB;
                const int nx = it + PF;
                if (nx < NI) read_bt(nx / NB, nx % NB, bt[nx % (PF + 1)]);
                if (nb == 1 && s == 0) split_x(1, xp[1]);
                __builtin_amdgcn_sched_barrier(0);
                R[nb] = wx6_mfma(bt[it % (PF + 1)], xp[s], R[nb]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        split_b(runs, bw);
        __builtin_amdgcn_sched_barrier(0);
        load_runs_x6<NH>(runs, p, B_g, C_g, min(c + 2, c_end - 1), N, j0, u, hf);

        // ---- G2: y += M . dtX (t block tb needs j < 16 (tb + 1)) -----------
        // K step s covers j blocks 2s and 2s + 1; for tb = 0 and 2 the second
        // lies above the diagonal (lanes q >= 2), where M was not written.
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            bf16x8 xp[3];
            x6_split8(xb[s], xp);
#pragma unroll
            for (int tb = 2 * s; tb < 4; ++tb) {
                bf16x8 mv[3];
                x6_read<HELIX_CS, 8>(sMh, 16 * tb + c16, 4 * s + q, mv);
                if (tb == 2 * s) {
                    const unsigned keep = q < 2 ? ~0u : 0u;
#pragma unroll
                    for (int pl = 0; pl < 3; ++pl)
                        mv[pl] = __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, mv[pl]) & keep);
                }
                acc[tb] = wx6_mfma(mv, xp, acc[tb]);
            }
        }
        if constexpr (YACC) {
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) acc[tb] += yprev[tb];
            store_y16<float, HELIX_NT, false>(acc, p, b, seq, h, t0, head_ok ? tlen : 0, p0, pw, pp, q);
        } else {
            store_y16<float>(acc, p, b, seq, h, t0, head_ok ? tlen : 0, p0, pw, pp, q);
        }
        __syncthreads();   // (3)
    }
}

#define HELIX_PASS_C_WALK_X6(NP)                                                                \
    extern "C" __global__ __launch_bounds__(HELIX_WG * 2) void helix_scan_walk_x6_n##NP(         \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk_x6_impl<NP>(p, b);                                                            \
    }

// The single pass without scratch (HelixScanParams::ytile).
#define HELIX_PASS_C_WALK_X6_Y(NP)                                                              \
    extern "C" __global__ __launch_bounds__(HELIX_WG * 2) void helix_scan_walk_x6_y_n##NP(       \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk_x6_impl<NP, true>(p, b);                                                      \
    }

// The walks of the second and later blocks of state indices.
#define HELIX_PASS_C_WALK_X6_ACC(NP)                                                            \
    extern "C" __global__ __launch_bounds__(HELIX_WG * 2) void helix_scan_walk_x6_acc_n##NP(     \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        scan_walk_x6_impl<NP, false, true>(p, b);                                               \
    }

HELIX_PASS_C_WALK_X6(64)
HELIX_PASS_C_WALK_X6(128)
HELIX_PASS_C_WALK_X6_ACC(64)
HELIX_PASS_C_WALK_X6_ACC(128)
HELIX_PASS_C_WALK_X6_Y(64)
HELIX_PASS_C_WALK_X6_Y(128)
