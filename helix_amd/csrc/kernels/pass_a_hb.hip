// pass_a_hb.hip -- Pass A over head blocks: B is split once per workgroup and
// shared by HELIX_HB (head, P slab) items of one B/C group.
//
// Same computation and outputs as pass_a_x6.hip (reference helix_chunk_state_f32,
// src/kernels/helix_scan_multipass.metal:51-149, walked over a segment):
//     R <- exp(L_end_c) R + B_c^T . (decay . dt . x)_c
// with the GEMM on v_mfma_f32_32x32x16_bf16 over operands split into NS bf16
// planes (NS = 3: six products, fp32 accuracy; NS = 2: three products, the
// opt-in narrower state), issued smallest term first. The operand values, the
// K order and the product order are those of pass_a_x6.hip, so the two kernels
// produce the same segment aggregates. H16 (the bf16 path's default): two
// fp16 planes of operands scaled by powers of two, three products on
// v_mfma_f32_32x32x16_f16 (see hb_next_scale).
//
// What differs is how the work is laid out:
//   - One workgroup of 2 * HELIX_HB waves owns HELIX_HB items that share a B/C
//     group: the B operand of a chunk (64 tokens x d_state) is split into its
//     bf16 planes once, in LDS, for all of them. Items are (head, P slab)
//     pairs, so a group's heads and a head's slabs are tiled alike.
//   - Each wave owns one item's 32-channel P tile and every state index: it
//     loads its x values from global memory straight into the MFMA operand
//     layout (lane lo = channel, tokens 16 s + 8 hi + e), scales and splits
//     them in registers. x never touches LDS and no value is split twice.
//   - The B planes are double-buffered: the next chunk's are written while
//     this chunk's are read, so a chunk costs one barrier.
//   - The decay preamble of each item runs in one of its two waves, a chunk
//     ahead, the two taking turns, and reaches the other through LDS
//     (double-buffered, so the one barrier per chunk covers it).
//   - Every load of the chunk loop runs on every path, and every store but
//     the preamble's record (masked stores go through a zero-range resource
//     or an out-of-range offset): on gfx950 the vmcnt counter counts stores
//     too, and a memory instruction on one path only makes the compiler's
//     waits at the merge conservative.
//   - The bf16 copies of B and C for the walking Pass C are written by one
//     wave per block of its rows per group: wave w of item block ib copies
//     its block when ib == w % (item blocks per group).
// Grid: one workgroup per (seq, B/C group, item block, segment), 1-D and
// decoded XCD-aware so a segment's item blocks (which read the same B rows)
// run on one XCD.
#include "helix_common.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// fp16 planes (H16). The operands are scaled by powers of two into fp16's
// range, then split into a high and a low fp16 plane: v = v0 + v1 + e with
// |e| <= 2^-22 |v| wherever v1 is a normal number (|v| >= 2^-3 after scaling).
// Three products a0 b1 + a1 b0 + a0 b0 leave out a1 b1 and the e terms: about
// 3 * 2^-22 of |ab|, against fp32's 2^-24 per rounding.
//
// Scales. B's are per state index (a row of the aggregate), x's per channel
// (a column), so a scale factors out of every product of the row or column.
// Every scale starts at 2^127. A chunk whose max m (for x, a bound on it)
// reaches 2^15 once scaled (fp16's largest finite value is 65504) replaces
// it with 2^k, k = 12 - floor(log2 m), which puts m in [2^12, 2^13), and the
// accumulated row or column is first multiplied by the exact power of two
// between the two scales; while the row is still zero that is the first
// nonzero chunk, which so sets the scale. A row's values then keep full
// precision down to 2^-15 of the max that set its scale. Smaller later values
// keep the scale: a term that then loses bits lies 2^-26 or more below the
// largest term of its row and column so far, where fp32 accumulation loses it
// as well. The aggregate is divided by both scales when stored.
constexpr int HB_KINIT = 127;

// The scale exponent after a chunk whose max is m (the bits of a value >= 0,
// or of NaN, which takes the smallest scale); `changed`: the scale was
// replaced.
HELIX_DEV int hb_next_scale(int k, unsigned m, bool& changed) {
    const int eb = (int)(m >> 23);   // biased exponent
    changed = eb + k >= 127 + 15;
    return changed ? 127 + 12 - eb : k;
}

// Round-to-nearest-even fp16 pair (element 0 in the low half).
HELIX_DEV unsigned pk_f16(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(unsigned, __builtin_convertvector(v, f16x2));
}

// Two-way fp16 split of the pair (a, b), 4 VALU operations: the residuals
// a - v0 are exact in fp32, each one v_dot2_f32_f16 of the packed pair with
// (-1, 0) or (0, -1), held in a scalar register (bf16_pair_reg).
HELIX_DEV void split2h_pair(float a, float b, unsigned& w0, unsigned& w1) {
    w0 = pk_f16(a, b);
    const f16x2 h = __builtin_bit_cast(f16x2, w0);
    const float ra = __builtin_amdgcn_fdot2(h, __builtin_bit_cast(f16x2, bf16_pair_reg(0x0000bc00u)), a, false);
    const float rb = __builtin_amdgcn_fdot2(h, __builtin_bit_cast(f16x2, bf16_pair_reg(0xbc000000u)), b, false);
    w1 = pk_f16(ra, rb);
}

// The MFMA on operands that hold fp16 bits (the planes share the bf16 planes'
// storage and layout).
HELIX_DEV f32x16 mfma_f16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

// Max of v over lanes l and l ^ 16, and over lanes l and l ^ 32: a swap of
// 16- (32-) lane halves between two copies of v, then a max.
HELIX_DEV unsigned xor16_max(unsigned v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return max((unsigned)r[0], (unsigned)r[1]);
}
HELIX_DEV unsigned xor32_max(unsigned v) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max((unsigned)r[0], (unsigned)r[1]);
}

// Max of v (the bits of a value >= 0) over the wave.
HELIX_DEV unsigned wave_max_bits(unsigned v) {
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x121, 0xf, 0xf, false));   // row_ror:1
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x122, 0xf, 0xf, false));   // row_ror:2
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xf, 0xf, false));   // row_ror:4
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false));   // row_ror:8
    return xor32_max(xor16_max(v));
}

// Max of v (the bits of a value >= 0) over the lanes that hold the same state
// indices in the row-owner layout (hb_rows_at, OWN): lanes equal mod 4 (NP
// 128) or mod 2 (NP 64). Every lane ends with the max.
template <int NP>
HELIX_DEV unsigned hb_row_max(unsigned v) {
    if constexpr (NP == 64) v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x122, 0xf, 0xf, false));
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xf, 0xf, false));   // row_ror:4
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false));   // row_ror:8
    return xor32_max(xor16_max(v));
}

// x of the wave's P tile for one chunk, in storage form: channel 32 pt + lo,
// tokens 16 s + 8 hi + e.
template <typename IO>
struct HbX {
    typename IoWord<IO>::type v[4][8];
};

// This thread's share of a chunk's B rows, and of its C rows for the copies:
// state indices n .. n + 3 (a quad) of the L consecutive tokens t .. t + L - 1,
// one 16-byte run (8 bytes in 16-bit storage) per token, (n, t) = hb_rows_at.
// Few, wide loads: a chunk step stays under the vmcnt counter's 63
// outstanding operations.
template <int NP, typename IO>
struct HbRows {
    static constexpr int L = NP / 32;                       // tokens per lane (4 at NP 128, 2 at 64)
    static constexpr int W = sizeof(IO) == 4 ? 4 : 2;       // 32-bit words per run
    unsigned b[L][W];
    unsigned c[L][4];
};

// The first state index and token of this thread's rows. NP 128: wave w owns
// tokens 16 (w % 4) .. + 15 and state indices 64 (w / 4) .. + 63; lane bits
// (1:0) and (5:4) pick the quad, bits (3:2) the run of four tokens. A load
// instruction then reads four rows of 256 contiguous bytes, and the staging
// writes of 16 consecutive lanes (four tokens of one state index each, at
// dword 36 n + t / 2 of the plane) cover the 16 bank pairs 16 (q % 4) + 2 r:
// no bank conflicts. NP 64: wave w owns tokens 8 w .. 8 w + 7, lane (q, r) =
// (lane % 16, lane / 16) quad q of tokens 8 w + 2 r.
//
// OWN (the fp16 planes): wave w owns every token of state indices 16 w .. + 15
// (NP 128) or 8 w .. + 7 (NP 64), so a state index's max over the chunk is a
// reduction within the wave: lane bits (1:0) (bit 0 at NP 64) pick the quad,
// the others the run of four (two) tokens. A load instruction reads 16 (32)
// rows of 64 (32) contiguous bytes; the staging writes of 16 consecutive lanes
// again cover distinct bank pairs.
template <int NP, bool OWN = false>
HELIX_DEV void hb_rows_at(int lane, int wave, int& n, int& t) {
    if constexpr (OWN) {
        if constexpr (NP == 128) {
            n = 16 * wave + 4 * (lane & 3);
            t = 4 * (lane >> 2);
        } else {
            n = 8 * wave + 4 * (lane & 1);
            t = 2 * (lane >> 1);
        }
    } else if constexpr (NP == 128) {
        const int q = (lane & 3) | ((lane >> 4) << 2);
        n = 64 * (wave >> 2) + 4 * q;
        t = 16 * (wave & 3) + 4 * ((lane >> 2) & 3);
    } else {
        n = 4 * (lane & 15);
        t = 8 * wave + 2 * (lane >> 4);
    }
}

template <typename IO>
HELIX_DEV typename IoWord<IO>::type io_load_at(helix_rsrc r, int voff_bytes, int soff_bytes) {
    if constexpr (sizeof(IO) == 4)
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff_bytes, soff_bytes, 0));
    else
        return (unsigned)__builtin_bit_cast(unsigned short,
                                            __builtin_amdgcn_raw_buffer_load_b16(r, voff_bytes, soff_bytes, 0));
}

// K step s (tokens 16 s + 8 hi + e) of chunk c's x. Branch-free: the row goes
// in the scalar offset and the lane's half (8 hi rows) in its own offset. In a
// ragged last chunk, rows past tlen fall outside the resource's range and read
// 0 when tokens are the outer dimension of x's layout; in any layout their
// weight is exactly 0 and the weighting is a legacy multiply (mul_legacy), so
// whatever such a row reads contributes nothing.
template <typename IO>
__device__ __forceinline__ void hb_load_xs(typename IoWord<IO>::type (&v)[8], const HelixScanParams& p,
                                           const IO* __restrict__ x_w, int c, int s, int lane, int pt, int pw) {
    constexpr int ES = (int)sizeof(IO);
    const int t0 = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const int sx2 = (int)p.s_x[2];
    const int sx0 = sgpr_fresh((int)p.s_x[0]);
    const helix_rsrc rx = make_rsrc(x_w + (long long)t0 * p.s_x[0],
                                    ((tlen - 1) * sx0 + (pw - 1) * sx2 + 1) * (unsigned)ES);
    const int lo = lane & 31, hi = lane >> 5;
    const int xc = min(32 * pt + lo, pw - 1) * sx2;
    const int vx = (xc + 8 * hi * sx0) * ES;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = io_load_at<IO>(rx, vx, (16 * s + e) * sgpr_fresh(sx0) * ES);
}

// dt of token lane of chunk c.
HELIX_DEV float hb_load_dt(const HelixScanParams& p, const float* __restrict__ dt_h, int c, int lane) {
    const int t0 = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const int sdt = (int)p.s_dt[0];
    const helix_rsrc rdt = make_rsrc(dt_h + (long long)t0 * p.s_dt[0], ((tlen - 1) * sdt + 1) * 4u);
    return buf_f32(rdt, min(lane, tlen - 1) * sdt * 4, 0);
}

// Scheduling fence for the vector memory instructions only: loads and stores
// stay where the program puts them (so a refill never moves above the last use
// of the registers it overwrites, and the in-order vmcnt waits keep their
// distance), while ALU, MFMA and LDS work may still be interleaved across it.
HELIX_DEV void vmem_fence() { __builtin_amdgcn_sched_barrier(0x0001 | 0x0002 | 0x0004 | 0x0008 | 0x0080 | 0x0400); }

// B rows (and C rows, for a copying wave) of chunk c. Rows clamp to the last
// valid token and state indices to d_state, so every load is in bounds; a wave
// that does not copy issues its C loads past the resource's range, which
// returns zeros without touching memory (the loads stay on every path, so the
// vmcnt waits are the same for every wave).
template <int NP, typename IO, bool BCC, bool OWN = false>
__device__ __forceinline__ void hb_load_rows(HbRows<NP, IO>& st, const HelixScanParams& p,
                                             const IO* __restrict__ B_g, const float* __restrict__ C_g, int c,
                                             int lane, int wave, int N, bool copier) {
    constexpr int ES = (int)sizeof(IO);
    constexpr int L = HbRows<NP, IO>::L;
    const int t0 = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const int sb0 = sgpr_fresh((int)p.s_b[0]);
    const helix_rsrc rb = make_rsrc(B_g + (long long)t0 * p.s_b[0], ((tlen - 1) * sb0 + N) * (unsigned)ES);
    int nq, j0;
    hb_rows_at<NP, OWN>(lane, wave, nq, j0);
    const int n0 = min(nq, N - 4);
#pragma unroll
    for (int i = 0; i < L; ++i) {
        const int jr = min(j0 + i, tlen - 1);
        const int off = (jr * sb0 + n0) * ES;
        if constexpr (ES == 4) {
            const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0);
#pragma unroll
            for (int k = 0; k < 4; ++k) st.b[i][k] = w[k];
        } else {
            const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rb, off, 0, 0);
            st.b[i][0] = w[0];
            st.b[i][1] = w[1];
        }
    }
    if constexpr (BCC) {
        const int sc0 = sgpr_fresh((int)p.s_c[0]);
        const helix_rsrc rc = make_rsrc(C_g + (long long)t0 * p.s_c[0], ((tlen - 1) * sc0 + N) * 4u);
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int jr = min(j0 + i, tlen - 1);
            const int off = (int)((unsigned)((jr * sc0 + n0) * 4) | (copier ? 0u : 0x80000000u));
            const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rc, off, 0, 0);
#pragma unroll
            for (int k = 0; k < 4; ++k) st.c[i][k] = w[k];
        }
    }
}

// State index k (< 4) of token i of this thread's B rows, as fp32.
template <int NP, typename IO>
HELIX_DEV float hb_b(const HbRows<NP, IO>& st, int i, int k) {
    if constexpr (sizeof(IO) == 4) {
        return as_f32(st.b[i][k]);
    } else {
        const unsigned w = st.b[i][k >> 1];
        return io_f32<IO>((unsigned short)((k & 1) ? (w >> 16) : (w & 0xffffu)));
    }
}

// B planes in LDS: [plane][row n][64 tokens], rows padded to HB_RS elements
// (36 dwords). An MFMA operand read takes 16 consecutive rows of one 16-byte
// chunk per 16 lanes; at a row stride of 4 mod 16 dwords those rows start on
// 16 distinct 4-bank groups, so the read is conflict-free. With padding rather
// than a swizzle, every read and write is one per-lane base plus an immediate
// offset, so the addresses cost a few registers instead of one per operand.
constexpr int HB_RS = HELIX_CS + 8;
template <int NP>
HELIX_DEV int hb_off(int k, int r, int c) {
    return (k * NP + r) * HB_RS + c * 8;
}

// Split the L consecutive tokens' values v[0..L-1] of state index n into NS
// planes and store them at tokens t .. t + L - 1 of row n (hb_off layout).
// H16: two fp16 planes, or one where the scaled values are exact in fp16.
template <int NP, int NS, int L, bool H16 = false>
HELIX_DEV void hb_stage_run(__bf16* planes, int n, int t, const float* v) {
    static_assert(L == 2 || L == 4, "runs of two or four tokens");
    unsigned q[NS][L / 2];
#pragma unroll
    for (int e = 0; e < L / 2; ++e) {
        unsigned w[3];
        if constexpr (H16 && NS == 1)
            w[0] = pk_f16(v[2 * e], v[2 * e + 1]);
        else if constexpr (H16)
            split2h_pair(v[2 * e], v[2 * e + 1], w[0], w[1]);
        else if constexpr (NS == 3)
            split3_pair(v[2 * e], v[2 * e + 1], w[0], w[1], w[2]);
        else
            split2_pair(v[2 * e], v[2 * e + 1], w[0], w[1]);
#pragma unroll
        for (int k = 0; k < NS; ++k) q[k][e] = w[k];
    }
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        __bf16* dst = &planes[(k * NP + n) * HB_RS + t];
        if constexpr (L == 4)
            *reinterpret_cast<u32x2*>(dst) = u32x2{q[k][0], q[k][1]};
        else
            *reinterpret_cast<unsigned*>(dst) = q[k][0];
    }
}

// The decay preamble of chunk c (lane = token): the weight w_lane = exp(L_end -
// Lcum_lane) dt_lane (0 past tlen) of the chunk's GEMM, L_end, and the token's
// decay record for Pass C (the forms of store_decay_record / store_decay_record64).
struct HbPre {
    float w;
    double lend;
    u32x4 rec;
};

// `shift` (<= 0) is the log-decay from the chunk's end to where the weighted
// sum is taken (0: the chunk's end), folded into the weight. R64: the record
// in the fp32 path's form (store_decay_record64), whatever the MODE.
template <int MODE, bool R64 = false>
__device__ __forceinline__ HbPre hb_preamble(const HelixScanParams& p, float dtraw, float A_h, int c, int lane,
                                             double shift) {
    const int t0 = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const float dtv = keep_if_lt(helix_dt(p, dtraw), lane, tlen);
    const double lcum = wave_incl_sum((double)A_h * (double)dtv);
    const double lend = bcast(lcum, 63);
    HbPre r;
    r.w = keep_if_lt(exp_diff(lend + shift, lcum) * dtv, lane, tlen);
    r.lend = lend;
    if constexpr (MODE == 2 && !R64) {
        const u32x2 w = walk_record(dtv, lcum);
        r.rec = u32x4{w[0], w[1], 0u, 0u};
    } else {
        const float e = expf((float)lcum);
        const unsigned long long u = __builtin_bit_cast(unsigned long long, lcum);
        r.rec = u32x4{as_u32(dtv), as_u32(e), (unsigned)u, (unsigned)(u >> 32)};
    }
    return r;
}

// MODE 0: store the in-segment prefix R_c (fp32) before each chunk, and the
// fp64 decay records of the fp32 path's Pass C; MODE 2: segment aggregates only,
// and the walk's decay records. IO: the caller's storage type of x and B. BCC:
// write the bf16 copies of B and C (fp32 storage). NS: split planes per operand.
// R64: MODE 2 with the fp32 path's records, for its bf16x6 walk. H16: two
// fp16 planes with power-of-two scales (see hb_next_scale), aggregates only.
template <int NP, int MODE, typename IO = float, bool BCC = false, int NS = 3, bool R64 = false, bool H16 = false>
__device__ __forceinline__ void chunk_state_hb_impl(const HelixScanParams& p, const HelixScanBuffers& b) {
    static_assert(NP == 64 || NP == 128, "the double-buffered B planes of d_state 256 exceed the LDS");
    static_assert(NS == 2 || NS == 3, "two or three split planes");
    static_assert(MODE == 0 || MODE == 2, "per-chunk fp32 prefixes or aggregates only");
    static_assert(!H16 || (NS == 2 && MODE == 2 && !R64), "fp16 planes: aggregates");
    constexpr int HB = HELIX_HB;
    constexpr int NTN = NP / 32;        // 32-row n tiles per wave
    // B's planes. With fp16 planes and 16-bit storage one: a bf16 or f16 value
    // (8 or 11 significant bits) scaled by a power of two is exact in fp16
    // wherever it stays a normal number, so B's low plane would be zero and
    // the products are a1 b0 + a0 b0.
    constexpr int NSB = (H16 && sizeof(IO) == 2) ? 1 : NS;
    constexpr int PLANES = NSB * NP * HB_RS;
    __shared__ __attribute__((aligned(16))) __bf16 sB[2 * PLANES];   // two chunks' planes
    // Per chunk parity and item: w_j of the chunk's 64 tokens, and L_end (fp64
    // bits) at [64], [65].
    __shared__ __attribute__((aligned(16))) float sW[2][HB][HELIX_CS + 4];
    // H16: the scale exponent of every state index for the planes of chunk
    // step it (buffer it % 3: a wave may read the previous step's while
    // another already writes the next one's), and per step parity and wave
    // whether a scale in use changed.
    __shared__ __attribute__((aligned(16))) int sKb[H16 ? 3 : 1][H16 ? NP : 4];
    __shared__ __attribute__((aligned(8))) unsigned char sFlag[H16 ? 2 : 1][8];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = wave_uniform(), lo = lane & 31, hi = lane >> 5;
    // Wave w owns P tile w / HB of item w % HB: each SIMD (waves s and s + 4)
    // holds one wave of each P tile, so the preamble waves (P tile 0) are
    // spread over the SIMDs.
    const int is = wave % HB, pt = wave / HB;

    const int ipg = p.heads_per_group * p.n_pslab;        // items per group
    const int nib = (ipg + HB - 1) / HB;                  // item blocks per group
    const unsigned total = (unsigned)p.n_seq * (unsigned)p.n_group * (unsigned)nib * (unsigned)p.n_seg;
    unsigned wid = xcd_logical_id(blockIdx.x, total);
    // Logical order: item block, group, segment, sequence. An XCD's share of
    // the logical ids is then a run of consecutive segments over every group:
    // its x reads are whole token rows of one stretch of the sequence, and a
    // segment's item blocks (which read the same B rows) stay on one XCD.
    // Groups as the slower index instead (an XCD per group: 2 KiB of every
    // 16 KiB token row at config 2) measured 4 us slower.
    const int ib = (int)(wid % (unsigned)nib);        wid /= (unsigned)nib;
    const int g = (int)(wid % (unsigned)p.n_group);   wid /= (unsigned)p.n_group;
    const int seg = (int)(wid % (unsigned)p.n_seg);   wid /= (unsigned)p.n_seg;
    const int seq = (int)wid;

    // Item of this wave; a block's spare waves repeat its last item and store nothing.
    const int ii_raw = ib * HB + is;
    const bool item_ok = ii_raw < ipg;
    const int ii = min(ii_raw, ipg - 1);
    const int h = g * p.heads_per_group + ii / p.n_pslab;
    const int slab = ii % p.n_pslab;
    const int p0 = slab * HELIX_HD;
    const int pw = min(HELIX_HD, p.head_dim - p0);
    const int N = p.d_state;

    const int c_begin = seg * p.seg_len;
    const int c_end = min(c_begin + p.seg_len, p.n_cg);
    if (c_begin >= c_end) return;

    const float A_h = b.A[(long long)h * p.s_a];
    const float* __restrict__ dt_h = b.dt + seq * p.seq_dt + h * p.s_dt[1];
    const IO* __restrict__ x_w = reinterpret_cast<const IO*>(b.x) + seq * p.seq_x + h * p.s_x[1] + p0 * p.s_x[2];
    const IO* __restrict__ B_g = reinterpret_cast<const IO*>(b.B) + seq * p.seq_b + g * p.s_b[1];
    const float* __restrict__ C_g = b.C + seq * p.seq_c + g * p.s_c[1];
    const bool copier = BCC && (wave % nib) == ib;
    const bool head_leader = item_ok && slab == 0;           // the head's records come from its first slab
    const bool leader = head_leader && pt == 0;              // stores the head's log-decay
    const long long tile_off = state_tile_off(p, h, slab);
    const unsigned tile_bytes = item_ok ? 64u * NP * 4u : 0u;   // spare waves store nothing

    f32x16 acc[NTN];
#pragma unroll
    for (int i = 0; i < NTN; ++i) acc[i] = zero16();

    // Chunk order. MODE 0 walks the segment forward: R_c is the prefix of the
    // chunks before c, and the accumulators take each chunk's decay. MODE 2
    // walks it backward: the log-decay from a chunk's end to the segment's end
    // (mu, the sum over the chunks already done) is known when the chunk's
    // weights are formed and is folded into them, so the accumulators are
    // never rescaled and end as the segment aggregate.
    const int n_ch = c_end - c_begin;
    auto nth = [&](int it) { return MODE == 0 ? min(c_begin + it, c_end - 1) : max(c_end - 1 - it, c_begin); };
    float lam = 0.0f;    // MODE 0: log-decay of the segment before the current chunk
    double mu = 0.0;     // MODE 2: log-decay from the current chunk's end to the segment's end
    double lend = 0.0;   // L_end of the current chunk, read from its weight buffer

    // B planes of chunk c into `planes` (state indices q4 + k, k0 <= k < k1, of
    // this thread's rows), and the bf16 copies of its B and C rows.
    constexpr int L = HbRows<NP, IO>::L;
    int q4, tr;   // this thread's first state index and token
    hb_rows_at<NP, H16>(lane, wave, q4, tr);
    // H16: scale exponents of state indices q4 .. q4 + 3 (the same in every
    // lane of the quad) and of this lane's channel.
    int kb[4] = {HB_KINIT, HB_KINIT, HB_KINIT, HB_KINIT};
    int kx = HB_KINIT;
    auto stage_planes = [&](const HbRows<NP, IO>& rows, __bf16* planes, int k0, int k1) {
#pragma unroll
        for (int k = k0; k < k1; ++k) {
            float v[L];
#pragma unroll
            for (int i = 0; i < L; ++i) {
                v[i] = hb_b<NP, IO>(rows, i, k);
                if constexpr (H16) v[i] = __builtin_ldexpf(v[i], kb[k]);
            }
            hb_stage_run<NP, NSB, L, H16>(planes, q4 + k, tr, v);
        }
    };
    // H16: the scales of the state indices of the chunk in `rows`, whose
    // planes chunk step `st` reads, into sKb[st % 3], and whether a scale in
    // use changed into sFlag[st & 1]. Each lane first checks its own tokens of
    // its four rows against the scales in use; only where one of them would
    // overflow does the wave reduce the rows' maxima and choose scales again.
    auto update_b_scales = [&](const HbRows<NP, IO>& rows, int st) {
        if constexpr (H16) {
            float m[4];
            bool need = false;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                m[k] = 0.0f;
#pragma unroll
                for (int i = 0; i < L; ++i) m[k] = fmaxf(m[k], fabsf(hb_b<NP, IO>(rows, i, k)));
                need |= (int)(__builtin_bit_cast(unsigned, m[k]) >> 23) + kb[k] >= 127 + 15;
            }
            bool any = false;
            if (__builtin_amdgcn_ballot_w64(need) != 0) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    bool ch;
                    kb[k] = hb_next_scale(kb[k], hb_row_max<NP>(__builtin_bit_cast(unsigned, m[k])), ch);
                    any |= ch;
                }
            }
            if (tr == 0) *reinterpret_cast<int4*>(&sKb[st % 3][q4]) = int4{kb[0], kb[1], kb[2], kb[3]};
            const bool wany = __builtin_amdgcn_ballot_w64(any) != 0;
            if (lane == 0) sFlag[st & 1][wave] = wany ? 1 : 0;
        }
    };
    auto copy_rows = [&](const HbRows<NP, IO>& rows, int c) {
        if constexpr (BCC) {
            const int t0 = (p.chunk_base + c) * HELIX_CS;
            const int tlen = min(HELIX_CS, p.n_tok - t0);
            const long long gn = (long long)p.n_group * N;
            const long long base = ((long long)seq * p.cpg * HELIX_CS + (long long)c * HELIX_CS) * gn + (long long)g * N;
            const unsigned bytes = copier ? (unsigned)((HELIX_CS - 1) * gn + N) * 2u : 0u;
            const helix_rsrc rb = make_rsrc_u(static_cast<__bf16*>(b.bcopy) + base, bytes);
            const helix_rsrc rc = make_rsrc_u(static_cast<__bf16*>(b.ccopy) + base, bytes);
            const int gni = (int)gn;
#pragma unroll
            for (int i = 0; i < L; ++i) {
                const int j = tr + i;
                const int off = store_off_if_lt((j * gni + q4) * 2, j, tlen, q4, N);
                const u32x2 wb = {pk_bf16(as_f32(rows.b[i][0]), as_f32(rows.b[i][1])),
                                  pk_bf16(as_f32(rows.b[i][2]), as_f32(rows.b[i][3]))};
                const u32x2 wc = {pk_bf16(as_f32(rows.c[i][0]), as_f32(rows.c[i][1])),
                                  pk_bf16(as_f32(rows.c[i][2]), as_f32(rows.c[i][3]))};
                __builtin_amdgcn_raw_buffer_store_b64(wb, rb, off, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b64(wc, rc, off, 0, 0);
            }
        }
    };

    HbX<IO> xs;
    HbRows<NP, IO> rows;
    float dtraw;   // dt of token lane of the chunk the next preamble forms

    // The preamble of chunk c (weights shifted by `shift`) into the chunk's
    // weight buffer, with its L_end (fp64 bits) at [64] and [65]. Then the
    // chunk's record and (MODE 0) ld[c] = lam_c, cancelled by a zero range
    // past the head's first P slab, and when the call only repeats the
    // segment's last chunk (`live` false: they are already stored). One wave
    // of an item forms it, the item's two waves taking turns chunk by chunk
    // (both sit on one SIMD, so forming it in both doubled its ALU work on
    // that SIMD: 2.4 us of a config-2 scan); the other reads the weights and
    // L_end from LDS after the chunk's barrier.
    auto preamble = [&](int c, double shift, float lam_c, float (*wdst)[HELIX_CS + 4], bool live) {
        const HbPre pr = hb_preamble<MODE, R64>(p, dtraw, A_h, c, lane, shift);
        wdst[is][lane] = pr.w;
        // H16: the chunk's largest weight (>= 0) at [66], for the x scales.
        const float wmax = H16 ? __builtin_bit_cast(float, wave_max_bits(__builtin_bit_cast(unsigned, pr.w))) : 0.0f;
        if (lane == 0) {
            const unsigned long long u = __builtin_bit_cast(unsigned long long, pr.lend);
            wdst[is][HELIX_CS] = __builtin_bit_cast(float, (unsigned)u);
            wdst[is][HELIX_CS + 1] = __builtin_bit_cast(float, (unsigned)(u >> 32));
            if constexpr (H16) wdst[is][HELIX_CS + 2] = wmax;
        }
        // The record's address is formed unconditionally (a select of two
        // pointers becomes a branch); without records its range is zero.
        const bool rec = live && head_leader && b.pre != nullptr;
        constexpr int RB = (MODE == 2 && !R64) ? HELIX_REC_WALK_BYTES : HELIX_REC64_BYTES;
        const unsigned long long recp =
            (unsigned long long)b.pre + (unsigned long long)((((long long)seq * p.cpg + c) * p.n_head + h) * (HELIX_CS * RB));
        const helix_rsrc rr = make_rsrc_u((const void*)recp, rec ? HELIX_CS * RB : 0u);
        if constexpr (RB == 8)
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{pr.rec[0], pr.rec[1]}, rr, lane * 8, 0, 0);
        else
            __builtin_amdgcn_raw_buffer_store_b128(pr.rec, rr, lane * 16, 0, 0);
        if constexpr (MODE == 0) {
            const float* ldp = b.ld + seq * p.ld_seq + (long long)c * p.n_head + h;
            __builtin_amdgcn_raw_buffer_store_b32(as_u32(lam_c), make_rsrc_u(ldp, live && head_leader ? 4u : 0u),
                                                  lane == 0 ? 0 : (int)0x80000000, 0, 0);
        }
    };

    // R[n][p] += sum_j B^T[n][j] (w_j x[j][p]) over four K steps of 16 tokens,
    // in groups of two n tiles.
    constexpr int NG = NTN / 2;                 // groups of two n tiles per K step
    auto read_group = [&](const __bf16* planes, int s, int i0, bf16x8 (&bp)[2][NSB]) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int k = 0; k < NSB; ++k)
                bp[i][k] = *reinterpret_cast<const bf16x8*>(&planes[hb_off<NP>(k, 32 * (i0 + i) + lo, 2 * s + hi)]);
    };
    auto read_w = [&](const float* __restrict__ wrow, int s, f32x4& w0, f32x4& w1) {
        w0 = *reinterpret_cast<const f32x4*>(&wrow[16 * s + 8 * hi]);
        w1 = *reinterpret_cast<const f32x4*>(&wrow[16 * s + 8 * hi + 4]);
    };
    // Smallest terms first, the two accumulators interleaved so no MFMA
    // waits on the one before it.
    auto mfma_group = [&](int i0, const bf16x8 (&bp)[2][NSB], const bf16x8 (&xp)[NS]) {
        if constexpr (H16 && NSB == 1) {
#pragma unroll
            for (int i = 0; i < 2; ++i) acc[i0 + i] = mfma_f16(bp[i][0], xp[1], acc[i0 + i]);
#pragma unroll
            for (int i = 0; i < 2; ++i) acc[i0 + i] = mfma_f16(bp[i][0], xp[0], acc[i0 + i]);
            return;
        } else if constexpr (H16) {
#pragma unroll
            for (int i = 0; i < 2; ++i) acc[i0 + i] = mfma_f16(bp[i][1], xp[0], acc[i0 + i]);
#pragma unroll
            for (int i = 0; i < 2; ++i) acc[i0 + i] = mfma_f16(bp[i][0], xp[1], acc[i0 + i]);
#pragma unroll
            for (int i = 0; i < 2; ++i) acc[i0 + i] = mfma_f16(bp[i][0], xp[0], acc[i0 + i]);
            return;
        }
        if constexpr (NS == 3) {
#pragma unroll
            for (int i = 0; i < 2; ++i) acc[i0 + i] = mfma_bf16(bp[i][2], xp[0], acc[i0 + i]);
#pragma unroll
            for (int i = 0; i < 2; ++i) acc[i0 + i] = mfma_bf16(bp[i][1], xp[1], acc[i0 + i]);
#pragma unroll
            for (int i = 0; i < 2; ++i) acc[i0 + i] = mfma_bf16(bp[i][0], xp[2], acc[i0 + i]);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[i0 + i] = mfma_bf16(bp[i][1], xp[0], acc[i0 + i]);
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[i0 + i] = mfma_bf16(bp[i][0], xp[1], acc[i0 + i]);
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[i0 + i] = mfma_bf16(bp[i][0], xp[0], acc[i0 + i]);
    };
    // The x operand planes of K step s of the chunk in xs, weighted by w0, w1.
    auto split_x = [&](int s, const f32x4& w0, const f32x4& w1, bf16x8 (&xp)[NS]) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = mul_legacy(w0[e], io_widen<IO>(xs.v[s][e]));
            v[4 + e] = mul_legacy(w1[e], io_widen<IO>(xs.v[s][4 + e]));
        }
        if constexpr (H16) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = __builtin_ldexpf(v[e], kx);
        }
        u32x4 xq[NS];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            unsigned w[3];
            if constexpr (H16)
                split2h_pair(v[2 * e], v[2 * e + 1], w[0], w[1]);
            else if constexpr (NS == 3)
                split3_pair(v[2 * e], v[2 * e + 1], w[0], w[1], w[2]);
            else
                split2_pair(v[2 * e], v[2 * e + 1], w[0], w[1]);
#pragma unroll
            for (int k = 0; k < NS; ++k) xq[k][e] = w[k];
        }
#pragma unroll
        for (int k = 0; k < NS; ++k) xp[k] = __builtin_bit_cast(bf16x8, xq[k]);
    };

    // H16, before a chunk's products: the accumulated rows whose state index
    // took a new scale for this chunk (planes of step it, scales in buffer
    // it % 3, the previous step's in (it + 2) % 3) are multiplied by the exact
    // power of two between the two scales; then the columns, for the bound
    // max |x| * max w of the chunk's weighted x in each channel (over its two
    // lanes; the largest weight from the preamble, wrow[66]), which puts the
    // largest |w x| at or below 2^13 once scaled.
    auto chunk_scales = [&](int it, const float* __restrict__ wrow) {
        if constexpr (H16) {
            if (it > 0 && *reinterpret_cast<const unsigned long long*>(&sFlag[it & 1][0]) != 0ull) {
                const int kn = it % 3, ko = (it + 2) % 3;
#pragma unroll
                for (int i = 0; i < NTN; ++i)
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const int row = 32 * i + acc_row(j, hi);
                        acc[i][j] = __builtin_ldexpf(acc[i][j], sKb[kn][row] - sKb[ko][row]);
                    }
            }
            float mx = 0.0f;
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(io_widen<IO>(xs.v[s][e])));
            const float bound = __builtin_bit_cast(float, xor32_max(__builtin_bit_cast(unsigned, mx))) * wrow[HELIX_CS + 2];
            bool ch;
            const int kn = hb_next_scale(kx, __builtin_bit_cast(unsigned, bound), ch);
            if (__builtin_amdgcn_ballot_w64(ch) != 0) {
                const int d = ch ? kn - kx : 0;
#pragma unroll
                for (int i = 0; i < NTN; ++i)
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[i][j] = __builtin_ldexpf(acc[i][j], d);
            }
            kx = kn;
        }
    };

    // Chunk nth(it). Its B planes are in `cur` and its weights in `wcur` (both
    // staged a step earlier), its x in xs; `rows` holds the B (and C) rows and
    // dtraw the dt of the chunk after it, cn. Every memory instruction runs on
    // every path; past the segment's last chunk the loads and the staging
    // repeat that chunk (nothing reads the result). The loop is not unrolled:
    // the loop-carried registers then keep one assignment, with no copies at
    // the back edge.
    auto step = [&](int it, const __bf16* cur, __bf16* nxt, float (*wcur)[HELIX_CS + 4],
                    float (*wnxt)[HELIX_CS + 4]) {
        const int c = nth(it), cn = nth(it + 1);
        const float* __restrict__ wrow = wcur[is];
        // L_end of this chunk, from its preamble a step earlier.
        lend = __builtin_bit_cast(double, (unsigned long long)__builtin_bit_cast(unsigned, wrow[HELIX_CS]) |
                                              ((unsigned long long)__builtin_bit_cast(unsigned, wrow[HELIX_CS + 1]) << 32));
        const float lendf = (float)lend;
        const bool forms = pt == (it & 1);   // this wave forms the next chunk's preamble
        if constexpr (MODE == 0) {
            // R_c, the state entering chunk c from this segment's own chunks
            // (none for its first chunk: a zero range stores nothing).
            const float* dst = static_cast<const float*>(b.s_local) + seq * p.sl_seq + (long long)c * p.sl_cg +
                               tile_off;
            const helix_rsrc rd = make_rsrc_u(dst, c > c_begin ? tile_bytes : 0u);
#pragma unroll
            for (int i = 0; i < NTN; ++i)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    buf_store_unit<float>(rd, acc[i][4 * r4], acc[i][4 * r4 + 1], acc[i][4 * r4 + 2],
                                          acc[i][4 * r4 + 3], lane, tile_unit(NTN, pt, i, r4, 0));
        }
        const float a_c = MODE == 0 ? expf(lendf) : 1.0f;
        chunk_scales(it, wrow);

        // The B planes of the next group and the weights of the next K step
        // are read from LDS while the current group's MFMAs run, so no MFMA
        // waits on the LDS.
        bf16x8 bq[2][2][NSB];       // the B planes of two groups, in turn
        f32x4 w0, w1;
        read_group(cur, 0, 0, bq[0]);
        read_w(wrow, 0, w0, w1);
        // MODE 0: the decay of the state carried in, on each group's
        // accumulators just before their first products of the chunk.
        if constexpr (MODE == 0) {
            acc[0] *= a_c;
            acc[1] *= a_c;
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            bf16x8 xp[NS];
            split_x(s, w0, w1, xp);
            if (s + 1 < 4) read_w(wrow, s + 1, w0, w1);
            // K step s of the next chunk's x into the registers just split:
            // it has a whole chunk step to arrive.
            vmem_fence();
            hb_load_xs<IO>(xs.v[s], p, x_w, cn, s, lane, pt, pw);
            // The next chunk's preamble (K step 1) and B planes and copies
            // (K steps 2 and 3): ALU and LDS work with no dependence on this
            // chunk's products, written among them so it overlaps the MFMAs.
            if (s == 1) {
                if constexpr (MODE == 0) {
                    lam += lendf;
                    if (forms) preamble(cn, 0.0, lam, wnxt, it + 1 < n_ch);
                } else {
                    mu += lend;
                    if (forms) preamble(cn, mu, 0.0f, wnxt, it + 1 < n_ch);
                }
            }
            vmem_fence();
            if (s == 2) update_b_scales(rows, it + 1);
            if (s >= 2) stage_planes(rows, nxt, 2 * (s - 2), 2 * (s - 2) + 2);
            if (s == 3) copy_rows(rows, cn);
            vmem_fence();
#pragma unroll
            for (int gi = 0; gi < NG; ++gi) {
                const int q = (s * NG + gi) & 1;          // buffer of this group
                const int s_n = gi + 1 < NG ? s : s + 1;  // the next group's K step
                const int g_n = gi + 1 < NG ? gi + 1 : 0;
                if (s_n < 4) read_group(cur, s_n, 2 * g_n, bq[q ^ 1]);
                if (MODE == 0 && s == 0 && gi > 0) {
                    acc[2 * gi] *= a_c;
                    acc[2 * gi + 1] *= a_c;
                }
                mfma_group(2 * gi, bq[q], xp);
            }
        }
        // The rows and dt of the chunk after cn.
        vmem_fence();
        const int cnn = nth(it + 2);
        hb_load_rows<NP, IO, BCC, H16>(rows, p, B_g, C_g, cnn, lane, wave, N, copier);
        dtraw = hb_load_dt(p, dt_h, cnn, lane);
        __syncthreads();
    };

    // Prologue: the first chunk's weights and B planes in buffer 0, its x in
    // flight, the second chunk's rows and dt in flight.
    const int c0 = nth(0), c1 = nth(1);
    dtraw = hb_load_dt(p, dt_h, c0, lane);
    hb_load_rows<NP, IO, BCC, H16>(rows, p, B_g, C_g, c0, lane, wave, N, copier);
#pragma unroll
    for (int s = 0; s < 4; ++s) hb_load_xs<IO>(xs.v[s], p, x_w, c0, s, lane, pt, pw);
    if (pt == 1) preamble(c0, 0.0, 0.0f, sW[0], true);
    update_b_scales(rows, 0);
    stage_planes(rows, sB, 0, 4);
    copy_rows(rows, c0);
    hb_load_rows<NP, IO, BCC, H16>(rows, p, B_g, C_g, c1, lane, wave, N, copier);
    dtraw = hb_load_dt(p, dt_h, c1, lane);
    __syncthreads();
    // MODE 2 takes the segment's last chunk out of the loop (last_step).
    const int n_loop = MODE == 2 ? n_ch - 1 : n_ch;
#pragma unroll 1
    for (int it = 0; it < n_loop; ++it) {
        const int par = it & 1;
        step(it, sB + par * PLANES, sB + (PLANES - par * PLANES), sW[par], sW[par ^ 1]);
    }

    // Accumulator tiles i0 .. i1 - 1 of the segment aggregate D_s: in scratch,
    // or in y for the single pass without scratch (p.ytile; ytile_* in
    // helix_common.h, the range covering the rows the tile and the log-decay
    // take).
    // H16: accumulator tiles i0 .. i1 - 1 divided by the scales of their rows
    // and column.
    auto unscale_tiles = [&](int i0, int i1) {
        if constexpr (H16) {
            const int kbuf = n_loop % 3;
#pragma unroll
            for (int i = i0; i < i1; ++i)
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    acc[i][j] = __builtin_ldexpf(acc[i][j], -(kx + sKb[kbuf][32 * i + acc_row(j, hi)]));
        }
    };
    auto store_tiles = [&](int i0, int i1) {
        if (MODE == 2 && p.ytile) {
            const int upr = pw >> 2;
            const unsigned yrows = (unsigned)((16 * NP + 1 + upr - 1) / upr);
            const helix_rsrc ry = make_rsrc_u(b.y + ytile_base(p, seq, h, slab, seg),
                                              item_ok ? yrows * (unsigned)p.s_y[0] * 4u : 0u);
#pragma unroll
            for (int i = i0; i < i1; ++i)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int off = (int)ytile_unit(p, tile_unit(NTN, pt, i, r4, 0) + lane, pw) * 4;
                    const u32x4 w = {as_u32(acc[i][4 * r4]), as_u32(acc[i][4 * r4 + 1]),
                                     as_u32(acc[i][4 * r4 + 2]), as_u32(acc[i][4 * r4 + 3])};
                    __builtin_amdgcn_raw_buffer_store_b128(w, ry, off, 0, 0);
                }
        } else {
            const float* sg = b.s_seg + seq * p.sg_seq + (long long)seg * p.sg_seg + tile_off;
            const helix_rsrc rs = make_rsrc_u(sg, tile_bytes);
#pragma unroll
            for (int i = i0; i < i1; ++i)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    buf_store_unit<float>(rs, acc[i][4 * r4], acc[i][4 * r4 + 1], acc[i][4 * r4 + 2],
                                          acc[i][4 * r4 + 3], lane, tile_unit(NTN, pt, i, r4, 0));
        }
    };

    if constexpr (MODE == 2) {
        // The segment's last chunk (the first in time): the step's products
        // without the next chunk's loads, preamble and staging (nothing would
        // read them), taken group of n tiles by group with each tile's
        // products in the step's order, so the aggregate is the same, and a
        // group's tiles are stored while the next group's MFMAs run. Its B
        // planes and weights are in the buffers of parity n_loop; it writes
        // no LDS, so it needs no barrier.
        const int par = n_loop & 1;
        const __bf16* cur = sB + par * PLANES;
        const float* __restrict__ wrow = sW[par][is];
        lend = __builtin_bit_cast(double, (unsigned long long)__builtin_bit_cast(unsigned, wrow[HELIX_CS]) |
                                              ((unsigned long long)__builtin_bit_cast(unsigned, wrow[HELIX_CS + 1]) << 32));
        mu += lend;
        chunk_scales(n_loop, wrow);
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
            bf16x8 bq[2][2][NSB];
            read_group(cur, 0, 2 * gi, bq[0]);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                f32x4 w0, w1;
                read_w(wrow, s, w0, w1);
                bf16x8 xp[NS];
                split_x(s, w0, w1, xp);
                if (s + 1 < 4) read_group(cur, s + 1, 2 * gi, bq[(s + 1) & 1]);
                mfma_group(2 * gi, bq[s & 1], xp);
            }
            unscale_tiles(2 * gi, 2 * gi + 2);
            store_tiles(2 * gi, 2 * gi + 2);
        }
        if (p.ytile) {
            if (leader && lane == 0) b.y[ytile_segld(p, seq, h, seg)] = (float)mu;
        } else {
            if (leader && lane == 0) b.segld[seq * p.sd_seq + (long long)seg * p.n_head + h] = (float)mu;
        }
        return;
    }
    store_tiles(0, NTN);
    if (leader && lane == 0) b.segld[seq * p.sd_seq + (long long)seg * p.n_head + h] = lam;
}

#define HELIX_PASS_A_HB(NP)                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_x6f32_n##NP(    \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 0>(p, b);                                                             \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_x6agg_n##NP(    \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2>(p, b);                                                             \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_x6agg_bc_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2, float, true>(p, b);                                                \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_x6agg_r64_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2, float, false, 3, true>(p, b);                                      \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_x6agg_bf16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2, __bf16>(p, b);                                                     \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_x6agg_f16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2, _Float16>(p, b);                                                   \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_h3agg_n##NP(    \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2, float, false, 2, false, true>(p, b);                               \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_h3agg_bc_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2, float, true, 2, false, true>(p, b);                                \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_h3agg_bf16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2, __bf16, false, 2, false, true>(p, b);                              \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_h3agg_f16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2, _Float16, false, 2, false, true>(p, b);                            \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_x3agg_n##NP(    \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2, float, false, 2>(p, b);                                            \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_x3agg_bc_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2, float, true, 2>(p, b);                                             \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_x3agg_bf16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2, __bf16, false, 2>(p, b);                                           \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(HELIX_HB_THREADS) void helix_chunk_state_hb_x3agg_f16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                      \
        chunk_state_hb_impl<NP, 2, _Float16, false, 2>(p, b);                                         \
    }

HELIX_PASS_A_HB(64)
HELIX_PASS_A_HB(128)
