// pass_a_x6.hip -- Pass A on bf16 MFMA with three-way operand splitting.
//
// Same computation and outputs as pass_a.hip (reference helix_chunk_state_f32,
// src/kernels/helix_scan_multipass.metal:51-149, walked over a segment):
//     R <- exp(L_end_c) R + B_c^T . (decay . dt . x)_c
// but the GEMM runs on v_mfma_f32_32x32x16_bf16, which MI355X issues at 16x
// the fp32 matrix rate. Each fp32 operand v is split into three bf16 parts
//     v = v0 + v1 + v2,  v0 = bf16(v), v1 = bf16(v - v0), v2 = bf16(v - v0 - v1)
// (split3_pair and mfma_x6 in helix_common.h): fp32 accuracy from six bf16
// products per fp32 product.
// The terms are issued smallest first so the large ones are added last.
//
// Layout: the workgroup computes R[n][p] (N x 64), M = n, N = p, K = token.
// The split operands are staged in LDS k-contiguous: three planes of
// B^T[n][j] and three of dtXs^T[p][j], rows of 64 tokens (eight 16-byte
// chunks, swizzled as x6_off describes). Wave w owns P tile (w & 1) and N
// tiles (w >> 1) + 2i, and stages tokens 16w .. 16w+15 (chunks 2w and 2w+1)
// of every row: dtXs^T row p = lane both chunks; B^T rows NB*lo ..
// NB*lo + NB-1 (NB = NP/32) chunk 2w + hi.
#include "helix_common.h"

// One chunk's global inputs for this thread, 1 + 16 + 8 loads (two stages
// fit the 63 loads the vmcnt counter can track):
//   x   tokens 16 wave + i (i < 16), channel p = lane
//   B   tokens 16 wave + 8 hi + e (e < 8), state indices NB lo .. NB lo + NB-1,
//       one 8/16/32-byte load per token (NB = NP/32 consecutive floats)
// x and B stay in storage form until they are split (x6_b): the words of a
// B run are kept as loaded, fp32 bits or two 16-bit values per word.
template <int NP, typename IO>
struct StageX6 {
    static constexpr int BW = sizeof(IO) == 4 ? NP / 32 : NP / 64;   // words per B run
    float dtraw;
    typename IoWord<IO>::type x[16];
    unsigned b[8][BW];
};

// State index k of token e's B run, widened to fp32.
template <int NP, typename IO>
HELIX_DEV float x6_b(const StageX6<NP, IO>& st, int e, int k) {
    if constexpr (sizeof(IO) == 4) {
        return as_f32(st.b[e][k]);
    } else {
        const unsigned w = st.b[e][k >> 1];
        return io_f32<IO>((unsigned short)((k & 1) ? (w >> 16) : (w & 0xffffu)));
    }
}

// Rows are clamped to the last valid token, channels to the slab and state
// indices to d_state, so every load is in bounds; nothing is masked (see the
// staging comment in the kernel).
// IO: the caller's storage type of x and B. A lane's run of NB state
// indices is one 8/16/32-byte load in fp32 and one 4/8/16-byte load in 16-bit
// storage.
template <int NP, typename IO>
__device__ __forceinline__ void load_stage_x6(StageX6<NP, IO>& st, const HelixScanParams& p,
                                              const float* __restrict__ dt_h,
                                              const IO* __restrict__ x_h,
                                              const IO* __restrict__ B_g, int c, int lane,
                                              int wave, int pw, int N) {
    constexpr int ES = (int)sizeof(IO);
    const int t0   = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const int sdt = (int)p.s_dt[0], sx0 = sgpr_fresh((int)p.s_x[0]), sx2 = (int)p.s_x[2];
    const int sb0 = sgpr_fresh((int)p.s_b[0]);
    const helix_rsrc rdt = make_rsrc(dt_h + (long long)t0 * p.s_dt[0], ((tlen - 1) * sdt + 1) * 4u);
    const helix_rsrc rx  = make_rsrc(x_h + (long long)t0 * p.s_x[0],
                                     ((tlen - 1) * sx0 + (pw - 1) * sx2 + 1) * (unsigned)ES);
    const helix_rsrc rb  = make_rsrc(B_g + (long long)t0 * p.s_b[0], ((tlen - 1) * sb0 + N) * (unsigned)ES);
    st.dtraw = buf_elem<float>(rdt, min(lane, tlen - 1) * sdt, 0);
    const int xc = min(lane, pw - 1) * sx2;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int jr = min(16 * wave + i, tlen - 1);
        st.x[i] = io_load_word<IO>(rx, xc, jr * sx0);
    }
    constexpr int NB = NP / 32;
    const int lo = lane & 31, hi = lane >> 5;
    const int nb = min(NB * lo, N - NB) * ES;           // byte offset of the lane's run
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int jr = min(16 * wave + 8 * hi + e, tlen - 1);
        const int off = nb + jr * sb0 * ES;
        // The run's BW words: 4, 8, 16 or 32 bytes, in 16-byte loads at most.
        constexpr int BW = StageX6<NP, IO>::BW;
        if constexpr (BW == 1) {
            st.b[e][0] = __builtin_amdgcn_raw_buffer_load_b32(rb, off, 0, 0);
        } else if constexpr (BW == 2) {
            const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rb, off, 0, 0);
            st.b[e][0] = w[0];
            st.b[e][1] = w[1];
        } else {
#pragma unroll
            for (int q = 0; q < BW / 4; ++q) {
                const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rb, off + 16 * q, 0, 0);
#pragma unroll
                for (int k = 0; k < 4; ++k) st.b[e][4 * q + k] = w[k];
            }
        }
    }
}

// bf16 copies of B and C for the walking Pass C (bcopy/ccopy, helix_params.h).
// The K = heads_per_group * n_pslab workgroups of a chunk share its 64 rows:
// workgroup `id` takes rows j = id + K k. Thread tid handles the quads
// (four state indices) q = tid + 256 i, i < 2, of those rows: row slot
// k = q / (N/4), quad u = q % (N/4) (the host selects this only when the
// rows fit: ceil(64 / K) * N/4 <= 512). The fp32 quads travel with the
// chunk's register stage; rows past tlen are neither read nor written.
struct CopyBC {
    u32x4 b[2], c[2];
};
struct CopyMap {
    int j[2], u[2];     // row and quad of slot i; j >= 64 means none
};

__device__ __forceinline__ CopyMap copy_map(int tid, int id, int K, int N) {
    CopyMap m;
    const int nq = N >> 2;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = tid + 256 * i;
        const int k = q / nq;
        m.u[i] = q - k * nq;
        m.j[i] = min(id + K * k, 64);
    }
    return m;
}

__device__ __forceinline__ void load_copy_bc(CopyBC& cp, const CopyMap& m, const HelixScanParams& p,
                                             const float* __restrict__ B_g, const float* __restrict__ C_g,
                                             int c, int N) {
    const int t0   = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const int sb0 = sgpr_fresh((int)p.s_b[0]), sc0 = sgpr_fresh((int)p.s_c[0]);
    const helix_rsrc rb = make_rsrc(B_g + (long long)t0 * p.s_b[0], ((tlen - 1) * sb0 + N) * 4u);
    const helix_rsrc rc = make_rsrc(C_g + (long long)t0 * p.s_c[0], ((tlen - 1) * sc0 + N) * 4u);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        cp.b[i] = __builtin_amdgcn_raw_buffer_load_b128(
            rb, store_off_if_lt((m.j[i] * sb0 + 4 * m.u[i]) * 4, m.j[i], tlen, 0, 1), 0, 0);
        cp.c[i] = __builtin_amdgcn_raw_buffer_load_b128(
            rc, store_off_if_lt((m.j[i] * sc0 + 4 * m.u[i]) * 4, m.j[i], tlen, 0, 1), 0, 0);
    }
}

// Store the staged quads as bf16 (round to nearest even, as Pass C rounds
// its operands) at rows j of chunk c of the group's copy.
__device__ __forceinline__ void store_copy_bc(const CopyBC& cp, const CopyMap& m, const HelixScanParams& p,
                                              const HelixScanBuffers& b, int seq, int g, int c, int N) {
    const int t0   = (p.chunk_base + c) * HELIX_CS;
    const int tlen = min(HELIX_CS, p.n_tok - t0);
    const long long gn = (long long)p.n_group * N;
    const long long base = ((long long)seq * p.cpg * HELIX_CS + (long long)c * HELIX_CS) * gn + (long long)g * N;
    const unsigned bytes = (unsigned)((HELIX_CS - 1) * gn + N) * 2u;
    const helix_rsrc rb = make_rsrc(static_cast<__bf16*>(b.bcopy) + base, bytes);
    const helix_rsrc rc = make_rsrc(static_cast<__bf16*>(b.ccopy) + base, bytes);
    const int gni = (int)gn;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int off = store_off_if_lt((m.j[i] * gni + 4 * m.u[i]) * 2, m.j[i], tlen, 0, 1);
        const u32x2 wb = {pk_bf16(as_f32(cp.b[i][0]), as_f32(cp.b[i][1])), pk_bf16(as_f32(cp.b[i][2]), as_f32(cp.b[i][3]))};
        const u32x2 wc = {pk_bf16(as_f32(cp.c[i][0]), as_f32(cp.c[i][1])), pk_bf16(as_f32(cp.c[i][2]), as_f32(cp.c[i][3]))};
        __builtin_amdgcn_raw_buffer_store_b64(wb, rb, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b64(wc, rc, off, 0, 0);
    }
}

// Stage 16 consecutive tokens (chunks c0, c0 + 1) of row r of an NS-plane
// operand from fp32 values v[0..15].
template <int ROWS, int NS>
HELIX_DEV void stage_split_row(__bf16* planes, int r, int c0, const float (&v)[16]) {
    stage_split8<ROWS, NS>(planes, r, c0, v);
    stage_split8<ROWS, NS>(planes, r, c0 + 1, v + 8);
}

// MODE as in pass_a.hip: 0 store R_c fp32, 1 store R_c bf16, 2 aggregates only.
// IO: the caller's storage type of x and B. BCC: also write the bf16 copies
// of B and C (fp32 storage only). NS: bf16 planes per operand, 3 (six
// products, fp32 accuracy) or 2 (three products, about 2^-16 relative; the
// segment aggregates that only the bf16 path's walking Pass C and Pass B
// consume).
template <int NP, int MODE, typename IO = float, bool BCC = false, int NS = 3>
__device__ __forceinline__ void chunk_state_x6_impl(const HelixScanParams& p, const HelixScanBuffers& b) {
    static_assert(NS == 2 || NS == 3, "two or three split planes");
    constexpr bool SBF = MODE == 1;
    constexpr int NTW = NP / 64;      // N tiles per wave
    __shared__ __attribute__((aligned(16))) __bf16 sBt[NS * NP * HELIX_CS];
    __shared__ __attribute__((aligned(16))) __bf16 sXt[NS * HELIX_HD * HELIX_CS];

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
    const IO* __restrict__ x_h = reinterpret_cast<const IO*>(b.x) + seq * p.seq_x + h * p.s_x[1] + p0 * p.s_x[2];
    const IO* __restrict__ B_g = reinterpret_cast<const IO*>(b.B) + seq * p.seq_b + g * p.s_b[1];
    const float* __restrict__ C_g = b.C + seq * p.seq_c + g * p.s_c[1];
    const CopyMap cmap = BCC ? copy_map(tid, (h % p.heads_per_group) * p.n_pslab + slab,
                                        p.heads_per_group * p.n_pslab, N)
                             : CopyMap{};

    const long long tile_off = state_tile_off(p, h, slab);
    const unsigned tile_elems = 64u * NP;

    const int pt  = wave & 1;
    const int nt0 = wave >> 1;

    f32x16 acc[NTW];
#pragma unroll
    for (int i = 0; i < NTW; ++i) acc[i] = zero16();
    float lam = 0.0f;  // log-decay accumulated over this segment before chunk c

    // Decay preamble of chunk c (lane = token; dtv = 0 past tlen), formed by
    // one wave per chunk: wave (c - c_begin) % 4, one chunk ahead, while its
    // MFMAs for the previous chunk run. It leaves cf_j = exp(L_end - Lcum_j)
    // dt_j for the 64 tokens and (float)L_end in sPre[(c - c_begin) % 2],
    // and stores the chunk's decay record for Pass C.
    __shared__ __attribute__((aligned(16))) float sPre[2][HELIX_CS + 4];
    auto preamble = [&](float dtraw, int c) {
        const int t0   = (p.chunk_base + c) * HELIX_CS;
        const int tlen = min(HELIX_CS, p.n_tok - t0);
        const float dtv = keep_if_lt(helix_dt(p, dtraw), lane, tlen);
        const double lcum = wave_incl_sum((double)A_h * (double)dtv);
        const double lend = __shfl(lcum, 63, 64);
        float* dst = sPre[(c - c_begin) & 1];
        dst[lane] = keep_if_lt(exp_diff(lend, lcum) * dtv, lane, tlen);
        if (lane == 0) dst[HELIX_CS] = (float)lend;
        if (MODE == 2 && b.pre && slab == 0) store_decay_record(p, b, seq, c, h, lane, dtv, lcum);
        if (MODE == 0 && b.pre && slab == 0) store_decay_record64(p, b, seq, c, h, lane, dtv, lcum);
    };

    // Two register stages in turn: the loads of chunk c+2 are issued while
    // chunks c and c+1 are processed (a copy between stages would wait on them).
    // next_dtraw is chunk c+1's dt, from the other stage.
    auto step = [&](StageX6<NP, IO>& st, CopyBC& cp, int c, float next_dtraw) {
        const int buf  = (c - c_begin) & 1;
        const float lendf = sPre[buf][HELIX_CS];

        // dtXs^T[p][j] = exp(L_end - Lcum_j) dt_j x[j][p], row p = lane, and
        // B^T[n][j] (rows below). No masks: tokens past tlen have
        // cf_j = 0, so their B rows (clamped, finite) meet zeros; channels past
        // the slab and state indices past d_state only reach padding rows and
        // columns of R, which every consumer ignores.
        {
            float v[16];
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const f32x4 cf4 = *reinterpret_cast<const f32x4*>(&sPre[buf][16 * wave + 4 * i4]);
#pragma unroll
                for (int k = 0; k < 4; ++k) v[4 * i4 + k] = cf4[k] * io_widen<IO>(st.x[4 * i4 + k]);
            }
            stage_split_row<HELIX_HD, NS>(sXt, lane, 2 * wave, v);
        }
        // B^T rows NB lo + k, chunk 2 wave + hi (tokens 16 wave + 8 hi + e).
#pragma unroll
        for (int k = 0; k < NP / 32; ++k) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = x6_b(st, e, k);
            stage_split8<NP, NS>(sBt, (NP / 32) * lo + k, 2 * wave + hi, v);
        }

        if constexpr (BCC) store_copy_bc(cp, cmap, p, b, seq, g, c, N);

        if (MODE != 2 && c > c_begin) {
            const long long off = seq * p.sl_seq + (long long)c * p.sl_cg + tile_off;
            const void* dst = SBF ? (const void*)(static_cast<const __bf16*>(b.s_local) + off)
                                  : (const void*)(static_cast<const float*>(b.s_local) + off);
            const helix_rsrc rd = make_rsrc(dst, tile_elems * (SBF ? 2u : 4u));
#pragma unroll
            for (int i = 0; i < NTW; ++i) {
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int u = tile_unit(NP / 32, pt, nt0 + 2 * i, r4, 0);
                    const float v0 = acc[i][4 * r4], v1 = acc[i][4 * r4 + 1];
                    const float v2 = acc[i][4 * r4 + 2], v3 = acc[i][4 * r4 + 3];
                    if (SBF)
                        buf_store_unit<__bf16>(rd, v0, v1, v2, v3, lane, u);
                    else
                        buf_store_unit<float>(rd, v0, v1, v2, v3, lane, u);
                }
            }
        }
        if (slab == 0 && tid == 0) b.ld[seq * p.ld_seq + (long long)c * p.n_head + h] = lam;

        __syncthreads();

        // This register stage is free again: chunk c+2's inputs travel while
        // this chunk's and the next one's GEMMs run. The loads are issued on
        // every path (past the segment they re-read its last chunk, unused):
        // the compiler's vmcnt waits hold for every path through the loop, and
        // a skipped group would make the other stage's group the most recent
        // one, so each step would also wait for the loads just issued.
        {
            const int cn = min(c + 2, c_end - 1);
            load_stage_x6<NP, IO>(st, p, dt_h, x_h, B_g, cn, lane, wave, pw, N);
            if constexpr (BCC) load_copy_bc(cp, cmap, p, reinterpret_cast<const float*>(B_g), C_g, cn, N);
        }

        const float a_c = expf(lendf);
#pragma unroll
        for (int i = 0; i < NTW; ++i) acc[i] *= a_c;

        // R[n][p] += sum_j B^T[n][j] dtXs^T[p][j] over four K steps of 16 tokens.
#pragma unroll
        for (int s = 0; s < HELIX_CS / 16; ++s) {
            const int cx = 2 * s + hi;
            bf16x8 xs[NS];
#pragma unroll
            for (int k = 0; k < NS; ++k)
                xs[k] = *reinterpret_cast<const bf16x8*>(&sXt[x6_off<HELIX_HD, 8>(k, pt * 32 + lo, cx)]);
#pragma unroll
            for (int i = 0; i < NTW; ++i) {
                const int rn = (nt0 + 2 * i) * 32 + lo;
                bf16x8 bs[NS];
#pragma unroll
                for (int k = 0; k < NS; ++k)
                    bs[k] = *reinterpret_cast<const bf16x8*>(&sBt[x6_off<NP, 8>(k, rn, cx)]);
                // Smallest terms first.
                if constexpr (NS == 3) {
                    acc[i] = mfma_bf16(bs[2], xs[0], acc[i]);
                    acc[i] = mfma_bf16(bs[1], xs[1], acc[i]);
                    acc[i] = mfma_bf16(bs[0], xs[2], acc[i]);
                }
                acc[i] = mfma_bf16(bs[1], xs[0], acc[i]);
                acc[i] = mfma_bf16(bs[0], xs[1], acc[i]);
                acc[i] = mfma_bf16(bs[0], xs[0], acc[i]);
            }
        }
        // The next chunk's preamble, by one wave, while this chunk's MFMAs run;
        // the barrier below publishes it.
        if (c + 1 < c_end && wave == ((c + 1 - c_begin) & 3)) preamble(next_dtraw, c + 1);
        lam += lendf;
        __syncthreads();
    };
    StageX6<NP, IO> sa, sb;
    CopyBC ca, cb;
    load_stage_x6<NP, IO>(sa, p, dt_h, x_h, B_g, c_begin, lane, wave, pw, N);
    if constexpr (BCC) load_copy_bc(ca, cmap, p, reinterpret_cast<const float*>(B_g), C_g, c_begin, N);
    {
        const int cn = min(c_begin + 1, c_end - 1);
        load_stage_x6<NP, IO>(sb, p, dt_h, x_h, B_g, cn, lane, wave, pw, N);
        if constexpr (BCC) load_copy_bc(cb, cmap, p, reinterpret_cast<const float*>(B_g), C_g, cn, N);
    }
    if (wave == 0) preamble(sa.dtraw, c_begin);
    __syncthreads();
    for (int c = c_begin; c < c_end; c += 2) {
        step(sa, ca, c, sb.dtraw);
        if (c + 1 < c_end) step(sb, cb, c + 1, sa.dtraw);
    }

    const float* sg = b.s_seg + seq * p.sg_seq + (long long)seg * p.sg_seg + tile_off;
    const helix_rsrc rs = make_rsrc(sg, tile_elems * 4u);
#pragma unroll
    for (int i = 0; i < NTW; ++i) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int u = tile_unit(NP / 32, pt, nt0 + 2 * i, r4, 0);
            buf_store_unit<float>(rs, acc[i][4 * r4], acc[i][4 * r4 + 1], acc[i][4 * r4 + 2],
                                  acc[i][4 * r4 + 3], lane, u);
        }
    }
    if (slab == 0 && tid == 0) b.segld[seq * p.sd_seq + (long long)seg * p.n_head + h] = lam;
}

#define HELIX_PASS_A_X6(NP)                                                                     \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_state_x6f32_n##NP(        \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_state_x6_impl<NP, 0>(p, b);                                                       \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_state_x6agg_n##NP(        \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_state_x6_impl<NP, 2>(p, b);                                                       \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_state_x6agg_bc_n##NP(     \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_state_x6_impl<NP, 2, float, true>(p, b);                                          \
    }

// Segment aggregates on two split planes (three products) for the bf16 path's
// walking Pass C: fp32 storage, with and without the bf16 copies of B and C,
// and 16-bit storage of x and B.
#define HELIX_PASS_A_X3(NP)                                                                     \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_state_x3agg_n##NP(        \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_state_x6_impl<NP, 2, float, false, 2>(p, b);                                      \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_state_x3agg_bc_n##NP(     \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_state_x6_impl<NP, 2, float, true, 2>(p, b);                                       \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_state_x3agg_bf16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_state_x6_impl<NP, 2, __bf16, false, 2>(p, b);                                     \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_state_x3agg_f16io_n##NP(  \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_state_x6_impl<NP, 2, _Float16, false, 2>(p, b);                                   \
    }

// Aggregates from 16-bit storage of x and B (io_dtype BF16 / F16), for the
// chunk-walking Pass C.
#define HELIX_PASS_A_X6_IO(NP)                                                                  \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_state_x6agg_bf16io_n##NP( \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_state_x6_impl<NP, 2, __bf16>(p, b);                                               \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(HELIX_WG) void helix_chunk_state_x6agg_f16io_n##NP(  \
        HelixScanParams p, HelixScanBuffers b) {                                                \
        chunk_state_x6_impl<NP, 2, _Float16>(p, b);                                             \
    }

// d_state 256 only: up to 128 the head-block kernels (pass_a_hb.hip) serve.
HELIX_PASS_A_X6(256)
HELIX_PASS_A_X6_IO(256)
HELIX_PASS_A_X3(256)
