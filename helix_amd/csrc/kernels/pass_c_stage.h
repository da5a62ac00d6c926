// pass_c_stage.h -- register staging shared by the fp32 and bf16 Pass C kernels.
#ifndef HELIX_PASS_C_STAGE_H
#define HELIX_PASS_C_STAGE_H

#include "helix_common.h"

// One (head, P slab) item's global inputs for this thread: dt, x, and the two
// halves of S_init (S_seg of the segment, fp32, and R_c, the in-segment prefix
// Pass A left). Loaded for item k+1 while item k's GEMMs run. All addresses are
// clamped in bounds; the tile masks are applied when staging into LDS.
// Wave w takes the slab tile's units with r4 = w: unit m of its share is
// tile (pt, nt) = (m / NT, m % NT), i.e. rows p = pt*32 + lo and state
// indices n = nt*32 + 8w + 4hi + 0..3. The units stay in their loaded form
// until staged, so none of these loads has a consumer before then.
// REC: the item's decay record (store_decay_record64) replaces dt and A.
template <int NP, typename SL, bool REC = false>
struct StageC {
    float A;
    float dtraw;
    u32x4 rec;
    float ld;
    float x[16];
    u32x4 sg[NP / 16];
    typename RawUnit<SL>::type sl[NP / 16];   // R_c; 0 for a segment's first chunk
};

template <int NP, typename SL, bool REC = false>
__device__ __forceinline__ void load_stage_c(StageC<NP, SL, REC>& st, const HelixScanParams& p,
                                             const HelixScanBuffers& b, const float* __restrict__ x_s,
                                             const float* __restrict__ dt_s, const SL* __restrict__ sl_s,
                                             const float* __restrict__ sg_s, int seq, int cg, int t0,
                                             int tlen, int cis, int h, int slab, int lane, int wave) {
    const int P = p.head_dim;
    const int p0 = slab * HELIX_HD;
    const int pw = min(HELIX_HD, P - p0);
    if constexpr (!REC) st.A = b.A[(long long)h * p.s_a];
    st.ld = b.ld[seq * p.ld_seq + (long long)cg * p.n_head + h];
    // dt and x of this head and chunk through buffer resources based at the
    // chunk's first token (the host keeps a chunk's extent below 2 GiB).
    const int sdt = (int)p.s_dt[0], sx0 = sgpr_fresh((int)p.s_x[0]), sx2 = (int)p.s_x[2];
    const helix_rsrc rdt = make_rsrc(dt_s + h * p.s_dt[1] + (long long)t0 * p.s_dt[0],
                                     ((tlen - 1) * sdt + 1) * 4u);
    const helix_rsrc rx = make_rsrc(x_s + h * p.s_x[1] + (long long)t0 * p.s_x[0] + (long long)p0 * p.s_x[2],
                                    ((tlen - 1) * sx0 + (pw - 1) * sx2 + 1) * 4u);
    if constexpr (REC) {
        const helix_rsrc rr = make_rsrc(b.pre + (((long long)seq * p.cpg + cg) * p.n_head + h) * (HELIX_CS * 4),
                                        HELIX_CS * 16u);
        st.rec = __builtin_amdgcn_raw_buffer_load_b128(rr, lane * 16, 0, 0);
    } else {
        st.dtraw = buf_elem<float>(rdt, min(lane, tlen - 1) * sdt, 0);
    }
    const int xc = min(lane, pw - 1) * sx2;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int jr = min(16 * wave + i, tlen - 1);    // wave w: tokens 16w .. 16w+15
        st.x[i] = buf_elem<float>(rx, xc, jr * sx0);
    }
    // The slab tile is one contiguous, wave-uniform region: buffer loads with
    // the lane as the VGPR offset and the unit row as a constant. R_c is zero
    // for a segment's first chunk, which Pass A never writes: an empty range
    // makes those loads return 0 without a branch.
    const long long toff = state_tile_off(p, h, slab);
    const helix_rsrc rg = make_rsrc(sg_s + toff, 64u * NP * sizeof(float));
    const helix_rsrc rl = make_rsrc(sl_s + toff, cis > 0 ? 64u * NP * sizeof(SL) : 0u);
#pragma unroll
    for (int m = 0; m < NP / 16; ++m) {
        const int u = sgpr_fresh((m * 4 + wave) * 64);   // tile_unit(NT, m / NT, m % NT, wave, 0)
        st.sg[m] = buf_unit_raw<float>(rg, lane, u);
        st.sl[m] = buf_unit_raw<SL>(rl, lane, u);
    }
}

// Rows of C and B of one (seq, chunk, group) for this thread: row
// wave + NWV i (NWV waves), columns lane + 64 m, clamped in bounds (masked
// when staged). IO is the caller's storage type of B and C; the values stay
// in storage form (io_widen at the use).
template <int NP, typename IO = float, int NWV = 4>
__device__ __forceinline__ void load_cb_rows(typename IoWord<IO>::type (&vc)[HELIX_CS / NWV][NP / 64],
                                             typename IoWord<IO>::type (&vb)[HELIX_CS / NWV][NP / 64],
                                             const HelixScanParams& p, const HelixScanBuffers& b,
                                             int seq, int g, int t0, int tlen, int lane, int wave) {
    const int N = p.d_state;
    const int sc0 = (int)p.s_c[0], sb0 = (int)p.s_b[0];
    const IO* C = reinterpret_cast<const IO*>(b.C);
    const IO* B = reinterpret_cast<const IO*>(b.B);
    const helix_rsrc rc = make_rsrc(C + seq * p.seq_c + g * p.s_c[1] + (long long)t0 * p.s_c[0],
                                    ((tlen - 1) * sc0 + N) * (unsigned)sizeof(IO));
    const helix_rsrc rb = make_rsrc(B + seq * p.seq_b + g * p.s_b[1] + (long long)t0 * p.s_b[0],
                                    ((tlen - 1) * sb0 + N) * (unsigned)sizeof(IO));
#pragma unroll
    for (int i = 0; i < HELIX_CS / NWV; ++i) {
        const int jr = min(wave + NWV * i, tlen - 1);
#pragma unroll
        for (int m = 0; m < NP / 64; ++m) {
            const int nc = min(lane + 64 * m, N - 1);
            vc[i][m] = io_load_word<IO>(rc, nc, jr * sc0);
            vb[i][m] = io_load_word<IO>(rb, nc, jr * sb0);
        }
    }
}

// Store one 32 x 32 output tile (t block tb, P block pb of the slab at p0) of
// head h: lane (lo, hi), register r holds y[t = 32 tb + acc_row(r, hi)][32 pb + lo].
// Rows past tlen and columns past the slab width are not written; with
// tlen <= 0 nothing is (t0 must still address a row of y). IO is the
// caller's storage type of y; the stores are non-temporal.
template <typename IO = float>
__device__ __forceinline__ void store_y_tile(const f32x16& acc, const HelixScanParams& p,
                                             const HelixScanBuffers& b, int seq, int h, int t0,
                                             int tlen, int p0, int pw, int tb, int pb, int lo, int hi) {
    constexpr int ES = (int)sizeof(IO);
    const int sy0 = sgpr_fresh((int)p.s_y[0]), sy2 = (int)p.s_y[2];
    // tlen <= 0 stores nothing: the resource's range is empty, so the range
    // check drops every store whatever its offset.
    const unsigned bytes = tlen > 0 ? ((tlen - 1) * sy0 + (pw - 1) * sy2 + 1) * (unsigned)ES : 0u;
    const helix_rsrc ry = make_rsrc(reinterpret_cast<IO*>(b.y) + seq * p.seq_y + h * p.s_y[1] +
                                        (long long)t0 * p.s_y[0] + (long long)p0 * p.s_y[2],
                                    bytes);
    const int pp = pb * 32 + lo;
    const int voff = (4 * hi * sy0 + pp * sy2) * ES;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int t = tb * 32 + acc_row(r, hi);
        // The element goes through a float value: a bit cast applied to a
        // vector element in place reads element 0 with this compiler.
        const float v = acc[r];
        io_store<IO, HELIX_NT>(ry, v, store_off_if_lt(voff, t, tlen, pp, pw), (tb * 32 + 8 * (r >> 2) + (r & 3)) * sy0 * ES);
    }
}

// Store a walking wave's y tile of one chunk (16 x 16 MFMA layout, lane
// (q, c16) of P column pp): acc[tb] register r holds
// y[t = 16 tb + 4 q + r][pp]. Rows past tlen and columns past the slab width
// are dropped by the range check; with tlen <= 0 nothing is stored.
template <typename IO>
__device__ __forceinline__ void store_y16(const f32x4 (&acc)[4], const HelixScanParams& p,
                                          const HelixScanBuffers& b, int seq, int h, int t0, int tlen,
                                          int p0, int pw, int pp, int q) {
    constexpr int ES = (int)sizeof(IO);
    const int sy0 = sgpr_fresh((int)p.s_y[0]), sy2 = (int)p.s_y[2];
    const unsigned bytes = tlen > 0 ? ((tlen - 1) * sy0 + (pw - 1) * sy2 + 1) * (unsigned)ES : 0u;
    const helix_rsrc ry = make_rsrc(reinterpret_cast<IO*>(b.y) + seq * p.seq_y + h * p.s_y[1] +
                                        (long long)t0 * p.s_y[0] + (long long)p0 * p.s_y[2],
                                    bytes);
    const int voff = (4 * q * sy0 + pp * sy2) * ES;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 16 * tb + 4 * q + r;
            const float v = acc[tb][r];
            io_store<IO, HELIX_NT>(ry, v, store_off_if_lt(voff, t, tlen, pp, pw), (16 * tb + r) * sy0 * ES);
        }
}

#endif  // HELIX_PASS_C_STAGE_H
