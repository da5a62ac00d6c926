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
    with_y_acc(p, [&](auto acc_on) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = tb * 32 + acc_row(r, hi);
            // The element goes through a float value: a bit cast applied to a
            // vector element in place reads element 0 with this compiler.
            const float v = acc[r];
            y_store<IO, decltype(acc_on)::value>(ry, v, store_off_if_lt(voff, t, tlen, pp, pw),
                                                 (tb * 32 + 8 * (r >> 2) + (r & 3)) * sy0 * ES);
        }
    });
}

// Store a walking wave's y tile of one chunk (16 x 16 MFMA layout, lane
// (q, c16) of P column pp): acc[tb] register r holds
// y[t = 16 tb + 4 q + r][pp]. Rows past tlen and columns past the slab width
// are dropped by the range check; with tlen <= 0 nothing is stored. AUX: the
// stores' cache policy (HELIX_NT, or HELIX_NT_L2 for the walk on Pass A's
// bf16 copies of B and C). RT_ACC: add what y holds when p.y_acc is set (off
// for a caller that loaded it ahead with load_y16 and added it to acc).
template <typename IO, int AUX = HELIX_NT, bool RT_ACC = true>
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
    auto put = [&](auto acc_on) {
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * tb + 4 * q + r;
                const float v = acc[tb][r];
                y_store<IO, decltype(acc_on)::value, AUX>(ry, v, store_off_if_lt(voff, t, tlen, pp, pw),
                                                          (16 * tb + r) * sy0 * ES);
            }
    };
    if constexpr (RT_ACC)
        with_y_acc(p, put);
    else
        put(std::false_type{});
}

// What y holds at the elements store_y16 would store (fp32 storage), 0 where
// it would store nothing: for a walk that adds into y (HelixScanParams::y_acc),
// loaded a chunk's work ahead of the stores so the loads' latency is hidden.
__device__ __forceinline__ void load_y16(f32x4 (&yv)[4], const HelixScanParams& p, const HelixScanBuffers& b,
                                         int seq, int h, int t0, int tlen, int p0, int pw, int pp, int q) {
    const int sy0 = sgpr_fresh((int)p.s_y[0]), sy2 = (int)p.s_y[2];
    const unsigned bytes = tlen > 0 ? ((tlen - 1) * sy0 + (pw - 1) * sy2 + 1) * 4u : 0u;
    const helix_rsrc ry = make_rsrc(b.y + seq * p.seq_y + h * p.s_y[1] + (long long)t0 * p.s_y[0] +
                                        (long long)p0 * p.s_y[2],
                                    bytes);
    const int voff = (4 * q * sy0 + pp * sy2) * 4;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 16 * tb + 4 * q + r;
            yv[tb][r] = buf_f32(ry, store_off_if_lt(voff, t, tlen, pp, pw), (16 * tb + r) * sy0 * 4);
        }
}


// The start state R of a walk segment, in the walks' register layout: R[nb][r]
// = S[16 nb + 4 q + r][p0 + pp] (q = lane / 16, pp = 16 w4 + c16). Without
// p.fuse_b it is Pass B's S_seg tile of the Pass A segment the walk segment
// starts at; with p.fuse_b the tiles hold Pass A's segment aggregates and the
// workgroup runs Pass B's recurrence here. YT: the single pass without
// scratch (HelixScanParams::ytile, never with fuse_b): the tile is in y.
template <int NP, bool YT = false>
__device__ __forceinline__ void walk_start_state(f32x4 (&R)[NP / 16], const HelixScanParams& p,
                                                 const HelixScanBuffers& b, int seq, int h, int slab, int seg,
                                                 int p0, int pw, int pp, int q, int w4, int c16, bool head_ok) {
    constexpr int NB = NP / 16, NT32 = NP / 32;
    const int N = p.d_state, P = p.head_dim;
    // R[n][pp], n = 16 nb + 4 q + r, from the slab tile of S_seg(s): in the
    // tile's unit layout that is unit ((pt NT32 + nb/2) 4 + r4) 64 + lane'
    // with pt = w4/2, r4 = 2 (nb%2) + q/2, lane' = 32 (q%2) + 16 (w4%2) + c16.
    {
        const float* tiles = YT ? nullptr : b.s_seg + seq * p.sg_seq + state_tile_off(p, h, slab);
        const int vunit = 64 * (q >> 1) + 32 * (q & 1) + 16 * (w4 & 1) + c16;
        const int pt = w4 >> 1;
        if constexpr (YT) {
            // The tile of the walk's first Pass A segment, in y's rows of that
            // segment and the slab's columns (ytile_unit); the range covers
            // the rows the tile and its log-decay take.
            const int s = seg * (p.walk_len / p.seg_len);
            const int upr = pw >> 2;
            const unsigned rows = (unsigned)((16 * NP + 1 + upr - 1) / upr);
            const helix_rsrc ry = make_rsrc(b.y + ytile_base(p, seq, h, slab, s), rows * (unsigned)p.s_y[0] * 4u);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int u = vunit + ((pt * NT32 + (nb >> 1)) * 4 + 2 * (nb & 1)) * 64;
                R[nb] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      ry, (int)ytile_unit(p, u, pw) * 4, 0, 0));
            }
            return;
        }
        auto load_tile = [&](int s, f32x4 (&T)[NB]) {
            const helix_rsrc rg = make_rsrc(tiles + (long long)s * p.sg_seg, 64u * NP * sizeof(float));
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                T[nb] = buf_unit<float>(rg, vunit, ((pt * NT32 + (nb >> 1)) * 4 + 2 * (nb & 1)) * 64);
        };
        if (!p.fuse_b) {
            // S_seg of the Pass A segment this walk segment starts at, from Pass B.
            load_tile(seg * (p.walk_len / p.seg_len), R);
        } else {
            // Pass B folded in (single-group plans whose walk segments are Pass
            // A's segments): the tiles hold Pass A's
            // segment aggregates D_s, and this workgroup runs Pass B's
            // recurrence (helix_state_scan_f32, same operation order) up to
            // its own segment:
            //   carry = s0[ids[seq]];  carry = exp(segld_s) carry + D_s,  s < seg
            // The last segment's workgroup takes one more step and stores s1.
            // State index n = 16 nb + 4 q + r of channel p0 + pp; tile
            // padding (pp >= pw, n >= d_state) starts from zero, as in Pass B.
            // ids and the segment log-decays come through the scalar unit, so
            // using them does not wait for the first chunk's vector loads.
            const int src = p.has_ids ? sload_i32(b.ids, seq) : seq;
            const long long hs = (long long)h * p.s_s[0];
            const unsigned sbytes = (unsigned)(((long long)(P - 1) * p.s_s[1] + N) * 4);
            const int soff = (int)((p0 + pp) * p.s_s[1]) * 4;
            const helix_rsrc r0 = make_rsrc(b.s0 + src * p.seq_s + hs, sbytes);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int n = 16 * nb + 4 * q;
                const int off = store_off_if_lt(soff + 4 * n, pp, pw, n, N);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    R[nb][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r0, off + 4 * r, 0, 0));
            }
            const float* __restrict__ sd = b.segld + seq * p.sd_seq + h;
            const bool last = seg == p.n_seg - 1;
            const int nd = seg + (last ? 1 : 0);
            // Tiles in flight: four up to d_state 128, two at 256 (32 f32x4
            // registers either way; four tiles of 16 spill at d_state 256).
            constexpr int BLK = NB <= 8 ? 4 : 2;
            for (int sb = 0; sb < nd; sb += BLK) {
                f32x4 T[BLK][NB];
                float a[BLK];
#pragma unroll
                for (int k = 0; k < BLK; ++k) {
                    const int s = min(sb + k, nd - 1);
                    load_tile(s, T[k]);
                    a[k] = expf(sload_f32(sd, (long long)s * p.n_head));
                }
#pragma unroll
                for (int k = 0; k < BLK; ++k) {
                    if (sb + k >= nd) break;
                    if (sb + k < seg) {
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb) R[nb] = a[k] * R[nb] + T[k][nb];
                    } else if (head_ok) {
                        // s1[seq] = exp(segld_seg) S_seg(seg) + D_seg
                        // Element by element: with the quad formed as one
                        // vector expression, hipcc stored its first element
                        // four times.
                        const helix_rsrc r1 = make_rsrc(b.s1 + seq * p.seq_s + hs, sbytes);
                        const float ak = a[k];
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb) {
                            const int n = 16 * nb + 4 * q;
                            const int off = store_off_if_lt(soff + 4 * n, pp, pw, n, N);
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float v = ak * R[nb][r] + T[k][nb][r];
                                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r1,
                                                                      off + 4 * r, 0, 0);
                            }
                        }
                    }
                }
            }
        }
    }
}

#endif  // HELIX_PASS_C_STAGE_H
