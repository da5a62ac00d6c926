// pass_c_stage.h -- register staging shared by the fp32 and bf16 Pass C kernels.
#ifndef HELIX_PASS_C_STAGE_H
#define HELIX_PASS_C_STAGE_H

#include "helix_common.h"

// One (head, P slab) item's global inputs for this thread: dt, x, and the two
// halves of S_init (S_seg of the segment, fp32, and R_c, the in-segment prefix
// Pass A left). Loaded for item k+1 while item k's GEMMs run. All addresses are
// clamped in bounds; the tile masks are applied when staging into LDS.
template <int NP, typename SL>
struct StageC {
    float A;
    float dtraw;
    float ld;
    float x[16];
    float sg[16][NP / 64];
    SL    sl[16][NP / 64];
};

template <int NP, typename SL>
__device__ __forceinline__ void load_stage_c(StageC<NP, SL>& st, const HelixScanParams& p,
                                             const HelixScanBuffers& b, const float* __restrict__ x_s,
                                             const float* __restrict__ dt_s, const SL* __restrict__ sl_s,
                                             const float* __restrict__ sg_s, int seq, int cg, int t0,
                                             int tlen, int cis, int h, int slab, int lane, int wave) {
    const int N = p.d_state, P = p.head_dim;
    const int p0 = slab * HELIX_HD;
    const int pw = min(HELIX_HD, P - p0);
    st.A = b.A[(long long)h * p.s_a];
    st.ld = b.ld[seq * p.ld_seq + (long long)cg * p.n_head + h];
    st.dtraw = dt_s[h * p.s_dt[1] + (long long)(t0 + min(lane, tlen - 1)) * p.s_dt[0]];
    const float* xh = x_s + h * p.s_x[1] + (long long)(p0 + min(lane, pw - 1)) * p.s_x[2];
    const long long head_off = (long long)h * P * N;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int jr = min(wave + 4 * i, tlen - 1);
        st.x[i] = xh[(long long)(t0 + jr) * p.s_x[0]];
        const long long row = head_off + (long long)(p0 + min(wave + 4 * i, pw - 1)) * N;
#pragma unroll
        for (int m = 0; m < NP / 64; ++m) {
            const long long off = row + min(lane + 64 * m, N - 1);
            st.sg[i][m] = sg_s[off];
            if (cis > 0) st.sl[i][m] = sl_s[off];
        }
    }
}


#endif  // HELIX_PASS_C_STAGE_H
