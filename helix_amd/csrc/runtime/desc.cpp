// desc.cpp -- descriptor defaults and dense strides.
// Restates the reference's src/runtime/desc.cpp:9-46: same defaults, same
// dense strides for the layouts documented in include/helix/helix.h.
#include <cmath>
#include <cstring>

#include "helix/helix.h"

extern "C" void helix_scan_desc_init(helix_scan_desc* d, int32_t n_tok, int32_t n_seq,
                                     int32_t n_head, int32_t head_dim, int32_t d_state,
                                     int32_t n_group) {
    if (!d) return;
    std::memset(d, 0, sizeof(*d));
    d->n_tok = n_tok;
    d->n_seq = n_seq;
    d->n_head = n_head;
    d->head_dim = head_dim;
    d->d_state = d_state;
    d->n_group = n_group;

    const int64_t L = n_tok, H = n_head, P = head_dim, N = d_state, G = n_group;
    d->s_x[0] = H * P; d->s_x[1] = P; d->s_x[2] = 1; d->seq_x = L * H * P;
    d->s_y[0] = H * P; d->s_y[1] = P; d->s_y[2] = 1; d->seq_y = L * H * P;
    d->s_b[0] = G * N; d->s_b[1] = N; d->s_b[2] = 1; d->seq_b = L * G * N;
    d->s_c[0] = G * N; d->s_c[1] = N; d->s_c[2] = 1; d->seq_c = L * G * N;
    d->s_dt[0] = H;    d->s_dt[1] = 1;                d->seq_dt = L * H;
    d->s_s[0] = P * N; d->s_s[1] = N; d->s_s[2] = 1; d->seq_s = H * P * N;
    d->s_a = 1;

    d->chunk         = 0;
    d->a_form        = HELIX_A_SCALAR_PER_HEAD;
    d->io_dtype      = HELIX_F32;
    d->compute_dtype = HELIX_F32;
    d->backend       = HELIX_BACKEND_AUTO;
    d->multipass     = false;
    d->dt_min        = 0.0f;
    d->dt_max        = INFINITY;
}
