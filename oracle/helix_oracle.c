/* helix_oracle.c -- fp64 CPU oracle for the HELIX SSD scan. TEST INFRASTRUCTURE.
 *
 * A C restatement of the reference's ground truth. Each function names the
 * reference lines whose arithmetic it follows; the order of every floating
 * point operation is kept so that, built without FMA contraction, the outputs
 * are bit-identical to the reference's own C++ (checked in tests against
 * oracle/_ref, which is compiled from the reference sources).
 */
#include "helix_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* softplus with the v > 20 shortcut: scan_ref.cpp:13-17. */
static inline double softplus_d(double v) { return v > 20.0 ? v : log1p(exp(v)); }

/* softplus then clamp to [dt_min, dt_max]: scan_ref.cpp:19-24. */
static inline double dt_at(const helix_scan_desc* d, const float* dt,
                           int64_t seq, int64_t t, int64_t h) {
    double v = softplus_d((double)dt[seq * d->seq_dt + t * d->s_dt[0] + h * d->s_dt[1]]);
    if (v < d->dt_min) v = d->dt_min;
    if (v > d->dt_max) v = d->dt_max;
    return v;
}

/* A is one scalar per head or one per (head, state): scan_ref.cpp:26-29. */
static inline double a_at(const helix_scan_desc* d, const float* A, int64_t h, int64_t n) {
    return (double)A[h * d->s_a + (d->a_form == HELIX_A_DIAG_PER_CHANNEL ? n : 0)];
}

/* One (seq, head): every channel p walked over every token, scan_ref.cpp:42-73.
 * `s` is caller scratch of d_state doubles. When snaps != NULL the state after
 * the last token of each chunk is stored there (scan_ref.cpp:128-135). */
static void scan_head(const helix_scan_desc* d,
                      const float* s0, const float* x, const float* dt, const float* A,
                      const float* B, const float* C, const int32_t* ids,
                      float* y, float* s1, int64_t seq, int64_t h, double* s,
                      int32_t chunk, double* snaps, size_t snap_stride) {
    const int64_t P = d->head_dim, N = d->d_state;
    const int64_t heads_per_group = d->n_head / d->n_group;
    const int64_t src_seq = ids ? ids[seq] : seq;
    const int64_t g = h / heads_per_group;

    for (int64_t p = 0; p < P; ++p) {
        const float* s_in = s0 + src_seq * d->seq_s + h * d->s_s[0] + p * d->s_s[1];
        for (int64_t n = 0; n < N; ++n) s[n] = (double)s_in[n * d->s_s[2]];

        for (int64_t t = 0; t < d->n_tok; ++t) {
            const double dt_t = dt_at(d, dt, seq, t, h);
            const double x_t = (double)x[seq * d->seq_x + t * d->s_x[0] + h * d->s_x[1] + p * d->s_x[2]];
            const float* Bt = B + seq * d->seq_b + t * d->s_b[0] + g * d->s_b[1];
            const float* Ct = C + seq * d->seq_c + t * d->s_c[0] + g * d->s_c[1];

            double acc = 0.0;
            for (int64_t n = 0; n < N; ++n) {
                const double dA = exp(a_at(d, A, h, n) * dt_t);
                s[n] = dA * s[n] + dt_t * (double)Bt[n * d->s_b[2]] * x_t;
                acc += (double)Ct[n * d->s_c[2]] * s[n];
            }
            y[seq * d->seq_y + t * d->s_y[0] + h * d->s_y[1] + p * d->s_y[2]] = (float)acc;

            if (snaps && ((t + 1) % chunk == 0 || t + 1 == d->n_tok)) {
                const int64_t c = t / chunk;
                double* dst = snaps + (size_t)c * snap_stride + seq * d->seq_s + h * d->s_s[0] + p * d->s_s[1];
                for (int64_t n = 0; n < N; ++n) dst[n * d->s_s[2]] = s[n];
            }
        }

        float* s_out = s1 + seq * d->seq_s + h * d->s_s[0] + p * d->s_s[1];
        for (int64_t n = 0; n < N; ++n) s_out[n * d->s_s[2]] = (float)s[n];
    }
}

void oracle_scan(const helix_scan_desc* d,
                 const float* s0, const float* x, const float* dt, const float* A,
                 const float* B, const float* C, const int32_t* ids,
                 float* y, float* s1, const uint8_t* head_mask) {
    double* s = (double*)malloc(sizeof(double) * (size_t)(d->d_state > 0 ? d->d_state : 1));
    for (int64_t seq = 0; seq < d->n_seq; ++seq)
        for (int64_t h = 0; h < d->n_head; ++h) {
            if (head_mask && !head_mask[h]) continue;
            scan_head(d, s0, x, dt, A, B, C, ids, y, s1, seq, h, s, 0, NULL, 0);
        }
    free(s);
}

/* ------------------------------------------------------------------------- */
/* Threaded: the same per-(seq, head) work, distributed over POSIX threads.  */
/* ------------------------------------------------------------------------- */

typedef struct {
    const helix_scan_desc* d;
    const float *s0, *x, *dt, *A, *B, *C;
    const int32_t* ids;
    float *y, *s1;
    const uint8_t* head_mask;
    int tid, nthreads;
} mt_job;

static void* mt_worker(void* arg) {
    mt_job* j = (mt_job*)arg;
    const helix_scan_desc* d = j->d;
    double* s = (double*)malloc(sizeof(double) * (size_t)(d->d_state > 0 ? d->d_state : 1));
    const int64_t items = (int64_t)d->n_seq * d->n_head;
    for (int64_t i = j->tid; i < items; i += j->nthreads) {
        const int64_t seq = i / d->n_head, h = i % d->n_head;
        if (j->head_mask && !j->head_mask[h]) continue;
        scan_head(d, j->s0, j->x, j->dt, j->A, j->B, j->C, j->ids, j->y, j->s1, seq, h, s, 0, NULL, 0);
    }
    free(s);
    return NULL;
}

void oracle_scan_mt(const helix_scan_desc* d,
                    const float* s0, const float* x, const float* dt, const float* A,
                    const float* B, const float* C, const int32_t* ids,
                    float* y, float* s1, const uint8_t* head_mask, int nthreads) {
    if (nthreads <= 0) {
        long n = sysconf(_SC_NPROCESSORS_ONLN);
        nthreads = n > 0 ? (int)n : 1;
    }
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    mt_job jobs[256];
    for (int i = 0; i < nthreads; ++i) {
        mt_job j = {d, s0, x, dt, A, B, C, ids, y, s1, head_mask, i, nthreads};
        jobs[i] = j;
        pthread_create(&th[i], NULL, mt_worker, &jobs[i]);
    }
    for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------------- */
/* Snapshots: scan_ref.cpp:80-143.                                           */
/* ------------------------------------------------------------------------- */

void oracle_scan_snapshots(const helix_scan_desc* d,
                           const float* s0, const float* x, const float* dt, const float* A,
                           const float* B, const float* C, const int32_t* ids,
                           float* y, float* s1, int32_t chunk, double* out_states) {
    if (!out_states || chunk <= 0) {
        oracle_scan(d, s0, x, dt, A, B, C, ids, y, s1, NULL);
        return;
    }
    const size_t state_elems = (size_t)d->n_seq * d->n_head * d->head_dim * d->d_state;
    const int32_t n_chunks = (d->n_tok + chunk - 1) / chunk;
    memset(out_states, 0, sizeof(double) * state_elems * (size_t)n_chunks);
    double* s = (double*)malloc(sizeof(double) * (size_t)(d->d_state > 0 ? d->d_state : 1));
    for (int64_t seq = 0; seq < d->n_seq; ++seq)
        for (int64_t h = 0; h < d->n_head; ++h)
            scan_head(d, s0, x, dt, A, B, C, ids, y, s1, seq, h, s, chunk, out_states, state_elems);
    free(s);
}

/* ------------------------------------------------------------------------- */
/* Chunked SSD in fp64: scan_chunked_ref.cpp:30-137.                          */
/* ------------------------------------------------------------------------- */

void oracle_scan_chunked(const helix_scan_desc* d,
                         const float* s0, const float* x, const float* dt, const float* A,
                         const float* B, const float* C, const int32_t* ids,
                         float* y, float* s1) {
    const int64_t H = d->n_head, P = d->head_dim, N = d->d_state, L = d->n_tok;
    const int64_t CK = d->chunk > 0 ? d->chunk : 64;
    const int64_t heads_per_group = d->n_head / d->n_group;

    double* S    = (double*)malloc(sizeof(double) * (size_t)(P * N));
    double* dtX  = (double*)malloc(sizeof(double) * (size_t)(CK * P));
    double* M    = (double*)malloc(sizeof(double) * (size_t)(CK * CK));
    double* Lcum = (double*)malloc(sizeof(double) * (size_t)CK);

    for (int64_t seq = 0; seq < d->n_seq; ++seq) {
        const int64_t src_seq = ids ? ids[seq] : seq;
        for (int64_t h = 0; h < H; ++h) {
            const int64_t g = h / heads_per_group;
            const double A_h = (double)A[h * d->s_a];
            const float* s_in = s0 + src_seq * d->seq_s + h * d->s_s[0];
            for (int64_t p = 0; p < P; ++p)
                for (int64_t n = 0; n < N; ++n)
                    S[p * N + n] = (double)s_in[p * d->s_s[1] + n * d->s_s[2]];

            for (int64_t t0 = 0; t0 < L; t0 += CK) {
                const int64_t tlen = (CK < L - t0) ? CK : (L - t0);

                /* dt, cumulative log-decay, dtX (scan_chunked_ref.cpp:66-79) */
                double run = 0.0;
                for (int64_t j = 0; j < tlen; ++j) {
                    double v = softplus_d((double)dt[seq * d->seq_dt + (t0 + j) * d->s_dt[0] + h * d->s_dt[1]]);
                    const double lo = d->dt_min, hi = d->dt_max;
                    v = (v < lo) ? lo : (hi < v) ? hi : v;   /* std::clamp */
                    run += A_h * v;
                    Lcum[j] = run;
                    for (int64_t p = 0; p < P; ++p)
                        dtX[j * P + p] = v * (double)x[seq * d->seq_x + (t0 + j) * d->s_x[0] + h * d->s_x[1] + p * d->s_x[2]];
                }
                const double L_end = Lcum[tlen - 1];

                /* G1: masked, decayed C.B^T (scan_chunked_ref.cpp:81-95) */
                for (int64_t t = 0; t < tlen; ++t) {
                    const float* Ct = C + seq * d->seq_c + (t0 + t) * d->s_c[0] + g * d->s_c[1];
                    for (int64_t j = 0; j < tlen; ++j) {
                        if (j > t) { M[t * CK + j] = 0.0; continue; }
                        const float* Bj = B + seq * d->seq_b + (t0 + j) * d->s_b[0] + g * d->s_b[1];
                        double cb = 0.0;
                        for (int64_t n = 0; n < N; ++n)
                            cb += (double)Ct[n * d->s_c[2]] * (double)Bj[n * d->s_b[2]];
                        M[t * CK + j] = cb * exp(Lcum[t] - Lcum[j]);
                    }
                }

                /* G2 + G3 (scan_chunked_ref.cpp:97-113) */
                for (int64_t t = 0; t < tlen; ++t) {
                    const float* Ct = C + seq * d->seq_c + (t0 + t) * d->s_c[0] + g * d->s_c[1];
                    const double exp_Lt = exp(Lcum[t]);
                    for (int64_t p = 0; p < P; ++p) {
                        double intra = 0.0;
                        for (int64_t j = 0; j <= t; ++j) intra += M[t * CK + j] * dtX[j * P + p];
                        double inter = 0.0;
                        for (int64_t n = 0; n < N; ++n) inter += (double)Ct[n * d->s_c[2]] * S[p * N + n];
                        y[seq * d->seq_y + (t0 + t) * d->s_y[0] + h * d->s_y[1] + p * d->s_y[2]] =
                            (float)(intra + exp_Lt * inter);
                    }
                }

                /* G4 + state update (scan_chunked_ref.cpp:115-128) */
                const double chunk_decay = exp(L_end);
                for (int64_t p = 0; p < P; ++p)
                    for (int64_t n = 0; n < N; ++n) {
                        double ds = 0.0;
                        for (int64_t j = 0; j < tlen; ++j) {
                            const float* Bj = B + seq * d->seq_b + (t0 + j) * d->s_b[0] + g * d->s_b[1];
                            ds += exp(L_end - Lcum[j]) * (double)Bj[n * d->s_b[2]] * dtX[j * P + p];
                        }
                        S[p * N + n] = chunk_decay * S[p * N + n] + ds;
                    }
            }

            float* s_out = s1 + seq * d->seq_s + h * d->s_s[0];
            for (int64_t p = 0; p < P; ++p)
                for (int64_t n = 0; n < N; ++n)
                    s_out[p * d->s_s[1] + n * d->s_s[2]] = (float)S[p * N + n];
        }
    }
    free(S); free(dtX); free(M); free(Lcum);
}

/* ------------------------------------------------------------------------- */
/* Generators                                                                */
/* ------------------------------------------------------------------------- */

/* xorshift64 with shifts 13/7/17: harness.hpp:22-34. */
typedef struct { uint64_t s; } rng_t;

static inline uint64_t rng_next(rng_t* r) {
    r->s ^= r->s << 13; r->s ^= r->s >> 7; r->s ^= r->s << 17;
    return r->s;
}
/* Uniform in [lo, hi) in float arithmetic: harness.hpp:29-33. */
static inline float rng_uniform(rng_t* r, float lo, float hi) {
    const float u = (float)(rng_next(r) >> 40) / 16777216.0f;
    return lo + u * (hi - lo);
}
static void fill_uniform(float* v, size_t n, rng_t* r, float lo, float hi) {
    for (size_t i = 0; i < n; ++i) v[i] = rng_uniform(r, lo, hi);
}

void oracle_problem_harness(int32_t n_tok, int32_t n_seq, int32_t n_head,
                            int32_t head_dim, int32_t d_state, int32_t n_group,
                            uint64_t seed, int memory,
                            float* s0, float* x, float* dt, float* A, float* B, float* C) {
    rng_t r = { seed ? seed : 1 };
    const size_t n_s  = (size_t)n_seq * n_head * head_dim * d_state;
    const size_t n_x  = (size_t)n_seq * n_tok * n_head * head_dim;
    const size_t n_dt = (size_t)n_seq * n_tok * n_head;
    const size_t n_bc = (size_t)n_seq * n_tok * n_group * d_state;

    fill_uniform(s0, n_s, &r, -0.5f, 0.5f);
    fill_uniform(x, n_x, &r, -1.0f, 1.0f);
    if (memory == 1) {                       /* LONG: harness.hpp:171-175 */
        fill_uniform(dt, n_dt, &r, -7.0f, -4.5f);
        for (int32_t h = 0; h < n_head; ++h) A[h] = -expf(rng_uniform(&r, -0.5f, 1.0f));
    } else {                                 /* SHORT: harness.hpp:176-179, 42-44 */
        fill_uniform(dt, n_dt, &r, -4.0f, 2.0f);
        for (int32_t h = 0; h < n_head; ++h) A[h] = -expf(rng_uniform(&r, -2.0f, 0.5f));
    }
    const float sc = 1.0f / sqrtf((float)d_state);   /* harness.hpp:182-184 */
    fill_uniform(B, n_bc, &r, -sc, sc);
    fill_uniform(C, n_bc, &r, -sc, sc);
}

/* Open-interval uniform double in (0, 1) from the top 53 bits. */
static inline double rng_u01(rng_t* r) {
    return ((double)(rng_next(r) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}
/* Box-Muller, cosine branch only: one normal per two draws. */
static inline double rng_normal(rng_t* r) {
    const double u1 = rng_u01(r), u2 = rng_u01(r);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
}

void oracle_problem_gauss(int32_t n_tok, int32_t n_seq, int32_t n_head,
                          int32_t head_dim, int32_t d_state, int32_t n_group,
                          uint64_t seed, double s0_sigma, double dt_mu, double dt_sigma,
                          double a_lo, double a_hi,
                          float* s0, float* x, float* dt, float* A, float* B, float* C) {
    rng_t r = { seed ? seed : 1 };
    const size_t n_s  = (size_t)n_seq * n_head * head_dim * d_state;
    const size_t n_x  = (size_t)n_seq * n_tok * n_head * head_dim;
    const size_t n_dt = (size_t)n_seq * n_tok * n_head;
    const size_t n_bc = (size_t)n_seq * n_tok * n_group * d_state;

    for (size_t i = 0; i < n_s; ++i) s0[i] = s0_sigma > 0.0 ? (float)(s0_sigma * rng_normal(&r)) : 0.0f;
    for (size_t i = 0; i < n_x; ++i) x[i] = (float)rng_normal(&r);
    for (size_t i = 0; i < n_dt; ++i) dt[i] = (float)(dt_mu + dt_sigma * rng_normal(&r));
    const double la = log(a_lo), lb = log(a_hi);
    for (int32_t h = 0; h < n_head; ++h) A[h] = (float)(-exp(la + (lb - la) * rng_u01(&r)));
    const double sc = 1.0 / sqrt((double)d_state);
    for (size_t i = 0; i < n_bc; ++i) B[i] = (float)(sc * rng_normal(&r));
    for (size_t i = 0; i < n_bc; ++i) C[i] = (float)(sc * rng_normal(&r));
}
