/* helix_oracle.h -- CPU oracle for the HELIX SSD scan. TEST INFRASTRUCTURE.
 *
 * This is the checker, not the product: only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it. The HIP library never links
 * it and never falls back to it.
 *
 * Every function computes in double and rounds to float only on store, as
 * the reference's fp64 oracle does (src/reference/scan_ref.cpp:33-143,
 * src/reference/scan_chunked_ref.cpp:30-137). Inputs and outputs are laid
 * out by the helix_scan_desc element strides (include/helix/helix.h).
 *
 * Pinning (how each function is checked, see tests/test_oracle.py):
 *   oracle_scan            bit-exact against the reference's own ref::scan
 *                          compiled from /root/reference into oracle/_ref,
 *                          against committed golden vectors, and against
 *                          closed forms (L=1, B=0 pure decay, x=0, P=N=1
 *                          brute force, softplus > 20 shortcut).
 *   oracle_scan_mt         bit-exact against oracle_scan (same per-element
 *                          arithmetic, threads split (seq, head) pairs).
 *   oracle_scan_chunked    against ref::scan_chunked (bit-exact) and
 *                          oracle_scan (f32 round-off), chunk invariance.
 *   oracle_scan_snapshots  against ref::scan_with_snapshots (bit-exact) and
 *                          the state-splitting invariant.
 *   oracle_problem_harness byte-exact against the reference's tests/harness.hpp
 *                          Problem::make compiled into oracle/_ref.
 *   oracle_problem_gauss   parity unpinned by the reference (BASELINE.json's
 *                          generator has no reference counterpart); its
 *                          moments are checked statistically.
 */
#ifndef HELIX_ORACLE_H
#define HELIX_ORACLE_H

#include <stdint.h>

#include "helix/helix.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Sequential fp64 recurrence per (seq, head, chan); scan_ref.cpp:33-76.
 * head_mask: NULL = every head, else heads with head_mask[h] == 0 are skipped
 * (their y rows and s1 rows are left untouched). */
void oracle_scan(const helix_scan_desc* d,
                 const float* s0, const float* x, const float* dt, const float* A,
                 const float* B, const float* C, const int32_t* ids,
                 float* y, float* s1, const uint8_t* head_mask);

/* Same arithmetic as oracle_scan, split over `nthreads` POSIX threads by
 * (seq, head) pair. nthreads <= 0 means one per online CPU. */
void oracle_scan_mt(const helix_scan_desc* d,
                    const float* s0, const float* x, const float* dt, const float* A,
                    const float* B, const float* C, const int32_t* ids,
                    float* y, float* s1, const uint8_t* head_mask, int nthreads);

/* Chunked / reassociated fp64 SSD (scalar-A only); scan_chunked_ref.cpp:30-137.
 * Uses d->chunk (0 => 64). */
void oracle_scan_chunked(const helix_scan_desc* d,
                         const float* s0, const float* x, const float* dt, const float* A,
                         const float* B, const float* C, const int32_t* ids,
                         float* y, float* s1);

/* Sequential scan that also records the state after the last token of every
 * chunk, in the caller's s layout, as doubles; scan_ref.cpp:80-143.
 * out_states holds ceil(n_tok/chunk) * (n_seq*seq_s) doubles. */
void oracle_scan_snapshots(const helix_scan_desc* d,
                           const float* s0, const float* x, const float* dt, const float* A,
                           const float* B, const float* C, const int32_t* ids,
                           float* y, float* s1, int32_t chunk, double* out_states);

/* The reference harness generator (tests/harness.hpp:22-44,151-186):
 * xorshift64 (13/7/17), uniform fills in the order s0, x, dt, A, B, C.
 * memory: 0 = SHORT, 1 = LONG. Arrays are dense in the helix.h layouts. */
void oracle_problem_harness(int32_t n_tok, int32_t n_seq, int32_t n_head,
                            int32_t head_dim, int32_t d_state, int32_t n_group,
                            uint64_t seed, int memory,
                            float* s0, float* x, float* dt, float* A, float* B, float* C);

/* Gaussian generator for the BASELINE.json configs. Same xorshift64 stream,
 * normals by Box-Muller (one normal per two draws), fill order s0, x, dt, A,
 * B, C:
 *   s0    ~ N(0, s0_sigma)            (all zero when s0_sigma == 0)
 *   x     ~ N(0, 1)
 *   dt    ~ N(dt_mu, dt_sigma)        pre-softplus, as the ABI expects
 *   A     =  -exp(U(ln a_lo, ln a_hi))
 *   B, C  ~ N(0, 1) / sqrt(d_state)                                       */
void oracle_problem_gauss(int32_t n_tok, int32_t n_seq, int32_t n_head,
                          int32_t head_dim, int32_t d_state, int32_t n_group,
                          uint64_t seed, double s0_sigma, double dt_mu, double dt_sigma,
                          double a_lo, double a_hi,
                          float* s0, float* x, float* dt, float* A, float* B, float* C);

#ifdef __cplusplus
}
#endif

#endif /* HELIX_ORACLE_H */
