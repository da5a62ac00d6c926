/* helix_host.h -- host-side extras of the MI355X HELIX build.
 *
 * None of these entry points has a counterpart in the reference ABI. The
 * host-only context and plan_info exist for callers that plan without a GPU
 * (build machines, schedulers sizing scratch pools ahead of time) and for the
 * CPU test suite; helix_scan_encode_noalloc for callers that cannot allocate.
 */
#ifndef HELIX_HOST_H
#define HELIX_HOST_H

#include "helix/helix.h"

#ifdef __cplusplus
extern "C" {
#endif

/* A context bound to no device. helix_scan_supported, helix_scan_scratch_size,
 * helix_ctx_select_backend, helix_ctx_backend_desc and helix_scan_plan_info
 * answer exactly as on a gfx950 context; helix_scan_encode* return
 * HELIX_ERR_NO_DEVICE without touching HIP. Free with helix_ctx_free. */
helix_status helix_ctx_create_host(helix_ctx** out);

/* The plan helix_scan_encode would use for `d`. With multipass = false, or a
 * diagonal A, it needs no scratch: one launch of kernel_1pass (one group,
 * kernel_a/b/c NULL), or, where state_in_y is 1, the three passes with their
 * state tiles in y. */
typedef struct {
    int32_t  n_chunks;          /* ceil(n_tok / 64)                              */
    int32_t  chunks_per_group;  /* chunks per super-chunk group (scratch bound)  */
    int32_t  n_groups;          /* sequential groups, carried through s1         */
    int32_t  seg_len;           /* chunks per Pass A segment                     */
    int32_t  segs_per_group;
    int32_t  hblk;              /* heads per Pass C workgroup                    */
    int32_t  n_hblk;            /* head blocks per B/C group                     */
    int32_t  bf16_state;        /* 1 on the bf16 path                            */
    uint64_t total_bytes;       /* == helix_scan_scratch_size()                  */
    uint64_t s_local_bytes;     /* per-chunk states                              */
    uint64_t s_seg_bytes;       /* segment aggregates / segment initial states   */
    int32_t  launches;          /* kernel launches per encode                    */
    int32_t  np;                /* d_state padding of the selected kernels       */
    const char* kernel_a;       /* code-object names of the Pass A, B and C      */
    const char* kernel_b;       /* kernels (static strings)                      */
    const char* kernel_c;
    const char* kernel_1pass;   /* the single-pass kernel, else NULL             */
    uint64_t bccopy_bytes;      /* bf16 copies of B and C Pass A writes for C    */
    uint64_t rec_bytes;         /* per-token decay records Pass A writes for C   */
    int32_t  walk_len;          /* chunks per walking Pass C workgroup (a
                                   multiple of seg_len; seg_len off the walk)    */
    int32_t  walks_per_group;
    int32_t  pass_b;            /* where Pass B's segment scan runs: one of
                                   HELIX_PASS_B_* (kernel_b is NULL unless it
                                   has a launch of its own)                      */
    int32_t  state_in_y;        /* 1: the single pass runs as kernel_a, kernel_b
                                   and kernel_c with their state tiles in y, no
                                   scratch (fp32 storage, scalar A, d_state
                                   <= 128, and a last segment long enough for a
                                   tile); helix_scan_encode runs kernel_1pass
                                   alone instead when y is not 16-byte aligned
                                   or overlaps x, dt, A, B, C, s0, ids or s1    */
    int32_t  state_blocks;      /* the number of blocks of state indices (equal,
                                   multiples of 8, at most 128) the scan runs
                                   as, one after another, each adding its share
                                   into y: 1 up to d_state 128; more above 256
                                   (the fp32 path) and, with fp32 storage and
                                   scalar A, from 129 (HELIX_STATE_BLOCKS=0:
                                   1 up to 256). The other fields describe one
                                   block (the largest); launches counts all of
                                   them. A single pass keeps its tiles in y
                                   (state_in_y) for the first block only     */
} helix_plan_info;

#define HELIX_PASS_B_LAUNCHED 0   /* kernel_b, between Pass A and Pass C         */
#define HELIX_PASS_B_IN_C     1   /* the walking Pass C's prologue               */

/* Returns HELIX_ERR_UNSUPPORTED_SHAPE when the descriptor is declined. */
helix_status helix_scan_plan_info(helix_ctx* ctx, const helix_scan_desc* d,
                                  helix_plan_info* out);

/* Size of the fixed scratch helix_scan_encode_noalloc uses on each GPU. */
#define HELIX_NOALLOC_SCRATCH_BYTES (128u << 20)

/* helix_scan_encode without a scratch argument, for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc. It has no counterpart in the reference ABI.
 *
 * Same descriptor, tensors, kernels and results as helix_scan_encode; the
 * scratch is a fixed device array of HELIX_NOALLOC_SCRATCH_BYTES that the
 * library holds on every GPU where this entry point has been called, until
 * the process ends (its address is resolved on the first call on that GPU).
 * The call allocates and frees nothing. Its plan is made for that array: a
 * scan whose plan under the context's budget needs more scratch is cut into
 * more super-chunk groups (carried through s1, as with a lower
 * HELIX_SCRATCH_MB), and only a scan that does not fit at one chunk per group
 * returns HELIX_ERR_SCRATCH_TOO_SMALL, before anything is enqueued; the
 * single pass needs none. No part of the array needs to start at zero: every
 * region a kernel reads is written earlier in the same encode.
 *
 * Every call on one GPU shares that GPU's array and it keeps the last call's
 * contents: calls whose work overlaps on one GPU (other streams, other
 * threads, other contexts) race and must be serialised by the caller. */
helix_status helix_scan_encode_noalloc(helix_ctx* ctx, void* stream, const helix_scan_desc* desc,
                                       helix_tensor s0, helix_tensor x, helix_tensor dt,
                                       helix_tensor A, helix_tensor B, helix_tensor C,
                                       helix_tensor ids, helix_tensor y, helix_tensor s1);

#ifdef __cplusplus
}
#endif

#endif /* HELIX_HOST_H */
