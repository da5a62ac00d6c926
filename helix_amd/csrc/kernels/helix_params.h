/* helix_params.h -- the structs shared by the C++ runtime and the gfx950
 * kernels. Plain C so both sides include it; passed by value as kernargs.
 *
 * Counterpart of the reference's HelixScanParams (src/kernels/helix_params.h:
 * 45-110), re-laid for MI355X: strides are int64 (288 GB of HBM admits tensors
 * past 2^31 elements; per-workgroup bases are formed once in scalar registers
 * and lane offsets inside a chunk stay 32-bit), and the multipass fields
 * describe the two-level segment scheme below instead of one scratch slot per
 * chunk.
 *
 * Two-level decomposition of the chunk recurrence S_{c+1} = a_c S_c + dS_c
 * (a_c = exp(sum of A*dt over chunk c), dS_c = B_c^T (decay . dt . x)_c):
 *
 *   Pass A  one workgroup per (seq, segment of seg_len chunks, head, P-slab)
 *           walks its chunks in order with the partial state held in MFMA
 *           accumulators. Before folding chunk c in, it stores the in-segment
 *           prefix R_c (state entering chunk c from this segment's own tokens,
 *           zero for the first chunk) to `s_local`. At the end it stores the
 *           segment aggregate D_s to `s_seg` and the log-decays to `ld`/`segld`.
 *   Pass B  per state element, scans the segments:
 *           S_seg(s) = carry; carry = exp(segld_s) carry + D_s   (in place)
 *           and writes the final carry to s1.
 *   Pass C  per (seq, chunk, group, head block): the state entering chunk c is
 *           S_init(c) = R_c + exp(ld_c) S_seg(s), assembled while staging;
 *           y = tril(C B^T . decay) (dt x) + exp(Lcum) . (C S_init).
 *
 * Scratch layouts (elements; every region 256-byte aligned):
 *   s_local [seq][cg][head][slab] x TILE   f32 (fp32 path) or bf16 (bf16 path)
 *   s_seg   [seq][seg][head][slab] x TILE  f32: D_s from Pass A, S_seg after Pass B
 *   ld      [seq][cg][head]                f32: sum of chunk log-decays before c
 *                                               within c's segment
 *   segld   [seq][seg][head]               f32: whole-segment log-decay
 *   bcopy, ccopy [seq][t][group][n]        bf16: B and C of the group's cpg*64
 *                                  tokens (t counted from the group's first
 *                                  token), written by Pass A for the walking
 *                                  Pass C (optional; rows past n_tok unwritten)
 * A TILE holds one 64-channel slab of one head's state, [64 p][np n] padded,
 * in the order Pass A's MFMA result registers hold it (v_mfma_f32_32x32x2_f32
 * computing R[n][p], M = n, N = p), grouped in units of four registers:
 *   unit(pt, nt, r4, lane) = ((pt * np/32 + nt) * 4 + r4) * 64 + lane
 *   holds state[p = pt*32 + lane%32][n = nt*32 + 8*r4 + 4*(lane/32) + 0..3]
 * A unit is four consecutive n of one p: 16 bytes in fp32, 8 in bf16. Each
 * group of four result registers stores as one 16-byte (8-byte) write per
 * lane, 1 KiB (512 B) contiguous per wave; Pass B moves s0/s1 as 16-byte runs
 * of the caller's [P][N] layout; and a lane's units are the B operand of
 * Pass C's C . S GEMM as they stand (the K order of an MFMA is free as long as
 * both operands use the same one).
 * Padding (p past head_dim in the last slab, n past d_state) holds finite
 * values no result depends on: Pass C zeroes it when staging S_init (and C is
 * zero past d_state), y is stored only for p < head_dim, and Pass B writes s1
 * only for valid (p, n).
 */
#ifndef HELIX_PARAMS_H
#define HELIX_PARAMS_H

/* Chunk length. 64 tokens = one wave64 lane per token for the decay scan. */
#define HELIX_CS 64
/* Head-dim slab width handled by one workgroup. */
#define HELIX_HD 64
/* Largest d_state one kernel launch serves (padded up to 64 / 128 / 256
 * inside the kernels). The host runs a larger d_state as blocks of state
 * indices, at most HELIX_N_BLOCK each, adding each block's share of y into y
 * (HelixScanParams::y_acc). */
#define HELIX_N_MAX 256
#define HELIX_N_BLOCK 128
/* Threads per workgroup: four wave64s, one per SIMD of a CU. */
#define HELIX_WG 256
/* Bytes of one token's decay record (HelixScanBuffers::pre): the walking bf16
 * Pass C's {dt, Lcum log2(e)}, and the fp32 path's {dt, exp(Lcum), Lcum as
 * fp64}. */
#define HELIX_REC_WALK_BYTES 8
#define HELIX_REC64_BYTES 16
/* Heads per workgroup of the chunk-walking Pass C (four waves per head):
 * two up to d_state 128; one at 256, where a head's state needs the whole
 * register budget of a wave. */
#define HELIX_WALK_HPW(np) ((np) <= 128 ? 2 : 1)
/* Heads per workgroup of the 16 x 16 tile walk: as for the 32 x 32 walk (one
 * head per workgroup, two workgroups per CU, measured slower at config 2:
 * the B and C staging is then done for every head). */
#define HELIX_WALK16_HPW(np) HELIX_WALK_HPW(np)
/* Waves per workgroup of the scalar-A single-pass kernels: eight up to
 * d_state 128; four at d_state 256, whose registers do not fit two waves per
 * SIMD (the diagonal-A kernels run four). */
#define HELIX_1PASS_WAVES(np) ((np) <= 128 ? 8 : 4)
/* Items ((head, P slab) pairs of one B/C group) per workgroup of the
 * head-block Pass A (pass_a_hb.hip), two waves each, d_state <= 128. */
#define HELIX_HB 4
#define HELIX_HB_THREADS (128 * HELIX_HB)

typedef struct HelixScanParams {
    int n_tok;
    int n_seq;
    int n_head;
    int head_dim;
    int d_state;
    int n_group;
    int heads_per_group;
    int n_pslab;          /* ceil(head_dim / HELIX_HD) */

    /* Element strides, as in helix_scan_desc. */
    long long s_x[3], seq_x;
    long long s_b[3], seq_b;
    long long s_c[3], seq_c;
    long long s_dt[2], seq_dt;
    long long s_s[3], seq_s;
    long long s_y[3], seq_y;
    long long s_a;

    int   has_ids;
    int   first_group;    /* 1 => Pass B carries in from s0 (through ids), else s1 */
    float dt_min;
    float dt_max;

    /* Super-chunk group currently encoded. */
    int chunk_base;       /* global index of the group's first chunk */
    int n_cg;             /* chunks in this group */
    int seg_len;          /* chunks per segment (Pass A, Pass B, chunk-parallel Pass C) */
    int n_seg;            /* segments in this group = ceil(n_cg / seg_len) */
    int walk_len;         /* chunks per walking Pass C workgroup, a multiple of
                             seg_len: walk segment w starts at segment
                             w * walk_len / seg_len */
    int n_walk;           /* walk segments in this group = ceil(n_cg / walk_len) */
    int hblk;             /* heads per Pass C workgroup */
    int n_hblk;           /* head blocks per B/C group */
    int np;               /* d_state padded to the kernels' tile width (64/128/256) */
    int cpg;              /* chunks per group of the plan (scratch strides) */
    int fuse_b;           /* 1 => no Pass B launch: the walking Pass C forms S_seg
                             from s0 and the aggregates D_s, and its last segment
                             writes s1 (single-group plans only) */
    int ytile;            /* 1 => the single pass (multipass = false) run as the
                             three passes with no scratch: the state tiles (Pass
                             A's aggregates, then the walks' start states) and the
                             segment log-decays live in y (ytile_* in
                             helix_common.h); single group, Pass B launched */
    int y_acc;            /* 1 => y += this launch's result (a block of state
                             indices after the first: y is the sum over the
                             blocks of C_n h_n); 0 => y = result */

    /* Scratch strides in elements (see the layout comment above). */
    long long sl_cg, sl_seq;     /* s_local: chunk stride (H*n_pslab*64*np), seq stride */
    long long sg_seg, sg_seq;    /* s_seg: segment stride (H*n_pslab*64*np), seq stride */
    long long ld_seq;            /* ld: seq stride (n_cg_max * H); chunk stride H */
    long long sd_seq;            /* segld: seq stride (n_seg_max * H); seg stride H */
} HelixScanParams;

/* Device pointers for one encode. s_local is float* on the fp32 path and a
 * bf16 array on the bf16 path. */
typedef struct HelixScanBuffers {
    const float* s0;
    const float* x;
    const float* dt;
    const float* A;
    const float* B;
    const float* C;
    const int*   ids;
    float*       y;
    float*       s1;
    void*        s_local;
    float*       s_seg;
    float*       ld;
    float*       segld;
    void*        bcopy;   /* bf16 copies of B and C (see the layout above), or null */
    void*        ccopy;
    float*       pre;     /* per-token decay records [seq][chunk][head][64] that
                             Pass A writes for the Pass C that reads them, or
                             null: {dt, Lcum log2(e)} (HELIX_REC_WALK_BYTES) for
                             the 16 x 16 walk, {dt, exp(Lcum), Lcum (fp64)}
                             (HELIX_REC64_BYTES) for the fp32 path's bf16x6 Pass C */
} HelixScanBuffers;

#endif /* HELIX_PARAMS_H */
