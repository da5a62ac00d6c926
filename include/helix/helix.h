/* helix.h -- HELIX public C ABI, MI355X (gfx950 / CDNA4) build.
 *
 * Chunked associative scan (SSD, the Mamba-2 state-space recurrence) for
 * prefill, exposed as a drop-in operator. Every name, enum value, struct
 * field and argument order below is the one the reference exposes in
 * include/helix/helix.h:36-218 (HELIX_ABI_VERSION 1), so a caller compiled
 * against that header links against this library unchanged. Only the meaning
 * of the opaque `void*` handles changes, because HIP has no command buffers
 * or encoders:
 *
 *   helix_ctx_create(out, device, code_object_path)
 *       device            NULL  -> the calling thread's current HIP device
 *                         else  -> (const int*) pointing at a HIP ordinal
 *       code_object_path  NULL  -> $HELIX_HSACO if set, else the gfx950 code
 *                                  object embedded in the library (libhelix.so
 *                                  or libhelix.a)
 *                         else  -> a gfx950 code object file to load instead
 *   helix_scan_encode(ctx, cmd_buffer, ...)        cmd_buffer is a hipStream_t
 *   helix_scan_encode_into(ctx, encoder, ...)      encoder is a hipStream_t
 *       NULL is the legacy default stream (valid in HIP, unlike a NULL Metal
 *       command buffer). Both forms enqueue the same kernels; ordering between
 *       passes comes from stream order.
 *   helix_tensor.buf      a device pointer (hipMalloc'd, or any pointer the
 *                         device can dereference); .offset is in BYTES.
 *
 * It is a pure encoder: it enqueues kernels on the caller's stream and never
 * allocates device memory, synchronizes, or waits. Scratch is caller-owned
 * and sized by helix_scan_scratch_size().
 *
 * Tensor layouts (fastest dimension last), element strides in the descriptor:
 *
 *   s0, s1 : (n_seq, n_head, head_dim, d_state)  f32  carried state
 *   x      : (n_seq, n_tok,  n_head,   head_dim)      input
 *   dt     : (n_seq, n_tok,  n_head)                  timestep, bias folded in,
 *                                                     BEFORE softplus
 *   A      : (n_head) scalar-per-head, or (n_head, d_state) diagonal
 *   B, C   : (n_seq, n_tok,  n_group,  d_state)
 *   y      : (n_seq, n_tok,  n_head,   head_dim)      output
 *
 * The operator applies softplus to dt (with the v > 20 shortcut) and the
 * optional [dt_min, dt_max] clamp. The D skip connection is the caller's.
 */

#ifndef HELIX_H
#define HELIX_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HELIX_ABI_VERSION 1

/* ------------------------------------------------------------------------- */
/* Enums (values fixed by ABI version 1)                                     */
/* ------------------------------------------------------------------------- */

typedef enum {
    HELIX_OK = 0,
    HELIX_ERR_UNSUPPORTED_SHAPE = 1, /* helix_scan_supported() would say false */
    HELIX_ERR_NO_DEVICE         = 2, /* no gfx950 device, or no code object   */
    HELIX_ERR_SCRATCH_TOO_SMALL = 3,
    HELIX_ERR_INVALID_ARG       = 4,
    HELIX_ERR_PIPELINE          = 5, /* kernel lookup / launch failed          */
} helix_status;

typedef enum {
    HELIX_F32  = 0,
    HELIX_F16  = 1,
    HELIX_BF16 = 2,
} helix_dtype;

typedef enum {
    /* One scalar A per head: Mamba-2 / SSD. The form this build accelerates. */
    HELIX_A_SCALAR_PER_HEAD = 0,
    /* One A per (head, state): Mamba-1 selective scan. Served by the fp32
     * single-pass kernel up to d_state 128 (the reference declines it). */
    HELIX_A_DIAG_PER_CHANNEL = 1,
} helix_a_form;

/* Backend names are kept for ABI compatibility. On MI355X:
 *   SGMMA -> the fp32 path: every result fp32-accurate. Passes A and C run
 *            fp32-accurate GEMMs on bf16 MFMA over operands split into three
 *            bf16 parts (six products); at d_state 256 Pass C runs on fp32
 *            MFMA (v_mfma_f32_32x32x2_f32)
 *   MPP   -> the bf16 path: Pass C's GEMM operands are bf16
 *            (v_mfma_f32_16x16x32_bf16, fp32 accumulation); Pass A keeps the
 *            fp32-accurate six-product GEMM and Pass B is fp32, so the carried
 *            state and s1 stay fp32-accurate
 *   AUTO  -> MPP whenever the shape is served by it, else SGMMA
 *   REF   -> reported when no usable context exists; never launched
 * multipass = false runs the fp32-accurate single-pass kernel under AUTO and
 * SGMMA. */
typedef enum {
    HELIX_BACKEND_AUTO  = 0,
    HELIX_BACKEND_SGMMA = 1,
    HELIX_BACKEND_MPP   = 2,
    HELIX_BACKEND_REF   = 3,
} helix_backend;

/* ------------------------------------------------------------------------- */
/* Tensors                                                                   */
/* ------------------------------------------------------------------------- */

/* A view into caller-owned device memory: `buf` is a device pointer and
 * `offset` is in BYTES from it. HELIX never frees or retains either. */
typedef struct {
    void*    buf;
    uint64_t offset;
} helix_tensor;

#ifdef __cplusplus
#define HELIX_TENSOR_NULL (helix_tensor{ NULL, 0 })
#else
#define HELIX_TENSOR_NULL ((helix_tensor){ NULL, 0 })
#endif

static inline bool helix_tensor_is_null(helix_tensor t) { return t.buf == NULL; }

/* ------------------------------------------------------------------------- */
/* Descriptor                                                                */
/* ------------------------------------------------------------------------- */

/* Strides are in ELEMENTS (ggml's nb[] divided by the element size). */
typedef struct {
    int32_t n_tok;     /* L, tokens in this slice           */
    int32_t n_seq;     /* independent sequences             */
    int32_t n_head;    /* H                                 */
    int32_t head_dim;  /* P (ggml: d_inner)                 */
    int32_t d_state;   /* N                                 */
    int32_t n_group;   /* G, divides n_head                 */

    int64_t s_x[3];    /* (tok, head, chan)                 */
    int64_t s_b[3];    /* (tok, group, state)               */
    int64_t s_c[3];    /* (tok, group, state)               */
    int64_t s_dt[2];   /* (tok, head)                       */
    int64_t s_s[3];    /* (head, chan, state) in a sequence */
    int64_t s_y[3];    /* (tok, head, chan)                 */
    int64_t s_a;       /* stride between heads in A         */
    int64_t seq_x;     /* per-sequence strides              */
    int64_t seq_b;
    int64_t seq_c;
    int64_t seq_dt;
    int64_t seq_s;
    int64_t seq_y;

    int32_t       chunk;          /* 0 => library chooses (64); else must be 64 */
    helix_a_form  a_form;
    helix_dtype   io_dtype;       /* storage of x/B/C/y: F32, F16 or BF16       */
    helix_dtype   compute_dtype;  /* must stay F32; bf16 is chosen by backend   */
    helix_backend backend;
    bool          multipass;      /* 3-pass chunk-parallel decomposition        */

    float dt_min;                 /* clamp of softplus(dt); 0 / +inf disables   */
    float dt_max;
} helix_scan_desc;

/* Fills every field with its default and the dense strides of the shape:
 * chunk 0, scalar-A, F32/F32, AUTO, multipass=false, dt_min 0, dt_max +inf. */
void helix_scan_desc_init(helix_scan_desc* d,
                          int32_t n_tok, int32_t n_seq, int32_t n_head,
                          int32_t head_dim, int32_t d_state, int32_t n_group);

/* ------------------------------------------------------------------------- */
/* Context                                                                   */
/* ------------------------------------------------------------------------- */

typedef struct helix_ctx helix_ctx;

/* Binds to one gfx950 device and resolves every kernel up front, so encode
 * only reads the context. See the top of this file for the handle meanings. */
helix_status helix_ctx_create(helix_ctx** out, void* device, const char* code_object_path);
void         helix_ctx_free(helix_ctx* ctx);

/* Last error message recorded by the calling thread on this context. Never
 * NULL; "" when nothing has failed. */
const char*  helix_ctx_last_error(const helix_ctx* ctx);

/* Which backend this descriptor resolves to on this context. */
helix_backend helix_ctx_select_backend(helix_ctx* ctx, const helix_scan_desc* d);

/* Static, never-NULL name of the kernel variant the shape resolves to, e.g.
 * "mfma bf16 pass C (d_state=128)". Selection fails soft, so this is the
 * only way to see which path actually runs. */
const char* helix_ctx_backend_desc(helix_ctx* ctx, const helix_scan_desc* d);

/* ------------------------------------------------------------------------- */
/* Scan                                                                      */
/* ------------------------------------------------------------------------- */

/* True if this build serves the descriptor. False means the caller keeps its
 * own implementation. */
bool helix_scan_supported(helix_ctx* ctx, const helix_scan_desc* d);

/* Bytes of device scratch the multipass path needs (0 when multipass=false).
 * Pure function of the descriptor and $HELIX_SCRATCH_MB. */
size_t helix_scan_scratch_size(helix_ctx* ctx, const helix_scan_desc* d);

/* Enqueues the scan on stream `cmd_buffer` (a hipStream_t). No allocation, no
 * synchronization. `ids` is an optional int32 (n_seq) map from output
 * sequence to source state row of s0 (HELIX_TENSOR_NULL = identity).
 * `scratch` may be HELIX_TENSOR_NULL when helix_scan_scratch_size() is 0.
 * On any error nothing has been enqueued. */
helix_status helix_scan_encode(helix_ctx*             ctx,
                               void*                  cmd_buffer,
                               const helix_scan_desc* d,
                               helix_tensor           s0,
                               helix_tensor           x,
                               helix_tensor           dt,
                               helix_tensor           A,
                               helix_tensor           B,
                               helix_tensor           C,
                               helix_tensor           ids,
                               helix_tensor           y,
                               helix_tensor           s1,
                               helix_tensor           scratch);

/* Identical to helix_scan_encode: `encoder` is also a hipStream_t. Kept so a
 * host written against the reference's encoder-reuse entry point links. */
helix_status helix_scan_encode_into(helix_ctx*             ctx,
                                    void*                  encoder,
                                    const helix_scan_desc* d,
                                    helix_tensor           s0,
                                    helix_tensor           x,
                                    helix_tensor           dt,
                                    helix_tensor           A,
                                    helix_tensor           B,
                                    helix_tensor           C,
                                    helix_tensor           ids,
                                    helix_tensor           y,
                                    helix_tensor           s1,
                                    helix_tensor           scratch);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* HELIX_H */
