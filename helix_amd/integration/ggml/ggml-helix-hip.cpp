// ggml-helix-hip.cpp -- the bridge between ggml's HIP backend and HELIX.
//
// Counterpart of the reference's integration/ggml/ggml-helix.cpp:1-361, the
// ggml-metal bridge. On the HIP backend (ggml-cuda compiled for ROCm) the
// mapping is direct:
//   * a tensor's `data` is already a device pointer, views included, so each
//     operand is helix_tensor{data, 0} (no buffer-id lookup);
//   * the op runs on the backend context's hipStream_t, which is HELIX's
//     command buffer (stream order replaces Metal's encoder rules, so there is
//     no encode_into special case);
//   * ggml's nb[] are byte strides and helix_scan_desc takes element strides,
//     so the mapping is a division, not a repack.
//
// Layouts (ggml side, fastest dimension first), as in the reference
// (ggml-helix.cpp:14-27):
//   src0  s    {d_state, head_dim, n_head, n_seqs}
//   src1  x    {head_dim, n_head, n_tokens, n_seqs}
//   src2  dt   {n_head, n_tokens, n_seqs}
//   src3  A    {1 | d_state, n_head}
//   src4  B    {d_state, n_group, n_tokens, n_seqs}
//   src5  C    {d_state, n_group, n_tokens, n_seqs}
//   src6  ids  {n_seqs}                                  int32
//   dst        y (nelements(src1) floats, dense), then the final state
//
// HELIX writes s1 with s0's strides, so the bridge serves only a dense s0 (the
// state region of dst is dense); the reference maps any s0 strides onto the
// packed dst and would scatter s1 for a padded one.
#include "ggml-helix-hip.h"

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <unordered_map>

#include "ggml.h"
#include "helix/helix.h"

namespace {

// ---------------------------------------------------------------------------
// Switches, read per call (cheap; lets a host flip them between graphs)
// ---------------------------------------------------------------------------

bool env_is_one(const char* name) {
    const char* v = std::getenv(name);
    return v && v[0] == '1';
}

int min_tokens() {
    if (const char* t = std::getenv("GGML_HELIX_MIN_TOKENS")) return std::atoi(t);
    return 64;
}

// ---------------------------------------------------------------------------
// One HELIX context per device, created on first use and kept for the process
// (encode only reads it, so concurrent encoding threads share it).
// ---------------------------------------------------------------------------

std::mutex g_ctx_mu;
std::unordered_map<int, helix_ctx*> g_ctx;

helix_ctx* context_for(int device) {
    std::lock_guard<std::mutex> lock(g_ctx_mu);
    auto it = g_ctx.find(device);
    if (it != g_ctx.end()) return it->second;
    helix_ctx* c = nullptr;
    int dev = device;
    const helix_status st = helix_ctx_create(&c, &dev, nullptr);
    if (st != HELIX_OK) {
        std::fprintf(stderr, "ggml-helix: HELIX unavailable on device %d (status %d), using ggml kernels\n",
                     device, (int)st);
        c = nullptr;
    }
    g_ctx.emplace(device, c);
    return c;
}

// ---------------------------------------------------------------------------
// Fallback scratch: per thread and device, grown on demand, never shrunk
// (reference ggml-helix.cpp:94-130 keeps its scratch the same way, because
// llama.cpp may encode graph segments from several threads).
// ---------------------------------------------------------------------------

struct Scratch {
    void*  ptr = nullptr;
    size_t size = 0;
};
thread_local std::unordered_map<int, Scratch> t_scratch;

void* scratch_for(int device, hipStream_t stream, size_t bytes) {
    Scratch& s = t_scratch[device];
    if (s.ptr && s.size >= bytes) return s.ptr;
    int prev = -1;
    (void)hipGetDevice(&prev);
    if (prev != device && hipSetDevice(device) != hipSuccess) return nullptr;
    if (s.ptr) {
        // Work already enqueued by this thread may still read the old buffer.
        (void)hipStreamSynchronize(stream);
        (void)hipFree(s.ptr);
        s = Scratch{};
    }
    void* p = nullptr;
    if (hipMalloc(&p, bytes) == hipSuccess) s = Scratch{p, bytes};
    if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
    return s.ptr;
}

// ggml nb[] are byte strides; helix_scan_desc takes element strides.
bool elems(size_t nb, int64_t* out) {
    if (nb % sizeof(float) != 0) return false;
    *out = (int64_t)(nb / sizeof(float));
    return true;
}

helix_tensor view(const ggml_tensor* t) {
    return t ? helix_tensor{t->data, 0} : HELIX_TENSOR_NULL;
}

bool prepare(int device, const ggml_tensor* op, helix_ctx** ctx, helix_scan_desc* d) {
    if (!op || env_is_one("GGML_HELIX_DISABLE")) return false;
    if (!helix_ggml_build_desc(op, d)) return false;
    *ctx = context_for(device);
    return *ctx && helix_scan_supported(*ctx, d);
}

}  // namespace

extern "C" bool helix_ggml_build_desc(const ggml_tensor* op, helix_scan_desc* d) {
    if (!op || !d) return false;
    const ggml_tensor* s  = op->src[0];
    const ggml_tensor* x  = op->src[1];
    const ggml_tensor* dt = op->src[2];
    const ggml_tensor* A  = op->src[3];
    const ggml_tensor* B  = op->src[4];
    const ggml_tensor* C  = op->src[5];
    if (!s || !x || !dt || !A || !B || !C) return false;

    // HELIX produces one final state; K > 1 asks for K rollback snapshots, a
    // different output contract (reference ggml-helix.cpp:165-169).
    if (op->op_params[0] != 1) return false;

    for (const ggml_tensor* t : {s, x, dt, A, B, C, op})
        if (t->type != GGML_TYPE_F32) return false;

    const int64_t d_state  = s->ne[0];
    const int64_t head_dim = s->ne[1];
    const int64_t n_head   = s->ne[2];
    const int64_t n_group  = B->ne[1];
    const int64_t n_tok    = x->ne[2];
    const int64_t n_seq    = x->ne[3];
    if (n_head <= 0 || n_group <= 0 || n_head % n_group != 0) return false;
    if (n_tok < min_tokens()) return false;
    if (n_tok > INT32_MAX || n_seq > INT32_MAX || n_head > INT32_MAX || head_dim > INT32_MAX ||
        d_state > INT32_MAX)
        return false;

    // The state region of dst is dense; s1 is written with s0's strides.
    const size_t fs = sizeof(float);
    if (s->nb[0] != fs || s->nb[1] != (size_t)d_state * fs || s->nb[2] != (size_t)(d_state * head_dim) * fs ||
        s->nb[3] != (size_t)(d_state * head_dim * n_head) * fs)
        return false;

    helix_scan_desc_init(d, (int32_t)n_tok, (int32_t)n_seq, (int32_t)n_head, (int32_t)head_dim,
                         (int32_t)d_state, (int32_t)n_group);
    bool ok = true;
    // s: (head, chan, state) within a sequence.
    ok = ok && elems(s->nb[2], &d->s_s[0]) && elems(s->nb[1], &d->s_s[1]) && elems(s->nb[0], &d->s_s[2]) &&
         elems(s->nb[3], &d->seq_s);
    // x: (tok, head, chan).
    ok = ok && elems(x->nb[2], &d->s_x[0]) && elems(x->nb[1], &d->s_x[1]) && elems(x->nb[0], &d->s_x[2]) &&
         elems(x->nb[3], &d->seq_x);
    // dt: (tok, head).
    ok = ok && elems(dt->nb[1], &d->s_dt[0]) && elems(dt->nb[0], &d->s_dt[1]) && elems(dt->nb[2], &d->seq_dt);
    // B and C: (tok, group, state).
    ok = ok && elems(B->nb[2], &d->s_b[0]) && elems(B->nb[1], &d->s_b[1]) && elems(B->nb[0], &d->s_b[2]) &&
         elems(B->nb[3], &d->seq_b);
    ok = ok && elems(C->nb[2], &d->s_c[0]) && elems(C->nb[1], &d->s_c[1]) && elems(C->nb[0], &d->s_c[2]) &&
         elems(C->nb[3], &d->seq_c);
    if (!ok) return false;

    // A is {1, n_head} for the scalar (Mamba-2 / SSD) form and {d_state,
    // n_head} for the per-channel diagonal (reference ggml-helix.cpp:247-258).
    if (A->ne[0] == 1)
        d->a_form = HELIX_A_SCALAR_PER_HEAD;
    else if (A->ne[0] == d_state)
        d->a_form = HELIX_A_DIAG_PER_CHANNEL;
    else
        return false;
    if (!elems(A->nb[1], &d->s_a)) return false;

    // y is the leading region of dst, dense in x's logical shape.
    d->s_y[0] = n_head * head_dim;
    d->s_y[1] = head_dim;
    d->s_y[2] = 1;
    d->seq_y  = n_tok * n_head * head_dim;

    // ggml applies no clamp to softplus(dt).
    d->dt_min = 0.0f;
    d->dt_max = INFINITY;

    d->multipass = true;
    d->backend   = env_is_one("GGML_HELIX_MPP") ? HELIX_BACKEND_AUTO : HELIX_BACKEND_SGMMA;
    return true;
}

extern "C" bool ggml_hip_ssm_scan_helix_plan(int device, const ggml_tensor* op, size_t* scratch_bytes) {
    helix_ctx* ctx = nullptr;
    helix_scan_desc d{};
    if (!prepare(device, op, &ctx, &d)) return false;
    if (scratch_bytes) *scratch_bytes = helix_scan_scratch_size(ctx, &d);
    return true;
}

extern "C" bool ggml_hip_op_ssm_scan_helix(void* stream, int device, const ggml_tensor* op, void* scratch,
                                           size_t scratch_bytes) {
    helix_ctx* ctx = nullptr;
    helix_scan_desc d{};
    if (!prepare(device, op, &ctx, &d)) return false;

    const hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t need = helix_scan_scratch_size(ctx, &d);
    void* sp = nullptr;
    if (need > 0) {
        if (scratch && scratch_bytes >= need)
            sp = scratch;
        else if (!scratch)
            sp = scratch_for(device, st, need);
        if (!sp) return false;
    }

    // dst holds y, then the final state at nelements(src1) floats.
    char* dst = static_cast<char*>(op->data);
    if (!dst) return false;
    const size_t s_off = (size_t)ggml_nelements(op->src[1]) * sizeof(float);
    const helix_tensor t_y  = helix_tensor{dst, 0};
    const helix_tensor t_s1 = helix_tensor{dst, (uint64_t)s_off};

    // Announce the kernel once: selection fails soft, so a declined shape or
    // an unexpected backend is otherwise invisible (reference :308-321).
    static std::once_flag announced;
    std::call_once(announced, [&] {
        std::fprintf(stderr, "ggml-helix: kernel = %s (d_state=%d head_dim=%d n_head=%d)\n",
                     helix_ctx_backend_desc(ctx, &d), (int)d.d_state, (int)d.head_dim, (int)d.n_head);
    });

    const helix_status rc =
        helix_scan_encode(ctx, st, &d, view(op->src[0]), view(op->src[1]), view(op->src[2]), view(op->src[3]),
                          view(op->src[4]), view(op->src[5]), view(op->src[6]), t_y, t_s1,
                          sp ? helix_tensor{sp, 0} : HELIX_TENSOR_NULL);
    if (rc != HELIX_OK) {
        // Nothing was enqueued: the caller's own kernel runs instead.
        std::fprintf(stderr, "ggml-helix: helix_scan_encode failed (%d): %s\n", (int)rc,
                     helix_ctx_last_error(ctx));
        return false;
    }
    return true;
}
