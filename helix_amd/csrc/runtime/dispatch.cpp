// dispatch.cpp -- the encoder.
//
// Counterpart of the reference's src/runtime/dispatch.mm:55-287. HELIX
// enqueues onto the caller's HIP stream and never allocates, synchronizes or
// waits. Every check (arguments, shape gate, scratch size, kernel handles,
// launch limits) happens before the first launch, so an error it reports
// leaves nothing enqueued. (A failure of the HIP launch call itself after the
// first group of a multi-group plan leaves the earlier groups enqueued.) Stream order sequences the passes; there are no barriers to
// insert.
//
// multipass = false, or a diagonal A: one launch of the single-pass kernel, grid
// (n_seq * n_head * n_pslab) x 256 threads, no scratch.
//
// Otherwise, per super-chunk group, in stream order:
//   Pass A  grid (n_seq * n_group * item blocks * segments) x 512 threads (the
//           head-block kernel, d_state <= 128; 1-D, decoded XCD-aware), or
//           grid (segments, n_head, n_seq * n_pslab) x 256 threads
//   Pass B  grid (ceil(n_pslab*16*np/256), n_head, n_seq) x 256 threads
//   Pass C  grid (chunks * n_group * n_hblk * n_seq)    x 256 threads (1-D,
//           decoded XCD-aware in the kernel); the walking variant runs one
//           workgroup of 256 * HELIX_WALK_HPW(np) threads per (walk segment,
//           block of that many heads of a group, P slab, seq) instead
// The ragged-tail padding and the bf16 staging of B and C that the reference
// runs as separate passes (dispatch.mm:218-245) happen inside the Pass A/C
// staging here, so there is nothing to launch before the group loop.
#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <string>

#include "helix/helix_host.h"
#include "helix_internal.h"

namespace {

using helix::rt::set_error;

inline void* dptr(helix_tensor t) {
    return t.buf ? static_cast<char*>(t.buf) + t.offset : nullptr;
}

// Byte range [lo, hi) of a tensor of n_seq sequences with the given
// per-sequence stride and (extent, stride) dimensions, element size es
// (strides are non-negative: the descriptor gate checks them).
struct ByteRange {
    uintptr_t lo = 0, hi = 0;
    bool overlaps(const ByteRange& o) const { return lo < o.hi && o.lo < hi; }
};
ByteRange byte_range(const void* base, long long n_seq, long long seq_stride,
                     std::initializer_list<std::pair<long long, long long>> dims, size_t es) {
    long long last = (n_seq - 1) * seq_stride;
    for (const auto& [n, st] : dims) last += (n - 1) * st;
    const uintptr_t lo = reinterpret_cast<uintptr_t>(base);
    return {lo, lo + (uintptr_t)(last + 1) * es};
}

// Whether y shares a byte with anything the single pass without scratch reads
// or writes besides y once its first launch has written state tiles into y:
// x, dt, A, B, C, s1, ids, and s0 (its rows 0 .. n_seq - 1 without ids; with
// ids the rows read are not known to the host and s0 is left out).
bool y_overlaps_others(const helix_scan_desc& d, const void* y, const void* x, const void* dt, const void* A,
                       const void* B, const void* C, const void* s0, const void* ids, const void* s1) {
    const long long T = d.n_tok, S = d.n_seq;
    const ByteRange ry = byte_range(y, S, d.seq_y, {{T, d.s_y[0]}, {d.n_head, d.s_y[1]}, {d.head_dim, d.s_y[2]}}, 4);
    auto state = [&](const void* p) {
        return byte_range(p, S, d.seq_s, {{d.n_head, d.s_s[0]}, {d.head_dim, d.s_s[1]}, {d.d_state, d.s_s[2]}}, 4);
    };
    const ByteRange others[] = {
        byte_range(x, S, d.seq_x, {{T, d.s_x[0]}, {d.n_head, d.s_x[1]}, {d.head_dim, d.s_x[2]}}, 4),
        byte_range(dt, S, d.seq_dt, {{T, d.s_dt[0]}, {d.n_head, d.s_dt[1]}}, 4),
        byte_range(A, 1, 0, {{d.n_head, d.s_a}}, 4),
        byte_range(B, S, d.seq_b, {{T, d.s_b[0]}, {d.n_group, d.s_b[1]}, {d.d_state, d.s_b[2]}}, 4),
        byte_range(C, S, d.seq_c, {{T, d.s_c[0]}, {d.n_group, d.s_c[1]}, {d.d_state, d.s_c[2]}}, 4),
        state(s1),
        ids ? byte_range(ids, S, 1, {}, 4) : state(s0),
    };
    for (const ByteRange& r : others)
        if (ry.overlaps(r)) return true;
    return false;
}

// One launch sequence for d_state <= HELIX_N_MAX, or for one block of state
// indices (inner: d is helix::rt::state_block's descriptor or the single-pass
// form of the caller's, already gated as part of it; y_acc: add into y).
// sel: the kernels d runs on (helix::rt::select_traits for the caller's
// descriptor, select_traits_unblocked for a block or the single-pass form).
// scratch_sized: the scratch is the library's own fixed array, already known
// to hold the plan (helix_scan_encode_noalloc), so its allocation is not
// queried.
// budget_cap: the plan's scratch budget is at most this many bytes (the fixed
// array of helix_scan_encode_noalloc).
// dry: run every check, enqueue nothing.
helix_status encode_one(helix_ctx* ctx, hipStream_t stream, const helix_scan_desc* d,
                        helix_tensor s0, helix_tensor x, helix_tensor dt, helix_tensor A,
                        helix_tensor B, helix_tensor C, helix_tensor ids, helix_tensor y,
                        helix_tensor s1, helix_tensor scratch, bool scratch_sized, size_t budget_cap,
                        bool inner, bool y_acc, bool dry, const HelixMatmulTraits& sel) {
    if (!s0.buf || !x.buf || !dt.buf || !A.buf || !B.buf || !C.buf || !y.buf || !s1.buf) {
        set_error(ctx, "null tensor (s0, x, dt, A, B, C, y and s1 are required)");
        return HELIX_ERR_INVALID_ARG;
    }
    if (!inner && !helix_scan_supported(ctx, d)) {
        set_error(ctx, "descriptor not supported (see helix_ctx_backend_desc)");
        return HELIX_ERR_UNSUPPORTED_SHAPE;
    }
    if (!ctx->module) {
        set_error(ctx, "context has no device (host-only context)");
        return HELIX_ERR_NO_DEVICE;
    }

    HelixScanParams params;
    std::string why;
    if (!helix::rt::build_params(*d, &params, &why)) {
        set_error(ctx, why);
        return HELIX_ERR_INVALID_ARG;
    }
    params.has_ids = ids.buf ? 1 : 0;
    params.y_acc = y_acc ? 1 : 0;

    // 16-bit storage: B and C rows are read as 16-byte runs of eight
    // elements, which needs their bases 4-byte aligned (the gate keeps the
    // strides even).
    if (d->io_dtype != HELIX_F32 &&
        ((reinterpret_cast<uintptr_t>(dptr(B)) | reinterpret_cast<uintptr_t>(dptr(C))) & 3)) {
        set_error(ctx, "B and C must be 4-byte aligned with 16-bit storage");
        return HELIX_ERR_INVALID_ARG;
    }

    const HelixMatmulTraits* trp = &sel;
    auto fn = [&](const char* name) -> hipFunction_t {
        if (!name) return nullptr;
        auto it = ctx->kernels.find(name);
        return it == ctx->kernels.end() ? nullptr : it->second;
    };

    // Single pass (reference dispatch.mm:122-138): no scratch. With fp32
    // storage, scalar A and d_state <= 128 it runs as the fp32 path's three
    // passes with their state tiles in y (plan_ytile; below), where y allows
    // it. Otherwise one launch, one workgroup per (seq, head, 16-channel block
    // of a P slab), the state carried in registers. Diagonal A always takes
    // the one-launch path.
    helix::rt::MultipassPlan yplan;
    bool ytile = false;
    // Not for a block that adds into y (y holds the sum so far); the first
    // block of a single pass may keep its tiles in y, which it then
    // overwrites with its share.
    if (trp->k_single && !y_acc) {
        const HelixMatmulTraits* ytr = nullptr;
        yplan = helix::rt::plan_ytile(ctx, *d, *trp, &ytr);
        ytile = ytr && (reinterpret_cast<uintptr_t>(dptr(y)) & 15) == 0 &&
                !y_overlaps_others(*d, dptr(y), dptr(x), dptr(dt), dptr(A), dptr(B), dptr(C), dptr(s0), dptr(ids),
                                   dptr(s1));
        if (ytile) trp = ytr;
    }
    const HelixMatmulTraits& tr = *trp;
    if (tr.k_single) {
        hipFunction_t f1 = fn(y_acc && tr.k_single_acc ? tr.k_single_acc : tr.k_single);
        if (!f1) {
            set_error(ctx, "kernel not resolved in code object");
            return HELIX_ERR_PIPELINE;
        }
        const long long n_wg = (long long)d->n_seq * d->n_head * params.n_pslab * 4;
        if (n_wg > 0xffffffffLL) {
            set_error(ctx, "launch grid exceeds 2^32 workgroups (n_seq * n_head * n_pslab * 4)");
            return HELIX_ERR_INVALID_ARG;
        }
        params.np = tr.np;
        if (dry) return HELIX_OK;
        HelixScanBuffers bufs;
        std::memset(&bufs, 0, sizeof(bufs));
        bufs.s0  = static_cast<const float*>(dptr(s0));
        bufs.x   = static_cast<const float*>(dptr(x));
        bufs.dt  = static_cast<const float*>(dptr(dt));
        bufs.A   = static_cast<const float*>(dptr(A));
        bufs.B   = static_cast<const float*>(dptr(B));
        bufs.C   = static_cast<const float*>(dptr(C));
        bufs.ids = static_cast<const int*>(dptr(ids));
        bufs.y   = static_cast<float*>(dptr(y));
        bufs.s1  = static_cast<float*>(dptr(s1));
        int prev = -1;
        (void)hipGetDevice(&prev);
        if (prev != ctx->device && hipSetDevice(ctx->device) != hipSuccess) {
            (void)hipGetLastError();
            set_error(ctx, "hipSetDevice failed");
            return HELIX_ERR_NO_DEVICE;
        }
        void* args[] = {&params, &bufs};
        const hipError_t e = hipModuleLaunchKernel(f1, (unsigned)n_wg, 1, 1, (unsigned)tr.single_threads, 1, 1, 0,
                                                   stream, args, nullptr);
        if (prev >= 0 && prev != ctx->device) (void)hipSetDevice(prev);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            set_error(ctx, std::string("kernel launch failed: ") + hipGetErrorString(e));
            return HELIX_ERR_PIPELINE;
        }
        return HELIX_OK;
    }

    const helix::rt::MultipassPlan plan = ytile ? yplan : helix::rt::plan_multipass(ctx, *d, tr, budget_cap);
    if (plan.n_chunks <= 0) {
        set_error(ctx, "empty problem");
        return HELIX_ERR_INVALID_ARG;
    }
    if (plan.total_bytes > 0 && !scratch_sized) {
        if (!scratch.buf) {
            set_error(ctx, "multipass requires a scratch buffer of helix_scan_scratch_size() bytes");
            return HELIX_ERR_SCRATCH_TOO_SMALL;
        }
        // The reference checks the MTLBuffer length (dispatch.mm:150-153);
        // the HIP analogue is the allocation containing the pointer.
        hipDeviceptr_t base = nullptr;
        size_t size = 0;
        void* sp = dptr(scratch);
        if (hipMemGetAddressRange(&base, &size, sp) == hipSuccess) {
            const size_t avail = (size_t)((char*)base + size - (char*)sp);
            if (avail < plan.total_bytes) {
                set_error(ctx, "scratch buffer smaller than helix_scan_scratch_size()");
                return HELIX_ERR_SCRATCH_TOO_SMALL;
            }
        } else {
            (void)hipGetLastError();  // not a hipMalloc allocation: cannot verify, trust the caller
        }
    }

    hipFunction_t fA = fn(tr.k_chunk_state), fB = fn(tr.k_state_scan),
                  fC = fn(y_acc && tr.k_chunk_out_acc ? tr.k_chunk_out_acc : tr.k_chunk_out);
    if (!fA || !fB || !fC) {
        set_error(ctx, "kernel not resolved in code object");
        return HELIX_ERR_PIPELINE;
    }

    // Scratch strides (helix_params.h layout: per head, n_pslab tiles of 64*np).
    const long long HT = (long long)d->n_head * params.n_pslab * 64 * tr.np;
    params.np      = tr.np;
    params.seg_len = plan.seg_len;
    params.walk_len = plan.walk_len;
    params.hblk    = plan.hblk;
    params.n_hblk  = plan.n_hblk;
    params.sl_cg   = HT;
    params.sl_seq  = (long long)plan.chunks_per_group * HT;
    params.sg_seg  = HT;
    params.sg_seq  = (long long)plan.segs_per_group * HT;
    params.ld_seq  = (long long)plan.chunks_per_group * d->n_head;
    params.sd_seq  = (long long)plan.segs_per_group * d->n_head;
    params.cpg     = plan.chunks_per_group;
    // A single-group plan on a walking Pass C that runs Pass B's segment scan
    // itself: no Pass B launch.
    const bool fuse_b = helix::rt::fuse_b_on(ctx, tr, plan);
    params.fuse_b  = fuse_b ? 1 : 0;
    params.ytile   = ytile ? 1 : 0;

    HelixScanBuffers bufs;
    std::memset(&bufs, 0, sizeof(bufs));
    bufs.s0  = static_cast<const float*>(dptr(s0));
    bufs.x   = static_cast<const float*>(dptr(x));
    bufs.dt  = static_cast<const float*>(dptr(dt));
    bufs.A   = static_cast<const float*>(dptr(A));
    bufs.B   = static_cast<const float*>(dptr(B));
    bufs.C   = static_cast<const float*>(dptr(C));
    bufs.ids = static_cast<const int*>(dptr(ids));
    bufs.y   = static_cast<float*>(dptr(y));
    bufs.s1  = static_cast<float*>(dptr(s1));
    if (!ytile) {   // ytile: no scratch; the kernels keep their tiles in y
        char* sc = static_cast<char*>(dptr(scratch));
        bufs.s_local = plan.sl_elems ? sc + plan.off_sl : nullptr;
        bufs.s_seg   = reinterpret_cast<float*>(sc + plan.off_sg);
        bufs.ld      = reinterpret_cast<float*>(sc + plan.off_ld);
        bufs.segld   = reinterpret_cast<float*>(sc + plan.off_sd);
        bufs.bcopy   = plan.bc_elems ? sc + plan.off_bc : nullptr;
        bufs.ccopy   = plan.bc_elems ? sc + plan.off_cc : nullptr;
        bufs.pre     = plan.rec_elems ? reinterpret_cast<float*>(sc + plan.off_rec) : nullptr;
    }

    // Launch sizes of the largest group, checked in 64 bits before anything is
    // enqueued: the kernels decode their 1-D Pass C grid as a 32-bit count.
    const unsigned hpg = (unsigned)(d->n_head / d->n_group);
    const unsigned hpw = tr.walk_hpw > 0 ? (unsigned)tr.walk_hpw : HELIX_WALK_HPW(tr.np);
    const unsigned pairs = (hpg + hpw - 1) / hpw;
    auto pass_c_groups = [&](int n_cg, int n_walk) -> long long {
        return tr.walk ? (long long)n_walk * d->n_group * pairs * params.n_pslab * d->n_seq
                       : (long long)n_cg * d->n_group * plan.n_hblk * d->n_seq;
    };
    // Head-block Pass A: item blocks of HELIX_HB (head, P slab) pairs per group.
    const long long ipg = (long long)hpg * params.n_pslab;
    const long long nib = (ipg + HELIX_HB - 1) / HELIX_HB;
    auto pass_a_groups = [&](int n_seg) -> long long { return (long long)d->n_seq * d->n_group * nib * n_seg; };
    {
        const int n_cg = std::min(plan.chunks_per_group, plan.n_chunks);
        const long long wg_c = pass_c_groups(n_cg, (n_cg + plan.walk_len - 1) / plan.walk_len);
        const long long wg_a = tr.a_hb ? pass_a_groups((n_cg + plan.seg_len - 1) / plan.seg_len) : 0;
        if (wg_c > 0xffffffffLL || wg_a > 0xffffffffLL) {
            set_error(ctx, "launch grid exceeds 2^32 workgroups");
            return HELIX_ERR_INVALID_ARG;
        }
    }
    if (dry) return HELIX_OK;

    // Debug-only per-pass timing split (reference dispatch.mm:207-216):
    // HELIX_ONLY_PASS=A|B|C enqueues just that pass, and a set of letters
    // (AB, AC, BC) just those passes; the output is then meaningless. 'X' (the
    // reference's pad/cast passes) enqueues nothing, because that work is
    // fused into the Pass A/C staging here.
    const char* only = std::getenv("HELIX_ONLY_PASS");
    const bool do_a = !only || std::strchr(only, 'A');
    const bool do_b = !only || std::strchr(only, 'B');
    const bool do_c = !only || std::strchr(only, 'C');

    int prev = -1;
    (void)hipGetDevice(&prev);
    if (prev != ctx->device && hipSetDevice(ctx->device) != hipSuccess) {
        (void)hipGetLastError();
        set_error(ctx, "hipSetDevice failed");
        return HELIX_ERR_NO_DEVICE;
    }

    helix_status st = HELIX_OK;
    const unsigned PN = (unsigned)(params.n_pslab * 16 * tr.np);   // Pass B threads (tile units) per head
    void* args[] = {&params, &bufs};
    for (int base = 0; base < plan.n_chunks && st == HELIX_OK; base += plan.chunks_per_group) {
        params.chunk_base  = base;
        params.n_cg        = std::min(plan.chunks_per_group, plan.n_chunks - base);
        params.n_seg       = (params.n_cg + plan.seg_len - 1) / plan.seg_len;
        params.n_walk      = (params.n_cg + plan.walk_len - 1) / plan.walk_len;
        params.first_group = base == 0 ? 1 : 0;

        hipError_t e = hipSuccess;
        if (do_a && tr.a_hb)
            e = hipModuleLaunchKernel(fA, (unsigned)pass_a_groups(params.n_seg), 1, 1, HELIX_HB_THREADS, 1, 1, 0,
                                      stream, args, nullptr);
        else if (do_a)
            e = hipModuleLaunchKernel(fA, (unsigned)params.n_seg, (unsigned)d->n_head,
                                      (unsigned)(d->n_seq * params.n_pslab), HELIX_WG, 1, 1, 0,
                                      stream, args, nullptr);
        if (e == hipSuccess && do_b && !fuse_b)
            e = hipModuleLaunchKernel(fB, (PN + HELIX_WG - 1) / HELIX_WG, (unsigned)d->n_head,
                                      (unsigned)d->n_seq, HELIX_WG, 1, 1, 0, stream, args, nullptr);
        if (e == hipSuccess && do_c) {
            const unsigned n_wg = (unsigned)pass_c_groups(params.n_cg, params.n_walk);
            const unsigned threads = tr.walk ? HELIX_WG * hpw : HELIX_WG;
            // With bf16 copies, Pass C reads B and C from them: dense
            // [seq][t][group][n] rows counted from the group's first token.
            // The base is moved back by that token so that the kernel's
            // absolute row t0 lands on the group's row t0 - 64 base.
            HelixScanParams pc = params;
            HelixScanBuffers bc = bufs;
            if (tr.bccopy) {
                const long long gn = (long long)d->n_group * d->d_state;
                for (long long* s3 : {pc.s_b, pc.s_c}) {
                    s3[0] = gn;
                    s3[1] = d->d_state;
                    s3[2] = 1;
                }
                pc.seq_b = pc.seq_c = (long long)plan.chunks_per_group * HELIX_CS * gn;
                const uintptr_t back = (uintptr_t)((long long)base * HELIX_CS * gn * 2);
                bc.B = reinterpret_cast<const float*>(reinterpret_cast<uintptr_t>(bufs.bcopy) - back);
                bc.C = reinterpret_cast<const float*>(reinterpret_cast<uintptr_t>(bufs.ccopy) - back);
            }
            void* args_c[] = {&pc, &bc};
            e = hipModuleLaunchKernel(fC, n_wg, 1, 1, threads, 1, 1, 0, stream, args_c, nullptr);
        }
        if (e != hipSuccess) {
            // Every argument and limit was checked above, so a launch failure
            // here comes from the runtime itself. Groups launched before the
            // failing one stay enqueued: a multi-group encode is not atomic.
            (void)hipGetLastError();
            set_error(ctx, std::string("kernel launch failed: ") + hipGetErrorString(e));
            st = HELIX_ERR_PIPELINE;
        }
    }
    if (prev >= 0 && prev != ctx->device) (void)hipSetDevice(prev);
    return st;
}

// The encoder behind every entry point. d_state above HELIX_N_MAX runs as
// helix::rt::n_state_blocks blocks of state indices in stream order, block k
// reading B, C and s0 and writing s1 at its first state index n0 and adding
// its share of y into y; every block is checked before the first is
// enqueued. y then must not overlap an input: a later block would read what
// an earlier one wrote.
helix_status encode_core(helix_ctx* ctx, hipStream_t stream, const helix_scan_desc* d,
                         helix_tensor s0, helix_tensor x, helix_tensor dt, helix_tensor A,
                         helix_tensor B, helix_tensor C, helix_tensor ids, helix_tensor y,
                         helix_tensor s1, helix_tensor scratch, bool scratch_sized = false,
                         size_t budget_cap = SIZE_MAX) {
    const int nb = helix::rt::n_state_blocks(ctx, *d);
    if (nb == 1)
        return encode_one(ctx, stream, d, s0, x, dt, A, B, C, ids, y, s1, scratch, scratch_sized, budget_cap,
                          /*inner=*/false, /*y_acc=*/false, /*dry=*/false, helix::rt::select_traits(ctx, *d));
    // Up to HELIX_N_MAX blocks are a choice: where y overlaps an input (in
    // place over x, say) d runs as the one-launch single pass instead, which
    // reads each chunk of x before it writes that chunk's y and needs no
    // scratch (helix_scan_scratch_size sizes the blocks' plan only).
    const bool overlap = y_overlaps_others(*d, dptr(y), dptr(x), dptr(dt), dptr(A), dptr(B), dptr(C), dptr(s0),
                                           dptr(ids), dptr(s1));
    if (overlap && d->d_state <= HELIX_N_MAX) {
        if (!helix_scan_supported(ctx, d)) {
            set_error(ctx, "descriptor not supported (see helix_ctx_backend_desc)");
            return HELIX_ERR_UNSUPPORTED_SHAPE;
        }
        helix_scan_desc one = *d;
        one.multipass = false;
        one.backend = HELIX_BACKEND_SGMMA;
        return encode_one(ctx, stream, &one, s0, x, dt, A, B, C, ids, y, s1, scratch, scratch_sized, budget_cap,
                          /*inner=*/true, /*y_acc=*/false, /*dry=*/false,
                          helix::rt::select_traits_unblocked(ctx, one));
    }
    if (!s0.buf || !x.buf || !dt.buf || !A.buf || !B.buf || !C.buf || !y.buf || !s1.buf) {
        set_error(ctx, "null tensor (s0, x, dt, A, B, C, y and s1 are required)");
        return HELIX_ERR_INVALID_ARG;
    }
    if (!helix_scan_supported(ctx, d)) {
        set_error(ctx, "descriptor not supported (see helix_ctx_backend_desc)");
        return HELIX_ERR_UNSUPPORTED_SHAPE;
    }
    if (overlap) {
        set_error(ctx, "y overlaps an input or s1; with d_state above " + std::to_string(HELIX_N_MAX) +
                           " y accumulates over blocks of state indices and must be a buffer of its own");
        return HELIX_ERR_INVALID_ARG;
    }
    for (int pass = 0; pass < 2; ++pass) {   // pass 0 checks every block, pass 1 enqueues them
        for (int k = 0; k < nb; ++k) {
            int n0 = 0;
            const helix_scan_desc sub = helix::rt::state_block(ctx, *d, k, &n0);
            auto at_n0 = [n0](helix_tensor t) {
                if (t.buf) t.offset += (uint64_t)n0 * sizeof(float);
                return t;
            };
            const helix_status st = encode_one(ctx, stream, &sub, at_n0(s0), x, dt, A, at_n0(B), at_n0(C), ids, y,
                                               at_n0(s1), scratch, scratch_sized, budget_cap, /*inner=*/true,
                                               /*y_acc=*/k > 0, /*dry=*/pass == 0,
                                               helix::rt::select_traits_unblocked(ctx, sub, /*block=*/true));
            if (st != HELIX_OK) return st;
        }
    }
    return HELIX_OK;
}

}  // namespace

extern "C" helix_status helix_scan_encode(helix_ctx* ctx, void* cmd_buffer, const helix_scan_desc* d,
                                          helix_tensor s0, helix_tensor x, helix_tensor dt,
                                          helix_tensor A, helix_tensor B, helix_tensor C,
                                          helix_tensor ids, helix_tensor y, helix_tensor s1,
                                          helix_tensor scratch) {
    if (!ctx || !d) return HELIX_ERR_INVALID_ARG;
    return encode_core(ctx, static_cast<hipStream_t>(cmd_buffer), d, s0, x, dt, A, B, C, ids, y, s1,
                       scratch);
}

extern "C" helix_status helix_scan_encode_into(helix_ctx* ctx, void* encoder, const helix_scan_desc* d,
                                               helix_tensor s0, helix_tensor x, helix_tensor dt,
                                               helix_tensor A, helix_tensor B, helix_tensor C,
                                               helix_tensor ids, helix_tensor y, helix_tensor s1,
                                               helix_tensor scratch) {
    if (!ctx || !d) return HELIX_ERR_INVALID_ARG;
    return encode_core(ctx, static_cast<hipStream_t>(encoder), d, s0, x, dt, A, B, C, ids, y, s1,
                       scratch);
}

namespace {

// Scratch of the plan helix_scan_encode_noalloc runs (0 for the single pass).
size_t noalloc_scratch_size(helix_ctx* ctx, const helix_scan_desc* d) {
    if (!d->multipass) return 0;
    const HelixMatmulTraits& tr = helix::rt::select_traits(ctx, *d);
    if (tr.k_single) return 0;
    return helix::rt::plan_multipass(ctx, helix::rt::plan_desc(ctx, *d), tr, HELIX_NOALLOC_SCRATCH_BYTES).total_bytes;
}

}  // namespace

extern "C" helix_status helix_scan_encode_noalloc(helix_ctx* ctx, void* stream, const helix_scan_desc* d,
                                                  helix_tensor s0, helix_tensor x, helix_tensor dt,
                                                  helix_tensor A, helix_tensor B, helix_tensor C,
                                                  helix_tensor ids, helix_tensor y, helix_tensor s1) {
    if (!ctx || !d) return HELIX_ERR_INVALID_ARG;
    if (!helix_scan_supported(ctx, d)) {
        set_error(ctx, "descriptor not supported (see helix_ctx_backend_desc)");
        return HELIX_ERR_UNSUPPORTED_SHAPE;
    }
    // Planned for the fixed array: a plan that would exceed it is cut into
    // more super-chunk groups (carried through s1), as with a lower
    // HELIX_SCRATCH_MB; only a plan that does not fit even at one chunk per
    // group is refused.
    const size_t need = noalloc_scratch_size(ctx, d);
    if (need > HELIX_NOALLOC_SCRATCH_BYTES) {
        set_error(ctx, "plan needs " + std::to_string(need) + " bytes of scratch at one chunk per group, more than the " +
                           std::to_string((size_t)HELIX_NOALLOC_SCRATCH_BYTES) +
                           " of the fixed scratch (HELIX_NOALLOC_SCRATCH_BYTES); use helix_scan_encode");
        return HELIX_ERR_SCRATCH_TOO_SMALL;
    }
    helix_tensor scratch = HELIX_TENSOR_NULL;
    if (need > 0) {
        if (!ctx->module) {
            set_error(ctx, "context has no device (host-only context)");
            return HELIX_ERR_NO_DEVICE;
        }
        std::string why;
        scratch.buf = helix::rt::noalloc_scratch(ctx->device, &why);
        if (!scratch.buf) {
            set_error(ctx, why);
            return HELIX_ERR_NO_DEVICE;
        }
    }
    return encode_core(ctx, static_cast<hipStream_t>(stream), d, s0, x, dt, A, B, C, ids, y, s1, scratch,
                       /*scratch_sized=*/true, HELIX_NOALLOC_SCRATCH_BYTES);
}

extern "C" helix_status helix_scan_plan_info(helix_ctx* ctx, const helix_scan_desc* d,
                                             helix_plan_info* out) {
    if (!ctx || !d || !out) return HELIX_ERR_INVALID_ARG;
    if (!helix_scan_supported(ctx, d)) return HELIX_ERR_UNSUPPORTED_SHAPE;
    const HelixMatmulTraits& tr = helix::rt::select_traits(ctx, *d);
    std::memset(out, 0, sizeof(*out));
    // Above HELIX_N_MAX: the plan of one block (the largest), run once per
    // block; the blocks add into y, so the single pass keeps no tiles there.
    const int nb = helix::rt::n_state_blocks(ctx, *d);
    const helix_scan_desc pd = helix::rt::plan_desc(ctx, *d);
    out->state_blocks = nb;
    const HelixMatmulTraits* ytr = nullptr;
    const helix::rt::MultipassPlan yplan =
        tr.k_single ? helix::rt::plan_ytile(ctx, pd, tr, &ytr) : helix::rt::MultipassPlan{};
    if (tr.k_single && !ytr) {
        out->n_chunks = (d->n_tok + HELIX_CS - 1) / HELIX_CS;
        out->chunks_per_group = out->n_chunks;
        out->n_groups = 1;
        out->seg_len = out->n_chunks;
        out->segs_per_group = 1;
        out->walk_len = out->n_chunks;
        out->walks_per_group = 1;
        out->hblk = 1;
        out->n_hblk = d->n_head / d->n_group;
        out->launches = nb;
        out->np = tr.np;
        out->kernel_1pass = tr.k_single;
        return HELIX_OK;
    }
    // The single pass with its state tiles in y: the fp32 path's passes, no
    // scratch (the one-launch kernel stays named as the encoder's fallback).
    if (ytr) {
        out->state_in_y = 1;
        out->kernel_1pass = tr.k_single;
    }
    const HelixMatmulTraits& tp = ytr ? *ytr : tr;
    const helix::rt::MultipassPlan pl = ytr ? yplan : helix::rt::plan_multipass(ctx, pd, tr);
    out->n_chunks = pl.n_chunks;
    out->chunks_per_group = pl.chunks_per_group;
    out->n_groups = pl.n_groups;
    out->seg_len = pl.seg_len;
    out->segs_per_group = pl.segs_per_group;
    out->walk_len = pl.walk_len;
    out->walks_per_group = pl.walks_per_group;
    out->hblk = pl.hblk;
    out->n_hblk = pl.n_hblk;
    out->bf16_state = tp.bf16_state ? 1 : 0;
    out->total_bytes = pl.total_bytes;
    if (!ytr) {   // state_in_y: every region lies in y
        out->s_local_bytes = pl.sl_elems * pl.sl_elem_bytes;
        out->s_seg_bytes = pl.sg_elems * sizeof(float);
        out->bccopy_bytes = pl.bc_elems * 2 * 2;
        out->rec_bytes = pl.rec_elems * sizeof(float);
    }
    const bool fuse_b = helix::rt::fuse_b_on(ctx, tp, pl);   // as helix_scan_encode decides
    // With blocks of state indices a single pass keeps tiles in y for its
    // first block only; the others run kernel_1pass.
    out->launches = ytr ? (fuse_b ? 2 : 3) + (nb - 1) : (fuse_b ? 2 : 3 * pl.n_groups) * nb;
    out->np = tp.np;
    out->kernel_a = tp.k_chunk_state;
    out->kernel_b = fuse_b ? nullptr : tp.k_state_scan;
    out->kernel_c = tp.k_chunk_out;
    out->pass_b = fuse_b ? HELIX_PASS_B_IN_C : HELIX_PASS_B_LAUNCHED;
    return HELIX_OK;
}
