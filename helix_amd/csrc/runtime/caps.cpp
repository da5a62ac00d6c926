// caps.cpp -- shape gate, backend selection, scratch planning, params packing.
//
// Counterpart of the reference's src/runtime/caps.mm:1-306. The contract is
// the same: helix_scan_supported() == false means the caller keeps its own
// kernel, selection never fails, and helix_scan_scratch_size() agrees exactly
// with what the encoder lays out. Everything here is plain C++ and runs
// without a GPU (ctx may be a host-only context or null for planning).
#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <mutex>
#include <tuple>
#include <string>
#include <vector>

#include "helix_internal.h"

namespace {

// Kernel families (helix_amd/csrc/kernels). d_state is padded to np = 64, 128
// or 256 and every family is instantiated at each np it serves.
//
//   Pass A runs the head-block kernels (pass_a_hb.hip: B split once per
//   workgroup of four items, helix_chunk_state_hb_*) up to d_state 128 and the
//   per-item kernels (pass_a_x6.hip, helix_chunk_state_x*) at d_state 256.
//   fp32 path (SGMMA, or HELIX_FORCE_BACKEND=s..., multipass, fp32 storage):
//     Pass A helix_chunk_state{_hb}_x6f32_n*  bf16x6 split products, stores
//                                        the per-chunk prefix states R_c (fp32)
//                                        and fp64 decay records
//     Pass B helix_state_scan_f32
//     Pass C helix_chunk_out_x6_n{64,128}  bf16x6 split products
//            helix_chunk_out_f32_n256      fp32 MFMA (the bf16x6 planes of a
//                                          d_state 256 tile exceed the LDS)
//   fp32 path at d_state <= 128 (fp32 storage): Pass C walks each segment's
//   chunks on bf16x6 products with the state in registers, so Pass A stores no
//   per-chunk states (HELIX_F32_WALK=0 keeps the chunk-parallel Pass C):
//     Pass A helix_chunk_state_hb_x6agg_r64_n{64,128}  segment aggregates,
//                                                      fp64 decay records
//     Pass B helix_state_scan_f32 (or the walk's prologue, fuse_b)
//     Pass C helix_scan_walk_x6_n{64,128}
//   bf16 path (AUTO or MPP, multipass): Pass C walks each segment's chunks on
//   bf16 MFMA with the state in registers; Pass A computes the segment
//   aggregates only, fp32-accurate (the reference's contract for the carried
//   state): up to d_state 128 on three products of scaled fp16 planes
//   (helix_chunk_state_hb_h3agg_{,bc_,bf16io_,f16io_}n*; HELIX_PASSA_F16=0
//   keeps six bf16 split products), otherwise on six bf16 split products, or,
//   opted into with HELIX_PASSA_SPLIT=3, on three.
//     Pass A helix_chunk_state{_hb}_x{6,3}agg_n*     fp32 storage
//            helix_chunk_state{_hb}_x{6,3}agg_bc_n*  ... also writes bf16 copies
//                                                    of B and C for the walk
//            helix_chunk_state{_hb}_x{6,3}agg_{bf16,f16}io_n*   16-bit storage
//     Pass B helix_state_scan_f32 (or the walk's prologue, fuse_b)
//     Pass C helix_scan_walk16_bf16{,_bc,_bf16io,_f16io}_n*
//   single pass (multipass = false): helix_scan_1pass_{f32,bf16io,f16io}_n*, no
//   scratch; fp32-accurate (bf16x6 products with fp32 storage up to d_state
//   128, fp32 MFMA otherwise); diagonal A: helix_scan_1pass_diag_f32_n{64,128}.

constexpr int kNps[3] = {64, 128, 256};

int np_index(int d_state) {
    if (d_state <= 64) return 0;
    if (d_state <= 128) return 1;
    return 2;
}

const char* const kIoTag[3] = {"", "bf16io_", "f16io_"};   // fp32, bf16, f16 storage

int io_index(helix_dtype io) { return io == HELIX_BF16 ? 1 : io == HELIX_F16 ? 2 : 0; }

// Traits are composed from these choices, once per process; the names live as
// long as the process.
struct TraitTable {
    // [io][k]: single pass; [k]: diagonal A; [k]: fp32 path; [k]: the fp32
    // path's walk (d_state <= 128); [io][split6][bccopy][k]: bf16 path (bccopy
    // only with fp32 storage).
    HelixMatmulTraits single[3][3], diag[2], f32[3], f32walk[2], bf16[3][2][2][3], ysingle[2];
    // [io][bccopy][k]: bf16 path with Pass A on scaled fp16 planes (d_state
    // <= 128; bccopy only with fp32 storage).
    HelixMatmulTraits h3[3][2][2];
    std::vector<std::string> names;   // every kernel name, deduplicated
    std::deque<std::string> store;    // backing storage of the strings above

    const char* keep(const std::string& v) {
        store.push_back(v);
        return store.back().c_str();
    }
    const char* kernel(const std::string& v) {
        for (const std::string& n : names)
            if (n == v) return keep(v);
        names.push_back(v);
        return keep(v);
    }

    TraitTable() {
        for (int k = 0; k < 3; ++k) {
            const std::string np = std::to_string(kNps[k]);
            const std::string upto = " (d_state<=" + np + ")";
            for (int io = 0; io < 3; ++io) {
                HelixMatmulTraits& t = single[io][k];
                t = HelixMatmulTraits{};
                t.backend = HELIX_BACKEND_SGMMA;
                t.name = keep(std::string("mfma fp32, single pass") +
                              (io == 0 ? "" : io == 1 ? ", bf16 storage" : ", f16 storage") + upto);
                // fp32 storage up to d_state 128: every product on six bf16
                // split products (pass_single.hip, X6); otherwise fp32 MFMA.
                t.mfma_a = t.mfma_c = io == 0 && kNps[k] <= 128 ? "v_mfma_f32_16x16x32_bf16 (bf16x6 split operands)"
                                                                : "v_mfma_f32_16x16x4_f32";
                t.np = kNps[k];
                t.k_single = kernel(std::string("helix_scan_1pass_") + (io == 0 ? "f32_" : kIoTag[io]) + "n" + np);
                if (io == 0 && kNps[k] <= HELIX_N_BLOCK) t.k_single_acc = kernel("helix_scan_1pass_f32_acc_n" + np);
                t.single_threads = 64 * HELIX_1PASS_WAVES(kNps[k]);
            }
            if (k < 2) {
                // The single pass (fp32 storage, scalar A) run as the three
                // passes with its state tiles in y: Pass A's aggregate kernel
                // (no records), Pass B, and the fp32 path's walk forming its
                // own decay preamble.
                HelixMatmulTraits& t = ysingle[k];
                t = HelixMatmulTraits{};
                t.backend = HELIX_BACKEND_SGMMA;
                t.name = keep("mfma fp32, single pass as three launches, state tiles in y" + upto);
                t.k_chunk_state = kernel("helix_chunk_state_hb_x6agg_n" + np);
                t.k_state_scan = kernel("helix_state_scan_y_f32");
                t.k_chunk_out = kernel("helix_scan_walk_x6_y_n" + np);
                t.mfma_a = "v_mfma_f32_32x32x16_bf16 (bf16x6 split operands)";
                t.mfma_c = "v_mfma_f32_16x16x32_bf16 (bf16x6 split operands)";
                t.np = kNps[k];
                t.walk = true;
                t.walk_hpw = 2;
                t.a_hb = true;
            }
            if (k < 2) {
                HelixMatmulTraits& t = diag[k];
                t = HelixMatmulTraits{};
                t.backend = HELIX_BACKEND_SGMMA;
                t.name = keep("mfma fp32, single pass, diagonal A" + upto);
                t.mfma_a = t.mfma_c = "v_mfma_f32_16x16x4_f32";
                t.np = kNps[k];
                t.k_single = kernel("helix_scan_1pass_diag_f32_n" + np);
                t.single_threads = HELIX_WG;
            }
            {
                HelixMatmulTraits& t = f32[k];
                t = HelixMatmulTraits{};
                t.backend = HELIX_BACKEND_SGMMA;
                const bool x6c = kNps[k] <= 128;
                t.name = keep(std::string(x6c ? "mfma fp32, passes A and C bf16x6" : "mfma fp32, pass A bf16x6") +
                              upto);
                t.k_chunk_state = kernel(std::string(kNps[k] <= 128 ? "helix_chunk_state_hb_x6f32_n"
                                                                    : "helix_chunk_state_x6f32_n") + np);
                t.a_hb = kNps[k] <= 128;
                t.k_state_scan = kernel("helix_state_scan_f32");
                t.k_chunk_out = kernel(x6c ? "helix_chunk_out_x6_n" + np : "helix_chunk_out_f32_n" + np);
                t.mfma_a = "v_mfma_f32_32x32x16_bf16 (bf16x6 split operands)";
                t.mfma_c = x6c ? "v_mfma_f32_32x32x16_bf16 (bf16x6 split operands)" : "v_mfma_f32_32x32x2_f32";
                t.np = kNps[k];
                t.rec_kind = x6c ? 2 : 0;
            }
            if (k < 2) {
                HelixMatmulTraits& t = f32walk[k];
                t = f32[k];
                t.name = keep("mfma fp32, passes A and C bf16x6, chunk walk" + upto);
                t.k_chunk_state = kernel("helix_chunk_state_hb_x6agg_r64_n" + np);
                t.k_chunk_out = kernel("helix_scan_walk_x6_n" + np);
                t.k_chunk_out_acc = kernel("helix_scan_walk_x6_acc_n" + np);
                t.mfma_c = "v_mfma_f32_16x16x32_bf16 (bf16x6 split operands)";
                t.walk = true;
                t.walk_hpw = 2;
                t.walk_fuse_b = true;
                t.rec_kind = 2;
            }
            for (int io = 0; io < 3; ++io)
                for (int s6 = 0; s6 < 2; ++s6)
                    for (int bc = 0; bc < 2; ++bc) {
                        HelixMatmulTraits& t = bf16[io][s6][bc][k];
                        t = HelixMatmulTraits{};
                        if (bc && io) continue;   // copies only from fp32 storage
                        t.backend = HELIX_BACKEND_MPP;
                        const char* split = s6 ? "x6" : "x3";
                        t.name = keep(std::string("mfma bf16 pass C, chunk walk, pass A ") +
                                      (s6 ? "bf16x6" : "bf16x3 (narrower state: opt-in)") +
                                      (io == 1 ? ", bf16 storage" : io == 2 ? ", f16 storage" : "") + upto);
                        const bool hb = kNps[k] <= 128;
                        t.k_chunk_state = kernel(std::string(hb ? "helix_chunk_state_hb_" : "helix_chunk_state_") +
                                                 split + "agg_" + (bc ? "bc_" : kIoTag[io]) + "n" + np);
                        t.a_hb = hb;
                        t.k_state_scan = kernel("helix_state_scan_f32");
                        t.k_chunk_out = kernel(std::string("helix_scan_walk16_bf16_") + (bc ? "bc_" : kIoTag[io]) +
                                               "n" + np);
                        if (io == 0 && kNps[k] <= HELIX_N_BLOCK)
                            t.k_chunk_out_acc = kernel(std::string("helix_scan_walk16_bf16_") + (bc ? "bc_" : "") +
                                                       "acc_n" + np);
                        t.bf16_state = true;
                        t.mfma_a = s6 ? "v_mfma_f32_32x32x16_bf16 (bf16x6 split operands)"
                                      : "v_mfma_f32_32x32x16_bf16 (bf16x3 split operands)";
                        t.mfma_c = "v_mfma_f32_16x16x32_bf16";
                        t.np = kNps[k];
                        t.walk = true;
                        t.walk_hpw = HELIX_WALK16_HPW(kNps[k]);
                        t.walk_fuse_b = true;
                        t.bccopy = bc != 0;
                        t.rec_kind = 1;
                    }
        }
        for (int io = 0; io < 3; ++io)
            for (int k = 0; k < 2; ++k)
                for (int bc = 0; bc < 2; ++bc) {
                    HelixMatmulTraits& t = h3[io][bc][k];
                    t = bf16[io][1][bc][k];
                    if (!t.name) continue;   // copies only from fp32 storage
                    const std::string np = std::to_string(kNps[k]);
                    t.name = keep(std::string("mfma bf16 pass C, chunk walk, pass A fp16x3 (scaled planes)") +
                                  (io == 1 ? ", bf16 storage" : io == 2 ? ", f16 storage" : "") + " (d_state<=" + np + ")");
                    t.k_chunk_state = kernel(std::string("helix_chunk_state_hb_h3agg_") + (bc ? "bc_" : kIoTag[io]) + "n" + np);
                    t.mfma_a = io ? "v_mfma_f32_32x32x16_f16 (one scaled fp16 plane of B, two of x: two products)"
                                  : "v_mfma_f32_32x32x16_f16 (two scaled fp16 planes, three products)";
                }
        // What helix_ctx_backend_desc reports for a descriptor run as blocks
        // of state indices on these kernels.
        auto blocks_name = [&](HelixMatmulTraits& t) {
            if (t.name) t.name_blocks = keep(std::string(t.name) + ", in blocks of at most " +
                                             std::to_string(HELIX_N_BLOCK) + " state indices");
        };
        for (auto& a : single) for (auto& t : a) blocks_name(t);
        for (auto& t : f32) blocks_name(t);
        for (auto& t : f32walk) blocks_name(t);
        for (auto& t : ysingle) blocks_name(t);
        for (auto& t : diag) blocks_name(t);
        for (auto& a : bf16) for (auto& b2 : a) for (auto& c2 : b2) for (auto& t : c2) blocks_name(t);
        for (auto& a : h3) for (auto& b2 : a) for (auto& t : b2) blocks_name(t);
    }
};

const TraitTable& table() {
    static const TraitTable t;
    return t;
}

// Pass A writes bf16 copies of B and C for the walking Pass C (fp32 storage);
// HELIX_WALK_BCCOPY=0 / 1 switches them off / on where the kernels can. At
// d_state 256 the per-item Pass A copies when the K = heads_per_group *
// n_pslab workgroups of a chunk cover its 64 rows with two quads of four state
// indices per thread (pass_a_x6.hip, copy_map). block: d is one block of
// state indices of a larger d_state.
bool bccopy_on(const helix_tuning& tu, const helix_scan_desc& d, bool block) {
    if (tu.bccopy == 0) return false;
    const long K = (long)(d.n_head / d.n_group) * ((d.head_dim + HELIX_HD - 1) / HELIX_HD);
    // The head-block Pass A (d_state <= 128) can copy at every shape (one
    // wave per 8-token block of a chunk and group, pass_a_hb.hip). The copies
    // pay off when many walk workgroups read a chunk's rows (measured at
    // configs 4a and 4b, 80 and 27 heads per group: 45 and 56 us faster);
    // at 8 (config 2) the walk reading the fp32 rows itself is 3 us faster.
    // Blocks of state indices: at config 2's shape with d_state 256 in two
    // blocks of 128, the walks reading their columns of the caller's rows took
    // 81 and 103 us, on the copies 69 and 79 us, for 15 us more per Pass A
    // (0.279 against 0.273 ms a scan; 9 us and 0.297 against 0.280 ms with
    // the six-product Pass A).
    if (d.d_state <= 128) return tu.bccopy == 1 || K > 8 || block;
    return (64 + K - 1) / K * (d.d_state / 4) <= 2 * 256;
}

const helix_tuning kDefaultTuning{};

const helix_tuning& tuning_of(const helix_ctx* ctx) { return ctx ? ctx->tuning : kDefaultTuning; }

// Workgroup counts the planner aims for: 256 CUs with a few resident
// workgroups each, so a launch fills the chip with a short tail.
constexpr long kTargetWgA = 512;
constexpr long kTargetWgC = 1024;

long env_long(const char* name, long dflt) {
    if (const char* v = std::getenv(name)) {
        char* end = nullptr;
        const long x = std::strtol(v, &end, 10);
        if (end != v && x > 0) return x;
    }
    return dflt;
}

int env_switch(const char* name) {   // -1 unset, else the first digit
    const char* v = std::getenv(name);
    if (!v || v[0] < '0' || v[0] > '9') return -1;
    return v[0] - '0';
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

thread_local std::string t_last_error;
thread_local const helix_ctx* t_last_ctx = nullptr;

}  // namespace

namespace helix::rt {

helix_tuning tuning_from_env() {
    helix_tuning t;
    t.scratch_mb = env_long("HELIX_SCRATCH_MB", t.scratch_mb);
    if (const char* f = std::getenv("HELIX_FORCE_BACKEND")) t.force_fp32 = f[0] == 's' || f[0] == 'S';
    if (env_switch("HELIX_PASSA_SPLIT") == 3) t.passa_split = 3;
    t.fuse_b = env_switch("HELIX_FUSE_B");
    const int f16 = env_switch("HELIX_PASSA_F16");
    if (f16 >= 0) t.passa_f16 = f16 > 0 ? 1 : 0;
    if (t.fuse_b > 1) t.fuse_b = 1;
    const int bc = env_switch("HELIX_WALK_BCCOPY");
    t.bccopy = bc == 0 ? 0 : bc > 0 ? 1 : -1;
    t.seg_len = (int)env_long("HELIX_SEG_LEN", 0);
    t.walk_len = (int)env_long("HELIX_WALK_LEN", 0);
    t.hblk = (int)env_long("HELIX_HBLK", 0);
    const int fw = env_switch("HELIX_F32_WALK");
    if (fw >= 0) t.f32_walk = fw > 0 ? 1 : 0;
    const int yt = env_switch("HELIX_1PASS_Y");
    if (yt >= 0) t.ytile = yt > 0 ? 1 : 0;
    const int sb = env_switch("HELIX_STATE_BLOCKS");
    if (sb >= 0) t.state_blocks = sb > 0 ? 1 : 0;
    return t;
}

const char* const* all_kernel_names(size_t* count) {
    static const std::vector<const char*> ptrs = [] {
        std::vector<const char*> v;
        for (const std::string& n : table().names) v.push_back(n.c_str());
        return v;
    }();
    *count = ptrs.size();
    return ptrs.data();
}

void set_error(const helix_ctx* ctx, const std::string& msg) {
    t_last_ctx = ctx;
    t_last_error = msg;
}

namespace {
int choose_walk_len(const helix_scan_desc& d, int cpg);
}

namespace {
bool state_blocks_on(const helix_ctx* ctx, const helix_scan_desc& d) {
    if (d.d_state > HELIX_N_MAX) return true;   // the gate admits fp32 storage and scalar A only
    if (d.d_state <= HELIX_N_BLOCK || d.io_dtype != HELIX_F32 || d.a_form != HELIX_A_SCALAR_PER_HEAD)
        return false;
    // Measured at L=8192 H=64 P=64 G=8, d_state 160, 192 and 256: blocks of
    // 128 and less took 0.28-0.30 ms against 0.39-0.41 on the bf16 path, and
    // 0.54-0.55 against 0.71-0.72 on the fp32 path (the d_state 256 kernels
    // are the per-item Pass A and, on the fp32 path, an fp32-MFMA Pass C).
    return tuning_of(ctx).state_blocks != 0;
}
}  // namespace

int n_state_blocks(const helix_ctx* ctx, const helix_scan_desc& d) {
    if (!state_blocks_on(ctx, d)) return 1;
    const int nb0 = (d.d_state + HELIX_N_BLOCK - 1) / HELIX_N_BLOCK;
    const int base = ((d.d_state + nb0 - 1) / nb0 + 7) / 8 * 8;   // <= HELIX_N_BLOCK
    return (d.d_state + base - 1) / base;
}

helix_scan_desc state_block(const helix_ctx* ctx, const helix_scan_desc& d, int k, int* n0) {
    helix_scan_desc b = d;
    const int nb = n_state_blocks(ctx, d);
    if (nb > 1) {
        const int base = ((d.d_state + nb - 1) / nb + 7) / 8 * 8;
        b.d_state = std::min(base, d.d_state - k * base);
        if (d.d_state > HELIX_N_MAX) b.backend = HELIX_BACKEND_SGMMA;
        if (n0) *n0 = k * base;
    } else if (n0) {
        *n0 = 0;
    }
    return b;
}

helix_scan_desc plan_desc(const helix_ctx* ctx, const helix_scan_desc& d) { return state_block(ctx, d, 0, nullptr); }

const HelixMatmulTraits& select_traits(const helix_ctx* ctx, const helix_scan_desc& d) {
    // Blocks of state indices: the kernels of their blocks.
    if (n_state_blocks(ctx, d) > 1) return select_traits_unblocked(ctx, plan_desc(ctx, d), /*block=*/true);
    return select_traits_unblocked(ctx, d);
}

const HelixMatmulTraits& select_traits_unblocked(const helix_ctx* ctx, const helix_scan_desc& d, bool block) {
    const helix_tuning& tu = tuning_of(ctx);
    const TraitTable& tt = table();
    const int k = np_index(d.d_state);
    if (d.a_form == HELIX_A_DIAG_PER_CHANNEL) return tt.diag[k < 1 ? k : 1];
    const int io = io_index(d.io_dtype);
    if (!d.multipass) return tt.single[io][k];
    // HELIX_FORCE_BACKEND=s... pins the fp32 path (reference caps.mm:82-86).
    const bool bf16 = (d.backend == HELIX_BACKEND_AUTO || d.backend == HELIX_BACKEND_MPP) && !tu.force_fp32;
    if (!bf16) {
        if (io) return tt.single[io][k];
        // A walk of one chunk carries no state between chunks: where the plan
        // gives one-chunk walks (short sequences of few heads), the
        // chunk-parallel Pass C is the faster form (config 0: 23.0 against
        // 24.0 us). HELIX_F32_WALK=0 / 1 pins either form.
        const bool walk = k < 2 && (tu.f32_walk == 1 ||
                                    (tu.f32_walk < 0 && choose_walk_len(d, (d.n_tok + HELIX_CS - 1) / HELIX_CS) > 1));
        return walk ? tt.f32walk[k] : tt.f32[k];
    }
    const int bc = io == 0 && bccopy_on(tu, d, block) ? 1 : 0;
    // Pass A on two scaled fp16 planes (three products) by default up to
    // d_state 128: config 2, 0.110 against 0.117 ms on six bf16 split
    // products, s1 at the same fp32 per-element bound; HELIX_PASSA_F16=0
    // keeps the six.
    if (k < 2 && tu.passa_split != 3 && tu.passa_f16 != 0) return tt.h3[io][bc][k];
    return tt.bf16[io][tu.passa_split == 3 ? 0 : 1][bc][k];
}

// The walk's prologue loads up to segs_per_group segment aggregates per
// workgroup, four at a time; past four segments the second round of loads
// costs more than Pass B's own launch (config 2, 8 segments: 149 vs 142 us;
// configs 4a/4b, 4 segments, fused against launched: 624 vs 635 and 668 vs
// 681 us).
constexpr int kFuseBMaxSegs = 4;

bool fuse_b_on(const helix_ctx* ctx, const HelixMatmulTraits& tr, const MultipassPlan& plan) {
    // The walk's prologue scans whole walk segments: only when they are Pass
    // A's segments too.
    if (!tr.walk_fuse_b || plan.n_groups != 1 || plan.walk_len != plan.seg_len) return false;
    const helix_tuning& tu = tuning_of(ctx);
    if (tu.fuse_b >= 0) return tu.fuse_b == 1;
    return plan.segs_per_group <= kFuseBMaxSegs;
}

namespace {

// Chunks per walk segment for a group of `cpg` chunks (the walking Pass C;
// also Pass A's segment on the per-item kernels): enough segments that there
// are ~kTargetWgA (seq, head, P slab) items x segments, and no more (a longer
// walk keeps more of the chunk recurrence in registers and shortens Pass B), up
// to kMaxSegLen (past that the walks get too long to fill the chip: at config
// 4a, 64-chunk segments took 1.03 ms and 16-chunk ones 0.95 ms).
constexpr long kMaxSegLen = 16;
// The head-block Pass A runs one 512-thread workgroup per CU (its LDS holds
// two chunks of split B planes): ~256 workgroups fill the chip.
constexpr long kTargetWgHb = 256;

int choose_walk_len(const helix_scan_desc& d, int cpg) {
    const long n_pslab = (d.head_dim + HELIX_HD - 1) / HELIX_HD;
    const long items = (long)d.n_seq * d.n_head * n_pslab;
    const long segs = std::max<long>(1, (kTargetWgA + items - 1) / items);
    const long len = std::min<long>((cpg + segs - 1) / segs, kMaxSegLen);
    return (int)std::max<long>(1, std::min<long>(len, cpg));
}

// Dispatch model of a one-workgroup-per-CU launch on MI355X, used to pick
// the walk length when every walk's start state comes from the walk's own
// prologue (fused Pass B). Workgroup b runs on XCD b % 8 (the kernels decode
// their logical id with xcd_logical_id); in each XCD, four shader engines of
// eight CUs take the XCD's workgroups round-robin, in dispatch order, and a
// workgroup waits for a CU of its own engine. Every running workgroup moves
// one chunk step per lat + k * load microseconds, load being the running
// workgroups over the chip (each weighted by the share of its heads or items
// that are real). lat and k, and a fixed cost per workgroup (o, plus g per
// segment aggregate a walk's prologue folds in), were fitted to Pass A and the
// bf16 walk timed at 19 lengths on S=8 L=4096 H=80 P=64 and H=27 P=192 (N=128):
// rms errors 1.8 and 2.0 %. Without the per-engine round robin the Pass A fit
// misses by up to 17 %: at H=27 and two segments, one engine in each XCD got
// six long and five short workgroups, ran three shorts in a row, and Pass A
// took the time of one 64-chunk segment.
struct DispatchCost {
    double lat, k, o, g;
};
constexpr DispatchCost kCostA{3.0, 0.009, 2.0, 0.0};
constexpr DispatchCost kCostWalk{2.25, 0.007, 0.5, 0.5};
constexpr int kXcds = 8, kEnginesPerXcd = 4, kCusPerEngine = 8;

// Microseconds for workgroups given in logical-id order as (chunk steps,
// weight). Every running workgroup advances at the same rate, so each
// engine's queue is list-scheduled at unit speed (the order of events does not
// depend on the rate) to the makespan T in chunk steps; the chip is busy
// throughout, and the integral of lat + k * load over T is
// lat * T + k * sum(weight * steps).
double dispatch_us(const std::vector<std::pair<double, double>>& wg, const DispatchCost& c) {
    const size_t n = wg.size();
    const size_t per = n / kXcds;
    double cu[kXcds * kEnginesPerXcd][kCusPerEngine] = {};
    double T = 0.0, work = 0.0;
    for (size_t b = 0; b < n; ++b) {
        const size_t x = b % kXcds, j = b / kXcds;
        const size_t wid = b < per * kXcds ? x * per + j : b;
        double* e = cu[x * kEnginesPerXcd + j % kEnginesPerXcd];
        int m = 0;
        for (int i = 1; i < kCusPerEngine; ++i)
            if (e[i] < e[m]) m = i;
        e[m] += wg[wid].first;
        T = std::max(T, e[m]);
        work += wg[wid].first * wg[wid].second;
    }
    return c.lat * T + c.k * work;
}

// Pass A (head-block kernel) and the walk with segments = walks of `len`
// chunks over a single group of `cpg` chunks: the workgroups of both launches
// in their kernels' logical order, priced by dispatch_us.
double fused_lengths_us(const helix_scan_desc& d, const HelixMatmulTraits& tr, int cpg, int len) {
    const int nseg = (cpg + len - 1) / len;
    const int nslab = (d.head_dim + HELIX_HD - 1) / HELIX_HD;
    const int hpg = d.n_head / d.n_group;
    auto seg_steps = [&](int s) { return (double)std::min(len, cpg - s * len); };
    std::vector<std::pair<double, double>> wg;
    // Pass A: (item block, group, segment, sequence), item = (head, P slab).
    const int ipg = hpg * nslab, nib = (ipg + HELIX_HB - 1) / HELIX_HB;
    wg.reserve((size_t)d.n_seq * nseg * d.n_group * nib);
    for (int seq = 0; seq < d.n_seq; ++seq)
        for (int s = 0; s < nseg; ++s)
            for (int g = 0; g < d.n_group; ++g)
                for (int ib = 0; ib < nib; ++ib)
                    wg.emplace_back(seg_steps(s) + kCostA.o,
                                    (double)std::min(HELIX_HB, ipg - HELIX_HB * ib) / HELIX_HB);
    const double a = dispatch_us(wg, kCostA);
    // Walk: (head block, group, slab, walk, sequence).
    const int hpw = tr.walk_hpw ? tr.walk_hpw : HELIX_WALK_HPW(tr.np);
    const int npair = (hpg + hpw - 1) / hpw;
    wg.clear();
    for (int seq = 0; seq < d.n_seq; ++seq)
        for (int s = 0; s < nseg; ++s)
            for (int sl = 0; sl < nslab; ++sl)
                for (int g = 0; g < d.n_group; ++g)
                    for (int pr = 0; pr < npair; ++pr)
                        wg.emplace_back(seg_steps(s) + kCostWalk.o + kCostWalk.g * s,
                                        (double)std::min(hpw, hpg - hpw * pr) / hpw);
    return a + dispatch_us(wg, kCostWalk);
}

// The walk length (= Pass A's segment) with the least modelled time among
// those of at most kFuseBMaxSegs walks, from `shortest` up. Memoized: the
// plan is remade on every encode.
int fused_walk_len(const helix_scan_desc& d, const HelixMatmulTraits& tr, int cpg, int shortest) {
    // Past 64 rounds of one-workgroup-per-CU walks, how the last round falls
    // is a small part of the time, and pricing every length would make the
    // first plan of a large batch slow: keep the default length.
    const long hpg = d.n_head / d.n_group;
    const long hpw = tr.walk_hpw ? tr.walk_hpw : HELIX_WALK_HPW(tr.np);
    const long walk_wg = (long)d.n_seq * d.n_group * ((hpg + hpw - 1) / hpw) *
                         ((d.head_dim + HELIX_HD - 1) / HELIX_HD) * ((cpg + shortest - 1) / shortest);
    if (walk_wg > 64L * kXcds * kEnginesPerXcd * kCusPerEngine) return shortest;
    using Key = std::tuple<int, int, int, int, int, int, int, int>;
    static std::mutex mu;
    static std::map<Key, int> memo;
    const Key key{d.n_seq, d.n_head, d.head_dim, d.n_group, tr.np, tr.walk_hpw, cpg, shortest};
    {
        std::lock_guard<std::mutex> lk(mu);
        const auto it = memo.find(key);
        if (it != memo.end()) return it->second;
    }
    int best = shortest;
    double best_us = fused_lengths_us(d, tr, cpg, shortest);
    for (int len = shortest + 1; len <= cpg; ++len) {
        const double us = fused_lengths_us(d, tr, cpg, len);
        if (us < best_us) {
            best_us = us;
            best = len;
        }
    }
    std::lock_guard<std::mutex> lk(mu);
    if (memo.size() > 4096) memo.clear();
    memo.emplace(key, best);
    return best;
}

// Pass A's segment (seg_len) and the walk's (walk_len, a multiple of it). The
// head-block Pass A takes the longest divisor of walk_len that still gives
// ~kTargetWgHb workgroups, so its segments nest in the walk's. HELIX_WALK_LEN
// sets walk_len, HELIX_SEG_LEN sets seg_len, and walk_len is then rounded to a
// multiple of it.
void choose_lengths(const helix_tuning& tu, const helix_scan_desc& d, const HelixMatmulTraits& tr, int cpg,
                    int* seg_len, int* walk_len) {
    int w = tu.walk_len > 0 ? std::min(tu.walk_len, cpg) : choose_walk_len(d, cpg);
    int a = w;
    if (tu.seg_len > 0) {
        a = std::min(tu.seg_len, cpg);
        w = std::max(a, (w / a) * a);
    } else if (tr.a_hb) {
        const long n_pslab = (d.head_dim + HELIX_HD - 1) / HELIX_HD;
        const long ipg = (long)(d.n_head / d.n_group) * n_pslab;
        const long per_seg = (long)d.n_seq * d.n_group * ((ipg + HELIX_HB - 1) / HELIX_HB);
        a = 1;
        for (int cand = w; cand >= 1; --cand) {
            if (w % cand) continue;
            if (per_seg * ((cpg + cand - 1) / cand) >= kTargetWgHb) {
                a = cand;
                break;
            }
        }
        // Walks that are Pass A's segments, few enough for the walk's prologue
        // to fold them in (fused Pass B), over a single group: a longer walk
        // may balance the one-workgroup-per-CU launches better. At S=8 L=4096
        // N=128 the model takes 43-chunk walks at H=80 P=64 and 22 at H=27
        // P=192, in place of 16: whole scans 605 -> 556 and 649 -> 588 us; on
        // seven other shapes of 2048-4096 tokens x 4-16 sequences it was 21-78
        // us faster on the bf16 path and no slower on the fp32 one.
        const int n_chunks = (d.n_tok + HELIX_CS - 1) / HELIX_CS;
        if (a == w && tu.walk_len <= 0 && tu.fuse_b != 0 && tr.walk && tr.walk_fuse_b && cpg == n_chunks &&
            (cpg + w - 1) / w <= kFuseBMaxSegs)
            a = w = fused_walk_len(d, tr, cpg, w);
    }
    if (!tr.walk) w = a;
    *seg_len = a;
    *walk_len = w;
}

void layout(const helix_tuning& tu, const helix_scan_desc& d, const HelixMatmulTraits& tr, int cpg,
            MultipassPlan* pl) {
    const bool bf16_state = tr.bf16_state, walk = tr.walk, bccopy = tr.bccopy, rec = tr.rec_kind != 0;
    const int np = tr.np;
    // State scratch is stored as padded slab tiles of 64 x np (helix_params.h).
    const size_t n_pslab = (size_t)(d.head_dim + HELIX_HD - 1) / HELIX_HD;
    const size_t state = (size_t)d.n_seq * d.n_head * n_pslab * 64 * (size_t)np;
    pl->chunks_per_group = cpg;
    choose_lengths(tu, d, tr, cpg, &pl->seg_len, &pl->walk_len);
    pl->segs_per_group = (cpg + pl->seg_len - 1) / pl->seg_len;
    pl->walks_per_group = (cpg + pl->walk_len - 1) / pl->walk_len;
    pl->sl_elem_bytes = bf16_state ? 2 : 4;
    pl->sl_elems = (pl->seg_len > 1 && !walk) ? state * (size_t)cpg : 0;
    pl->sg_elems = state * (size_t)pl->segs_per_group;
    pl->ld_elems = (size_t)d.n_seq * cpg * d.n_head;
    pl->sd_elems = (size_t)d.n_seq * pl->segs_per_group * d.n_head;
    pl->bc_elems = bccopy ? (size_t)d.n_seq * (size_t)cpg * HELIX_CS * d.n_group * d.d_state : 0;
    size_t off = 0;
    pl->off_sl = off; off += align256(pl->sl_elems * pl->sl_elem_bytes);
    pl->off_sg = off; off += align256(pl->sg_elems * sizeof(float));
    pl->off_ld = off; off += align256(pl->ld_elems * sizeof(float));
    pl->off_sd = off; off += align256(pl->sd_elems * sizeof(float));
    pl->off_bc = off; off += align256(pl->bc_elems * 2);
    pl->off_cc = off; off += align256(pl->bc_elems * 2);
    const size_t rec_bytes = tr.rec_kind == 1 ? HELIX_REC_WALK_BYTES : HELIX_REC64_BYTES;
    pl->rec_elems = rec ? (size_t)d.n_seq * (size_t)cpg * d.n_head * HELIX_CS * rec_bytes / sizeof(float) : 0;
    pl->off_rec = off; off += align256(pl->rec_elems * sizeof(float));
    pl->total_bytes = off;
}

}  // namespace

MultipassPlan plan_multipass(const helix_ctx* ctx, const helix_scan_desc& d, const HelixMatmulTraits& tr,
                             size_t budget_cap) {
    const helix_tuning& tu = tuning_of(ctx);
    MultipassPlan pl;
    if (d.n_tok <= 0 || d.n_seq <= 0 || d.n_head <= 0 || d.head_dim <= 0 || d.d_state <= 0 ||
        d.n_group <= 0)
        return pl;
    pl.n_chunks = (d.n_tok + HELIX_CS - 1) / HELIX_CS;

    // Default budget sized for MI355X's 288 GB: a 64-head 8K-token prefill
    // keeps all of its chunks in one group. HELIX_SCRATCH_MB=1 forces many
    // groups (reference caps.mm:170-176).
    const size_t budget = std::min((size_t)tu.scratch_mb << 20, budget_cap);
    // The most chunks per group whose layout fits the budget: all of them
    // when that fits (every BASELINE config under the default budget), else
    // a binary search (the layout grows with the chunks per group; one chunk
    // per group is the floor even past the budget).
    long lo = 1, hi = pl.n_chunks;
    auto fits = [&](long c) {
        layout(tu, d, tr, (int)c, &pl);
        return pl.total_bytes <= budget;
    };
    if (!fits(hi)) {
        while (hi - lo > 1) {
            const long mid = lo + (hi - lo) / 2;
            if (fits(mid)) lo = mid;
            else hi = mid;
        }
        layout(tu, d, tr, (int)lo, &pl);
    }
    pl.n_groups = (pl.n_chunks + pl.chunks_per_group - 1) / pl.chunks_per_group;

    // Pass C head blocks: share C.B^T over as many heads as possible while
    // keeping ~kTargetWgC workgroups per group launch.
    const int hpg = d.n_head / std::max(1, d.n_group);
    const long base = (long)d.n_seq * pl.chunks_per_group * d.n_group;
    long want_blocks = std::max<long>(1, (kTargetWgC + base - 1) / base);
    if (tu.hblk > 0) want_blocks = (hpg + tu.hblk - 1) / tu.hblk;
    want_blocks = std::min<long>(want_blocks, hpg);
    pl.hblk = (int)((hpg + want_blocks - 1) / want_blocks);
    pl.n_hblk = (hpg + pl.hblk - 1) / pl.hblk;
    return pl;
}

MultipassPlan plan_ytile(const helix_ctx* ctx, const helix_scan_desc& d, const HelixMatmulTraits& single,
                         const HelixMatmulTraits** tr_out) {
    MultipassPlan pl;
    *tr_out = nullptr;
    const helix_tuning& tu = tuning_of(ctx);
    if (tu.ytile == 0 || !single.k_single || d.a_form != HELIX_A_SCALAR_PER_HEAD || d.io_dtype != HELIX_F32 ||
        d.d_state > 128 || d.n_tok <= 0 || d.n_seq <= 0 || d.n_head <= 0 || d.head_dim <= 0 || d.n_group <= 0)
        return pl;
    // y's rows hold 16-byte tile units: channel stride 1, the others multiples
    // of four elements (the encoder also checks y's base).
    if (d.s_y[2] != 1 || (d.s_y[0] | d.s_y[1] | d.seq_y) % 4 != 0) return pl;
    const HelixMatmulTraits& tr = table().ysingle[np_index(d.d_state)];
    const long n_chunks = (d.n_tok + HELIX_CS - 1) / HELIX_CS;
    // Every segment must have the rows its tile and log-decay take, at the
    // narrowest slab width; the last segment is the shortest.
    const int n_pslab = (d.head_dim + HELIX_HD - 1) / HELIX_HD;
    const int pw_min = std::min(HELIX_HD, d.head_dim - (n_pslab - 1) * HELIX_HD);
    const long upr = pw_min / 4;
    const long rows = (16L * tr.np + 1 + upr - 1) / upr;
    auto fits = [&](long sl) {
        const long n_seg = (n_chunks + sl - 1) / sl;
        return d.n_tok - (n_seg - 1) * sl * HELIX_CS >= rows;
    };
    if (d.n_tok < rows || rows * d.s_y[0] * 4 >= (1LL << 31)) return pl;
    layout(tu, d, tr, (int)n_chunks, &pl);
    if (!fits(pl.seg_len)) {
        // Longer segments (the walk keeps its number of segments): the
        // shortest that gives every segment its rows. The whole sequence as
        // one segment always does, since n_tok >= rows.
        const int ratio = std::max(1, pl.walk_len / std::max(1, pl.seg_len));
        helix_tuning t2 = tu;
        for (long sl = std::max<long>(pl.seg_len + 1, (rows + HELIX_CS - 1) / HELIX_CS); sl <= n_chunks; ++sl) {
            if (!fits(sl)) continue;
            t2.seg_len = (int)sl;
            t2.walk_len = (int)std::min<long>(sl * ratio, n_chunks);
            break;
        }
        if (t2.seg_len <= 0) return pl = MultipassPlan{}, pl;
        layout(t2, d, tr, (int)n_chunks, &pl);
        if (!fits(pl.seg_len)) return pl = MultipassPlan{}, pl;
    }
    pl.n_chunks = (int)n_chunks;
    pl.n_groups = 1;
    pl.total_bytes = 0;   // nothing outside y
    pl.hblk = 1;
    pl.n_hblk = d.n_head / d.n_group;
    *tr_out = &tr;
    return pl;
}

bool build_params(const helix_scan_desc& d, HelixScanParams* o, std::string* why) {
    std::memset(o, 0, sizeof(*o));
    o->n_tok = d.n_tok;
    o->n_seq = d.n_seq;
    o->n_head = d.n_head;
    o->head_dim = d.head_dim;
    o->d_state = d.d_state;
    o->n_group = d.n_group;
    o->heads_per_group = d.n_head / d.n_group;
    o->n_pslab = (d.head_dim + HELIX_HD - 1) / HELIX_HD;
    for (int i = 0; i < 3; ++i) {
        o->s_x[i] = d.s_x[i];
        o->s_b[i] = d.s_b[i];
        o->s_c[i] = d.s_c[i];
        o->s_s[i] = d.s_s[i];
        o->s_y[i] = d.s_y[i];
    }
    o->s_dt[0] = d.s_dt[0];
    o->s_dt[1] = d.s_dt[1];
    o->seq_x = d.seq_x;
    o->seq_b = d.seq_b;
    o->seq_c = d.seq_c;
    o->seq_dt = d.seq_dt;
    o->seq_s = d.seq_s;
    o->seq_y = d.seq_y;
    o->s_a = d.s_a;
    o->dt_min = d.dt_min;
    o->dt_max = d.dt_max;

    // The kernels address one chunk of a tensor through a buffer resource
    // based at the chunk's first element, with 32-bit byte offsets: every
    // stride must be non-negative and a chunk's extent stay below 2 GiB.
    const long long strides[] = {d.s_x[0], d.s_x[1], d.s_x[2], d.s_b[0], d.s_b[1], d.s_c[0],
                                 d.s_c[1], d.s_dt[0], d.s_dt[1], d.s_y[0], d.s_y[1], d.s_y[2],
                                 d.seq_x, d.seq_b, d.seq_c, d.seq_dt, d.seq_s, d.seq_y, d.s_a};
    for (long long s : strides) {
        if (s < 0) {
            if (why) *why = "negative stride";
            return false;
        }
    }
    const long long kCs = HELIX_CS - 1, kHd = HELIX_HD - 1;
    const long long spans[] = {kCs * d.s_x[0] + kHd * d.s_x[2] + 1, kCs * d.s_y[0] + kHd * d.s_y[2] + 1,
                               kCs * d.s_b[0] + d.d_state, kCs * d.s_c[0] + d.d_state,
                               kCs * d.s_dt[0] + 1};
    for (long long e : spans) {
        if (e * (long long)sizeof(float) >= (1LL << 31)) {
            if (why) *why = "one chunk of a tensor spans 2 GiB or more";
            return false;
        }
    }

    // Grid y and z are 16-bit on the hardware dispatch packet.
    const long kMaxYZ = 65535;
    const long zA = (long)d.n_seq * o->n_pslab;
    if (d.n_head > kMaxYZ || zA > kMaxYZ || d.n_seq > kMaxYZ) {
        if (why) *why = "launch grid exceeds 65535 in y or z (n_head or n_seq*n_pslab too large)";
        return false;
    }
    return true;
}

}  // namespace helix::rt

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" const char* helix_ctx_last_error(const helix_ctx* ctx) {
    if (!ctx) return t_last_ctx == nullptr && !t_last_error.empty() ? t_last_error.c_str() : "null context";
    return t_last_ctx == ctx ? t_last_error.c_str() : "";
}

extern "C" bool helix_scan_supported(helix_ctx* ctx, const helix_scan_desc* d) {
    if (!ctx || !d) return false;
    if (d->n_tok <= 0 || d->n_seq <= 0 || d->n_head <= 0 || d->head_dim <= 0 ||
        d->d_state <= 0 || d->n_group <= 0)
        return false;
    if (d->n_head % d->n_group != 0) return false;
    // Scalar A runs on every path; diagonal A (one decay per state index) on
    // the fp32 single-pass walk only, up to d_state 128 (an explicit bf16
    // request for it is declined, as the reference declines diagonal A).
    if (d->a_form == HELIX_A_DIAG_PER_CHANNEL) {
        if (d->d_state > 128 || d->backend == HELIX_BACKEND_MPP) return false;
    } else if (d->a_form != HELIX_A_SCALAR_PER_HEAD) {
        return false;
    }
    // Storage of x/B/C/y in F32, F16 or BF16; compute_dtype stays F32 (the
    // bf16 compute path is chosen by backend, reference caps.mm:126).
    if (d->compute_dtype != HELIX_F32) return false;
    if (d->io_dtype != HELIX_F32) {
        if (d->io_dtype != HELIX_F16 && d->io_dtype != HELIX_BF16) return false;
        // 16-bit storage with scalar A only; B and C rows are read as runs of
        // eight elements, kept 4-byte aligned by even element strides.
        if (d->a_form != HELIX_A_SCALAR_PER_HEAD) return false;
        if ((d->s_b[0] | d->s_b[1] | d->seq_b | d->s_c[0] | d->s_c[1] | d->seq_c) & 1) return false;
    }
    if (d->d_state % 8 != 0 || d->head_dim % 8 != 0) return false;
    // A larger d_state runs as blocks of state indices on the fp32 path, each
    // adding its share into y (helix::rt::state_block): fp32 storage and
    // scalar A only, and no explicit bf16 request (the reference serves its
    // bf16 Pass C at d_state 128 and 256 only, caps.mm:65-73; AUTO takes the
    // fp32 path there too, caps.mm:89-93).
    if (d->d_state > HELIX_N_MAX &&
        (d->io_dtype != HELIX_F32 || d->a_form != HELIX_A_SCALAR_PER_HEAD || d->backend == HELIX_BACKEND_MPP))
        return false;
    // B, C rows and state rows are staged as contiguous d_state vectors.
    if (d->s_b[2] != 1 || d->s_c[2] != 1 || d->s_s[2] != 1) return false;
    if (d->s_s[1] != d->d_state) return false;
    if (d->chunk != 0 && d->chunk != HELIX_CS) return false;
    // An explicit bf16 (MPP) request must be serviceable, and the bf16 Pass C
    // exists only in the multipass decomposition (reference caps.mm:66,145-147).
    if (!d->multipass && d->backend == HELIX_BACKEND_MPP) return false;
    if (d->backend == HELIX_BACKEND_REF) return false;
    HelixScanParams unused;
    return helix::rt::build_params(*d, &unused, nullptr);
}

extern "C" size_t helix_scan_scratch_size(helix_ctx* ctx, const helix_scan_desc* d) {
    // The single-pass walks (multipass = false, diagonal A, 16-bit storage off
    // the bf16 path) use none.
    if (!d || !d->multipass) return 0;
    const HelixMatmulTraits& tr = helix::rt::select_traits(ctx, *d);
    if (tr.k_single) return 0;
    // Blocks run one after another in the same scratch: the largest block's
    // plan. (Where y overlaps an input, up to HELIX_N_MAX, the encoder runs
    // the one-launch single pass instead, which needs none.)
    return helix::rt::plan_multipass(ctx, helix::rt::plan_desc(ctx, *d), tr).total_bytes;
}

extern "C" helix_backend helix_ctx_select_backend(helix_ctx* ctx, const helix_scan_desc* d) {
    if (!ctx || !d) return HELIX_BACKEND_REF;
    if (d->backend == HELIX_BACKEND_SGMMA) return HELIX_BACKEND_SGMMA;
    return helix::rt::select_traits(ctx, *d).backend;
}

extern "C" const char* helix_ctx_backend_desc(helix_ctx* ctx, const helix_scan_desc* d) {
    if (!ctx || !d) return "unavailable (null context)";
    if (!helix_scan_supported(ctx, d)) return "declined (shape unsupported)";
    const HelixMatmulTraits& tr = helix::rt::select_traits(ctx, *d);
    return helix::rt::n_state_blocks(ctx, *d) > 1 && tr.name_blocks ? tr.name_blocks : tr.name;
}
