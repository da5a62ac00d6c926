// helix_internal.h -- C++ internals of the MI355X HELIX runtime. Not part of
// the ABI. Counterpart of the reference's src/runtime/helix_internal.h:12-112
// with the Metal device/library/pipeline objects replaced by one hipModule
// whose kernels are all resolved when the context is created.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>

#include "helix/helix.h"
#include "../kernels/helix_params.h"

// Tuning read from the environment once, when the context is created, so that
// every plan a context makes (helix_scan_scratch_size, helix_scan_encode,
// helix_scan_plan_info) is a pure function of the context and the descriptor.
// Two knobs carry the reference's meaning (caps.mm:82-86,170-176); the rest
// override planner choices for measurement and tests.
struct helix_tuning {
    long scratch_mb  = 2048;   // HELIX_SCRATCH_MB: scratch budget per encode
    bool force_fp32  = false;  // HELIX_FORCE_BACKEND=s...: pin the fp32 path
    int  passa_split = 6;      // HELIX_PASSA_SPLIT=3: bf16 path Pass A on two split
                               // planes (three products, state to about 2^-16;
                               // opt-in, narrower than the reference's fp32 Pass A)
    int  passa_f16   = -1;     // HELIX_PASSA_F16=0: bf16 path Pass A (d_state <= 128) on six
                               // bf16 split products instead of two scaled fp16 planes
                               // (three products)
    int  fuse_b      = -1;     // HELIX_FUSE_B=0|1: Pass B in the walk's prologue
    int  bccopy      = -1;     // HELIX_WALK_BCCOPY=0: no bf16 copies of B and C
    int  seg_len     = 0;      // HELIX_SEG_LEN: chunks per Pass A segment
    int  walk_len    = 0;      // HELIX_WALK_LEN: chunks per walk (rounded to a multiple of seg_len)
    int  hblk        = 0;      // HELIX_HBLK: heads per chunk-parallel Pass C workgroup
    int  f32_walk    = -1;     // HELIX_F32_WALK=0 / 1: the fp32 path's chunk-parallel Pass C / walk
                               // (on per-chunk states stored by Pass A) at d_state 128
    int  ytile       = -1;     // HELIX_1PASS_Y=0: the single pass in its one-launch form only
    int  state_blocks = -1;    // HELIX_STATE_BLOCKS=0|1: d_state 129..256 (fp32 storage,
                               // scalar A) as blocks of at most 128 state indices, or not
};

struct helix_ctx {
    helix_tuning tuning;
    int         device = -1;
    hipModule_t module = nullptr;
    std::string arch;          // gcnArchName, e.g. "gfx950:sramecc+:xnack-"
    std::string code_object;   // "<embedded>" or the file it was loaded from
    int         n_cu = 0;
    // Filled once at creation and only read afterwards, so encoding from
    // several host threads needs no lock.
    std::unordered_map<std::string, hipFunction_t> kernels;
};

// Which kernels a descriptor runs. Counterpart of the reference's
// HelixMatmulTraits (helix_internal.h:38-48, caps.mm:18-61): chosen per
// descriptor, never fails, and names the CDNA4 MFMA shape each pass uses.
struct HelixMatmulTraits {
    helix_backend backend;
    const char*   name;            // what helix_ctx_backend_desc reports
    const char*   name_blocks;     // the same for blocks of state indices
    const char*   k_chunk_state;   // Pass A
    const char*   k_state_scan;    // Pass B
    const char*   k_chunk_out;     // Pass C
    // Pass C of a block of state indices after the first, which adds into y
    // with y loaded ahead (null: k_chunk_out adds through y_acc itself).
    const char*   k_chunk_out_acc;
    bool          bf16_state;      // s_local kept in bf16 (Pass C takes bf16 operands)
    const char*   mfma_a;          // MFMA instruction of Pass A
    const char*   mfma_c;          // MFMA instruction of Pass C
    int           np;              // d_state padding the kernels are built for
    // Pass C walks the chunks of each segment with the state in registers
    // (one workgroup per segment x head x P slab); Pass A then stores only the
    // segment aggregates and there is no per-chunk state in scratch.
    bool          walk;
    // The single-pass kernel (multipass = false; reference k_single,
    // caps.mm:18-25). Set only in the single-pass trait set, where the three
    // pass names are null.
    const char*   k_single;
    // Its form for a block of state indices after the first, which adds into
    // y with y loaded ahead (null: k_single adds through y_acc itself).
    const char*   k_single_acc;
    int           single_threads;  // its workgroup size (64 x waves)
    // Heads per workgroup of a walking Pass C; 0 means HELIX_WALK_HPW(np).
    int           walk_hpw;
    // Pass A writes bf16 copies of B and C that the walking Pass C reads.
    bool          bccopy;
    // The walking Pass C can run Pass B's segment scan in its prologue
    // (HelixScanParams::fuse_b); the encoder then skips Pass B's launch
    // whenever the plan has a single group.
    bool          walk_fuse_b;
    // Pass A is the head-block kernel (pass_a_hb.hip): a 1-D grid of
    // HELIX_HB_THREADS-thread workgroups, one per (seq, group, item block,
    // segment); otherwise one 256-thread workgroup per (segment, head, seq x slab).
    bool          a_hb;
    // Pass A stores per-token decay records (HelixScanBuffers::pre) that Pass
    // C reads instead of recomputing its decay preamble: 0 none, 1 the
    // walk's form (store_decay_record), 2 the fp64 form of the fp32 path's
    // bf16x6 Pass C (store_decay_record64).
    int           rec_kind;
};

namespace helix::rt {

// The environment's tuning (see helix_tuning), read by helix_ctx_create*.
helix_tuning tuning_from_env();

// Every kernel name in the traits tables; all are resolved at context creation.
const char* const* all_kernel_names(size_t* count);

// Never fails: falls back to the fp32 path whenever bf16 is not requested or
// not serviceable. A pure function of the context's tuning and the
// descriptor; ctx == nullptr plans with the default tuning.
const HelixMatmulTraits& select_traits(const helix_ctx* ctx, const helix_scan_desc& d);
// The same for d run in one launch sequence (d_state <= HELIX_N_MAX), whether
// or not blocks of state indices would apply; block: d is one block of state
// indices of a larger d_state (state_block).
const HelixMatmulTraits& select_traits_unblocked(const helix_ctx* ctx, const helix_scan_desc& d,
                                                 bool block = false);

// How the multipass scan is tiled over the sequence (see helix_params.h):
// super-chunk groups bound live scratch; segments of seg_len chunks are the
// unit of Pass A's in-register walk and of Pass B's scan; head blocks are the
// unit of Pass C's reuse of C.B^T. A pure function of the descriptor, the
// selected kernels and the context's tuning, so helix_scan_scratch_size() and
// the encoder agree exactly.
struct MultipassPlan {
    int    n_chunks         = 0;
    int    chunks_per_group = 0;
    int    n_groups         = 0;
    int    seg_len          = 0;   // chunks per Pass A segment
    int    segs_per_group   = 0;
    int    walk_len         = 0;   // chunks per walking Pass C segment (multiple of seg_len)
    int    walks_per_group  = 0;
    int    hblk             = 0;
    int    n_hblk           = 0;
    size_t sl_elems         = 0;   // s_local elements (0 when seg_len == 1)
    size_t sl_elem_bytes    = 4;   // 4 (fp32 path) or 2 (bf16 path)
    size_t sg_elems         = 0;   // s_seg elements (fp32)
    size_t ld_elems         = 0;
    size_t sd_elems         = 0;
    size_t bc_elems         = 0;   // elements of each bf16 copy of B and C (0: none)
    size_t rec_elems        = 0;   // fp32 elements of the decay records (0: none)
    size_t off_sl = 0, off_sg = 0, off_ld = 0, off_sd = 0, off_bc = 0, off_cc = 0, off_rec = 0;
    size_t total_bytes      = 0;
};

// budget_cap (bytes) lowers the context's scratch budget for this plan
// (helix_scan_encode_noalloc plans for its fixed array).
MultipassPlan plan_multipass(const helix_ctx* ctx, const helix_scan_desc& d, const HelixMatmulTraits& tr,
                             size_t budget_cap = SIZE_MAX);

// Whether the walking Pass C runs Pass B's segment scan itself (no Pass B
// launch): a single-group plan of at most four segments on a kernel that can;
// the tuning's fuse_b (HELIX_FUSE_B=0 / 1) turns it off / on for any
// single-group plan.
bool fuse_b_on(const helix_ctx* ctx, const HelixMatmulTraits& tr, const MultipassPlan& plan);

// The single pass (multipass = false, fp32 storage, scalar A, d_state <= 128)
// run as the three passes of the fp32 path with no scratch: the state tiles
// and segment log-decays live in y (HelixScanParams::ytile), one group, Pass B
// launched. Returns the plan and sets *tr_out to its traits, or returns an
// empty plan (n_chunks 0) where the shape does not allow it: y's strides, a
// last segment too short for a tile, or HELIX_1PASS_Y=0. The encoder also
// needs y 16-byte aligned and overlapping no input.
MultipassPlan plan_ytile(const helix_ctx* ctx, const helix_scan_desc& d, const HelixMatmulTraits& single,
                         const HelixMatmulTraits** tr_out);


// Blocks of state indices (fp32 storage, scalar A): the recurrence is
// independent per state index and y sums C_n h_n over them, so the scan can
// run once per block of state indices, each block adding its share into y
// (HelixScanParams::y_acc). Above HELIX_N_MAX it must (one launch serves at
// most 256); from HELIX_N_BLOCK + 1 up to HELIX_N_MAX it may, where the
// blocks' d_state <= 128 kernels beat the d_state 256 ones
// (HELIX_STATE_BLOCKS pins it). n_state_blocks is 1 where no blocks apply;
// otherwise the blocks are equal (multiples of 8, at most HELIX_N_BLOCK).
// state_block is block k's descriptor: d_state the block's size, strides
// unchanged (s_s[1] stays the caller's d_state, the row length of s0 and
// s1), backend the fp32 path above HELIX_N_MAX (the caller's otherwise); *n0
// (if given) is its first state index, the element offset of B, C, s0 and
// s1.
int n_state_blocks(const helix_ctx* ctx, const helix_scan_desc& d);
helix_scan_desc state_block(const helix_ctx* ctx, const helix_scan_desc& d, int k, int* n0);
// The descriptor the plan and kernels are chosen for: block 0 (the largest)
// where blocks apply, else d itself.
helix_scan_desc plan_desc(const helix_ctx* ctx, const helix_scan_desc& d);

// Fills the kernel-side params from the public descriptor. Returns false and
// sets *why when a launch dimension would exceed the hardware grid limits.
bool build_params(const helix_scan_desc& d, HelixScanParams* out, std::string* why);

// Thread-local last-error bookkeeping.
void set_error(const helix_ctx* ctx, const std::string& msg);

// The fixed scratch of helix_scan_encode_noalloc (noalloc.hip): its device
// address on `device`, resolved on the entry point's first call there (with
// that device current) and kept; null, with *why set, if unavailable.
void* noalloc_scratch(int device, std::string* why);

}  // namespace helix::rt
