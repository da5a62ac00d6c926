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
#include <string>

#include "helix_internal.h"

namespace {

// The fp32 path: all three passes on v_mfma_f32_32x32x2_f32 (FP32 matrix and
// FP32 vector peaks are both 157.3 TFLOP/s on MI355X; the matrix path keeps
// the operands in LDS/registers instead of spending VALU issue slots).
constexpr HelixMatmulTraits kF32Traits[] = {
    {HELIX_BACKEND_SGMMA, "mfma fp32 (d_state<=64)", "helix_chunk_state_f32_n64",
     "helix_state_scan_f32", "helix_chunk_out_f32_n64", false,
     "v_mfma_f32_32x32x2_f32", "v_mfma_f32_32x32x2_f32", 64, false},
    {HELIX_BACKEND_SGMMA, "mfma fp32 (d_state<=128)", "helix_chunk_state_f32_n128",
     "helix_state_scan_f32", "helix_chunk_out_f32_n128", false,
     "v_mfma_f32_32x32x2_f32", "v_mfma_f32_32x32x2_f32", 128, false},
    {HELIX_BACKEND_SGMMA, "mfma fp32 (d_state<=256)", "helix_chunk_state_f32_n256",
     "helix_state_scan_f32", "helix_chunk_out_f32_n256", false,
     "v_mfma_f32_32x32x2_f32", "v_mfma_f32_32x32x2_f32", 256, false},
};

// The bf16 path (the reference's MPP slot): Pass C on v_mfma_f32_32x32x16_bf16
// with fp32 accumulators; Passes A and B stay fp32, so the carried state and
// s1 keep fp32 accuracy. The per-chunk state Pass C reads is stored as bf16.
constexpr HelixMatmulTraits kBf16Traits[] = {
    {HELIX_BACKEND_MPP, "mfma bf16 pass C (d_state<=64)", "helix_chunk_state_sbf_n64",
     "helix_state_scan_f32", "helix_chunk_out_bf16_n64", true,
     "v_mfma_f32_32x32x2_f32", "v_mfma_f32_32x32x16_bf16", 64, false},
    {HELIX_BACKEND_MPP, "mfma bf16 pass C (d_state<=128)", "helix_chunk_state_sbf_n128",
     "helix_state_scan_f32", "helix_chunk_out_bf16_n128", true,
     "v_mfma_f32_32x32x2_f32", "v_mfma_f32_32x32x16_bf16", 128, false},
    {HELIX_BACKEND_MPP, "mfma bf16 pass C (d_state<=256)", "helix_chunk_state_sbf_n256",
     "helix_state_scan_f32", "helix_chunk_out_bf16_n256", true,
     "v_mfma_f32_32x32x2_f32", "v_mfma_f32_32x32x16_bf16", 256, false},
};

// Alternative bf16 path: Pass A stores only segment aggregates (fp32) and
// Pass C walks each segment's chunks with the state in registers, so no
// per-chunk state is written or read. Passes A and B remain fp32.
constexpr HelixMatmulTraits kBf16WalkTraits[] = {
    {HELIX_BACKEND_MPP, "mfma bf16 pass C, chunk walk (d_state<=64)", "helix_chunk_state_agg_n64",
     "helix_state_scan_f32", "helix_scan_walk_bf16_n64", true,
     "v_mfma_f32_32x32x2_f32", "v_mfma_f32_32x32x16_bf16", 64, true},
    {HELIX_BACKEND_MPP, "mfma bf16 pass C, chunk walk (d_state<=128)", "helix_chunk_state_agg_n128",
     "helix_state_scan_f32", "helix_scan_walk_bf16_n128", true,
     "v_mfma_f32_32x32x2_f32", "v_mfma_f32_32x32x16_bf16", 128, true},
    {HELIX_BACKEND_MPP, "mfma bf16 pass C, chunk walk (d_state<=256)", "helix_chunk_state_agg_n256",
     "helix_state_scan_f32", "helix_scan_walk_bf16_n256", true,
     "v_mfma_f32_32x32x2_f32", "v_mfma_f32_32x32x16_bf16", 256, true},
};

// The single-pass path (multipass = false, the descriptor default; reference
// helix_scan_sgmma_f32): one launch per encode, one workgroup per (seq, head,
// P slab) walking every chunk with the state in registers, fp32 MFMA
// throughout, no scratch. AUTO and SGMMA both land here (the reference's MPP
// traits exist only for multipass, caps.mm:66).
constexpr HelixMatmulTraits kSingleTraits[] = {
    {HELIX_BACKEND_SGMMA, "mfma fp32, single pass (d_state<=64)", nullptr, nullptr, nullptr, false,
     "v_mfma_f32_16x16x4_f32", "v_mfma_f32_16x16x4_f32", 64, false, "helix_scan_1pass_f32_n64"},
    {HELIX_BACKEND_SGMMA, "mfma fp32, single pass (d_state<=128)", nullptr, nullptr, nullptr, false,
     "v_mfma_f32_16x16x4_f32", "v_mfma_f32_16x16x4_f32", 128, false, "helix_scan_1pass_f32_n128"},
    {HELIX_BACKEND_SGMMA, "mfma fp32, single pass (d_state<=256)", nullptr, nullptr, nullptr, false,
     "v_mfma_f32_16x16x4_f32", "v_mfma_f32_16x16x4_f32", 256, false, "helix_scan_1pass_f32_n256"},
};

// Diagonal A (A[h][n], HELIX_A_DIAG_PER_CHANNEL): the reference declines it
// (caps.mm:121-123) because its chunked factorization needs one decay per
// (head, token); here the single-pass walk serves it, with M summed on the
// VALU and the other decays folded into row scales (pass_single.hip). It runs
// for either value of `multipass` (there is no three-pass form) and needs no
// scratch. d_state <= 128.
constexpr HelixMatmulTraits kDiagTraits[] = {
    {HELIX_BACKEND_SGMMA, "mfma fp32, single pass, diagonal A (d_state<=64)", nullptr, nullptr, nullptr, false,
     "v_mfma_f32_16x16x4_f32", "v_mfma_f32_16x16x4_f32", 64, false, "helix_scan_1pass_diag_f32_n64"},
    {HELIX_BACKEND_SGMMA, "mfma fp32, single pass, diagonal A (d_state<=128)", nullptr, nullptr, nullptr, false,
     "v_mfma_f32_16x16x4_f32", "v_mfma_f32_16x16x4_f32", 128, false, "helix_scan_1pass_diag_f32_n128"},
};

// bf16x6 kernels: GEMMs on bf16 MFMA over operands split into three bf16
// parts, fp32 accuracy at 16x the fp32 matrix issue rate. Pass A uses them on
// every path (pass_a_x6.hip) and the fp32 path's Pass C for d_state <= 128
// (pass_c_x6.hip; d_state 256 does not fit its LDS budget). The default;
// HELIX_X6=0 selects the fp32-MFMA kernels above.
constexpr const char* kX6StateF32[] = {"helix_chunk_state_x6f32_n64", "helix_chunk_state_x6f32_n128",
                                       "helix_chunk_state_x6f32_n256"};
constexpr const char* kX6StateSbf[] = {"helix_chunk_state_x6sbf_n64", "helix_chunk_state_x6sbf_n128",
                                       "helix_chunk_state_x6sbf_n256"};
constexpr const char* kX6StateAgg[] = {"helix_chunk_state_x6agg_n64", "helix_chunk_state_x6agg_n128",
                                       "helix_chunk_state_x6agg_n256"};
constexpr const char* kWalk16[] = {"helix_scan_walk16_bf16_n64", "helix_scan_walk16_bf16_n128",
                                    "helix_scan_walk16_bf16_n256"};
constexpr const char* kWalk16Bc[] = {"helix_scan_walk16_bf16_bc_n64", "helix_scan_walk16_bf16_bc_n128",
                                      "helix_scan_walk16_bf16_bc_n256"};
constexpr const char* kX6StateAggBc[] = {"helix_chunk_state_x6agg_bc_n64", "helix_chunk_state_x6agg_bc_n128",
                                         "helix_chunk_state_x6agg_bc_n256"};
constexpr const char* kX6OutF32[] = {"helix_chunk_out_x6_n64", "helix_chunk_out_x6_n128", nullptr};
// Pass A on two split planes (three bf16 products, about 2^-16 relative per
// product) for the walking bf16 Pass C, whose own operands are bf16: the
// segment aggregates it and Pass B consume stay 500x more accurate than
// Pass C's output. HELIX_PASSA_SPLIT=6 keeps the six-product kernels.
constexpr const char* kX3StateAgg[] = {"helix_chunk_state_x3agg_n64", "helix_chunk_state_x3agg_n128",
                                       "helix_chunk_state_x3agg_n256"};
constexpr const char* kX3StateAggBc[] = {"helix_chunk_state_x3agg_bc_n64", "helix_chunk_state_x3agg_bc_n128",
                                         "helix_chunk_state_x3agg_bc_n256"};
constexpr const char* kMfmaX3 = "v_mfma_f32_32x32x16_bf16 (bf16x3 split operands)";

// The selectable trait sets: [family: fp32, bf16, bf16 walk][np index], with
// Pass A on fp32 MFMA or bf16x6. Built once; names live as long as the process.
struct TraitSets {
    HelixMatmulTraits t[2][3][3];
    HelixMatmulTraits w16[2][3];   // the walk family with the 16 x 16 tile Pass C
    HelixMatmulTraits w16bc[3];    // ... reading bf16 B and C copies from Pass A (bf16x6)
    HelixMatmulTraits w16x3[3], w16x3bc[3];   // the same two with Pass A on bf16x3
    std::string names[2][3][3], x3names[2][3];
    TraitSets() {
        const HelixMatmulTraits* base[3] = {kF32Traits, kBf16Traits, kBf16WalkTraits};
        const char* const* x6[3] = {kX6StateF32, kX6StateSbf, kX6StateAgg};
        for (int fam = 0; fam < 3; ++fam)
            for (int k = 0; k < 3; ++k) {
                t[0][fam][k] = base[fam][k];
                HelixMatmulTraits& v = t[1][fam][k];
                v = base[fam][k];
                std::string nm = v.name;
                const size_t at = nm.find(" (d_state");
                const bool x6c = fam == 0 && kX6OutF32[k] != nullptr;
                names[1][fam][k] =
                    nm.substr(0, at) + (x6c ? ", passes A and C bf16x6" : ", pass A bf16x6") + nm.substr(at);
                v.name = names[1][fam][k].c_str();
                v.k_chunk_state = x6[fam][k];
                v.mfma_a = "v_mfma_f32_32x32x16_bf16 (bf16x6 split operands)";
                if (x6c) {
                    v.k_chunk_out = kX6OutF32[k];
                    v.mfma_c = "v_mfma_f32_32x32x16_bf16 (bf16x6 split operands)";
                    v.rec_kind = 2;
                }
            }
        for (int x6 = 0; x6 < 2; ++x6)
            for (int k = 0; k < 3; ++k) {
                w16[x6][k] = t[x6][2][k];
                w16[x6][k].k_chunk_out = kWalk16[k];
                w16[x6][k].mfma_c = "v_mfma_f32_16x16x32_bf16";
                w16[x6][k].walk_hpw = HELIX_WALK16_HPW(64 << k);
                w16[x6][k].walk_fuse_b = true;
                w16[x6][k].rec_kind = 1;
            }
        for (int k = 0; k < 3; ++k) {
            w16bc[k] = w16[1][k];
            w16bc[k].k_chunk_state = kX6StateAggBc[k];
            w16bc[k].k_chunk_out = kWalk16Bc[k];
            w16bc[k].bccopy = true;
        }
        for (int k = 0; k < 3; ++k) {
            HelixMatmulTraits* dst[2] = {&w16x3[k], &w16x3bc[k]};
            const HelixMatmulTraits* src[2] = {&w16[1][k], &w16bc[k]};
            const char* ka[2] = {kX3StateAgg[k], kX3StateAggBc[k]};
            for (int i = 0; i < 2; ++i) {
                *dst[i] = *src[i];
                std::string nm = src[i]->name;
                const size_t at = nm.find("bf16x6");
                if (at != std::string::npos) nm.replace(at, 6, "bf16x3");
                x3names[i][k] = nm;
                dst[i]->name = x3names[i][k].c_str();
                dst[i]->k_chunk_state = ka[i];
                dst[i]->mfma_a = kMfmaX3;
            }
        }
    }
};

// Pass A of the walking bf16 path on two split planes unless
// HELIX_PASSA_SPLIT=6.
bool passa_x3_on() {
    const char* v = std::getenv("HELIX_PASSA_SPLIT");
    return !(v && v[0] == '6');
}

// Pass A writes bf16 copies of B and C for the walking Pass C (fp32
// storage, bf16x6 Pass A) unless HELIX_WALK_BCCOPY=0, when the K =
// heads_per_group * n_pslab workgroups of a chunk cover its 64 rows with two
// quads of four state indices per thread (pass_a_x6.hip, copy_map).
bool bccopy_on(const helix_scan_desc& d) {
    const char* v = std::getenv("HELIX_WALK_BCCOPY");
    if (v && v[0] == '0') return false;
    const long K = (long)(d.n_head / d.n_group) * ((d.head_dim + HELIX_HD - 1) / HELIX_HD);
    return (64 + K - 1) / K * (d.d_state / 4) <= 2 * 256;
}

// The walking Pass C runs on 16 x 16 tiles (pass_c_walk16.hip) unless
// HELIX_WALK=32 asks for the 32 x 32 tile kernel (pass_c_walk.hip).
bool walk16_on() {
    const char* v = std::getenv("HELIX_WALK");
    return !(v && v[0] == '3' && v[1] == '2');
}

const HelixMatmulTraits& pick_traits(int fam, int k, const helix_scan_desc& d) {
    static const TraitSets sets;
    const char* v = std::getenv("HELIX_X6");
    const int x6 = (v && v[0] == '0') ? 0 : 1;
    if (fam == 2 && walk16_on()) {
        if (x6 && passa_x3_on()) return bccopy_on(d) ? sets.w16x3bc[k] : sets.w16x3[k];
        return (x6 && bccopy_on(d)) ? sets.w16bc[k] : sets.w16[x6][k];
    }
    return sets.t[x6][fam][k];
}

// 16-bit storage of x, B, C and y (io_dtype F16 or BF16; dt, A and the states
// stay fp32). A bf16 multipass request walks segments in Pass C with Pass A's
// aggregate kernel reading the 16-bit operands; every other request runs the
// single-pass kernel with fp32 compute. [io: 0 bf16, 1 f16][0 walk, 1 single][np]
bool walk16_on();

struct IoTraitSets {
    HelixMatmulTraits t[2][2][3], w16[2][3], w16x3[2][3];
    std::string names[2][2][3], ka[2][3], kc[2][3], k1[2][3], kc16[2][3], ka3[2][3], names3[2][3];
    IoTraitSets() {
        const char* io[2] = {"bf16", "f16"};
        const int nps[3] = {64, 128, 256};
        for (int i = 0; i < 2; ++i)
            for (int k = 0; k < 3; ++k) {
                const std::string np = std::to_string(nps[k]);
                ka[i][k] = std::string("helix_chunk_state_x6agg_") + io[i] + "io_n" + np;
                kc[i][k] = std::string("helix_scan_walk_bf16_") + io[i] + "io_n" + np;
                k1[i][k] = std::string("helix_scan_1pass_") + io[i] + "io_n" + np;
                names[i][0][k] = std::string("mfma bf16 pass C, chunk walk, pass A bf16x6, ") + io[i] +
                                 " storage (d_state<=" + np + ")";
                names[i][1][k] = std::string("mfma fp32, single pass, ") + io[i] + " storage (d_state<=" + np + ")";
                t[i][0][k] = {HELIX_BACKEND_MPP, names[i][0][k].c_str(), ka[i][k].c_str(), "helix_state_scan_f32",
                              kc[i][k].c_str(), true, "v_mfma_f32_32x32x16_bf16 (bf16x6 split operands)",
                              "v_mfma_f32_32x32x16_bf16", nps[k], true, nullptr};
                t[i][1][k] = {HELIX_BACKEND_SGMMA, names[i][1][k].c_str(), nullptr, nullptr, nullptr, false,
                              "v_mfma_f32_16x16x4_f32", "v_mfma_f32_16x16x4_f32", nps[k], false,
                              k1[i][k].c_str()};
                kc16[i][k] = std::string("helix_scan_walk16_bf16_") + io[i] + "io_n" + np;
                w16[i][k] = t[i][0][k];
                w16[i][k].k_chunk_out = kc16[i][k].c_str();
                w16[i][k].mfma_c = "v_mfma_f32_16x16x32_bf16";
                w16[i][k].walk_hpw = HELIX_WALK16_HPW(nps[k]);
                w16[i][k].walk_fuse_b = true;
                w16[i][k].rec_kind = 1;
                ka3[i][k] = std::string("helix_chunk_state_x3agg_") + io[i] + "io_n" + np;
                names3[i][k] = std::string("mfma bf16 pass C, chunk walk, pass A bf16x3, ") + io[i] +
                               " storage (d_state<=" + np + ")";
                w16x3[i][k] = w16[i][k];
                w16x3[i][k].name = names3[i][k].c_str();
                w16x3[i][k].k_chunk_state = ka3[i][k].c_str();
                w16x3[i][k].mfma_a = kMfmaX3;
            }
    }
};

const HelixMatmulTraits& io_traits(helix_dtype io, bool walk, int k) {
    static const IoTraitSets sets;
    if (walk && walk16_on()) return (passa_x3_on() ? sets.w16x3 : sets.w16)[io == HELIX_F16 ? 1 : 0][k];
    return sets.t[io == HELIX_F16 ? 1 : 0][walk ? 0 : 1][k];
}

const char* const kKernelNames[] = {
    "helix_chunk_state_x6f32_n64", "helix_chunk_state_x6f32_n128", "helix_chunk_state_x6f32_n256",
    "helix_chunk_state_x6sbf_n64", "helix_chunk_state_x6sbf_n128", "helix_chunk_state_x6sbf_n256",
    "helix_chunk_state_x6agg_n64", "helix_chunk_state_x6agg_n128", "helix_chunk_state_x6agg_n256",
    "helix_chunk_out_x6_n64",      "helix_chunk_out_x6_n128",
    "helix_chunk_state_f32_n64",  "helix_chunk_state_f32_n128", "helix_chunk_state_f32_n256",
    "helix_chunk_state_sbf_n64",  "helix_chunk_state_sbf_n128", "helix_chunk_state_sbf_n256",
    "helix_state_scan_f32",
    "helix_chunk_out_f32_n64",    "helix_chunk_out_f32_n128",   "helix_chunk_out_f32_n256",
    "helix_chunk_out_bf16_n64",   "helix_chunk_out_bf16_n128",  "helix_chunk_out_bf16_n256",
    "helix_chunk_state_agg_n64",  "helix_chunk_state_agg_n128", "helix_chunk_state_agg_n256",
    "helix_scan_walk_bf16_n64",   "helix_scan_walk_bf16_n128",  "helix_scan_walk_bf16_n256",
    "helix_scan_1pass_f32_n64",   "helix_scan_1pass_f32_n128",  "helix_scan_1pass_f32_n256",
    "helix_scan_1pass_diag_f32_n64", "helix_scan_1pass_diag_f32_n128",
    "helix_chunk_state_x6agg_bf16io_n64", "helix_chunk_state_x6agg_bf16io_n128", "helix_chunk_state_x6agg_bf16io_n256",
    "helix_chunk_state_x6agg_f16io_n64",  "helix_chunk_state_x6agg_f16io_n128",  "helix_chunk_state_x6agg_f16io_n256",
    "helix_scan_walk_bf16_bf16io_n64",    "helix_scan_walk_bf16_bf16io_n128",    "helix_scan_walk_bf16_bf16io_n256",
    "helix_scan_walk_bf16_f16io_n64",     "helix_scan_walk_bf16_f16io_n128",     "helix_scan_walk_bf16_f16io_n256",
    "helix_scan_1pass_bf16io_n64",        "helix_scan_1pass_bf16io_n128",        "helix_scan_1pass_bf16io_n256",
    "helix_scan_1pass_f16io_n64",         "helix_scan_1pass_f16io_n128",         "helix_scan_1pass_f16io_n256",
    "helix_scan_walk16_bf16_n64",         "helix_scan_walk16_bf16_n128",         "helix_scan_walk16_bf16_n256",
    "helix_scan_walk16_bf16_bf16io_n64",  "helix_scan_walk16_bf16_bf16io_n128",  "helix_scan_walk16_bf16_bf16io_n256",
    "helix_scan_walk16_bf16_f16io_n64",   "helix_scan_walk16_bf16_f16io_n128",   "helix_scan_walk16_bf16_f16io_n256",
    "helix_scan_walk16_bf16_bc_n64",      "helix_scan_walk16_bf16_bc_n128",      "helix_scan_walk16_bf16_bc_n256",
    "helix_chunk_state_x6agg_bc_n64",     "helix_chunk_state_x6agg_bc_n128",     "helix_chunk_state_x6agg_bc_n256",
    "helix_chunk_state_x3agg_n64",        "helix_chunk_state_x3agg_n128",        "helix_chunk_state_x3agg_n256",
    "helix_chunk_state_x3agg_bc_n64",     "helix_chunk_state_x3agg_bc_n128",     "helix_chunk_state_x3agg_bc_n256",
    "helix_chunk_state_x3agg_bf16io_n64", "helix_chunk_state_x3agg_bf16io_n128", "helix_chunk_state_x3agg_bf16io_n256",
    "helix_chunk_state_x3agg_f16io_n64",  "helix_chunk_state_x3agg_f16io_n128",  "helix_chunk_state_x3agg_f16io_n256",
};

int np_index(int d_state) {
    if (d_state <= 64) return 0;
    if (d_state <= 128) return 1;
    return 2;
}

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

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

thread_local std::string t_last_error;
thread_local const helix_ctx* t_last_ctx = nullptr;

}  // namespace

namespace helix::rt {

const char* const* all_kernel_names(size_t* count) {
    *count = sizeof(kKernelNames) / sizeof(kKernelNames[0]);
    return kKernelNames;
}

void set_error(const helix_ctx* ctx, const std::string& msg) {
    t_last_ctx = ctx;
    t_last_error = msg;
}

namespace {
bool prefer_walk(const helix_scan_desc& d);
}  // namespace

const HelixMatmulTraits& select_traits(helix_ctx* ctx, const helix_scan_desc& d) {
    (void)ctx;
    const int k = np_index(d.d_state);
    if (d.a_form == HELIX_A_DIAG_PER_CHANNEL) return kDiagTraits[k < 1 ? k : 1];
    if (d.io_dtype != HELIX_F32) {
        const char* f = std::getenv("HELIX_FORCE_BACKEND");
        const bool bf16 = (d.backend == HELIX_BACKEND_AUTO || d.backend == HELIX_BACKEND_MPP) &&
                          !(f && f[0] == 's');
        return io_traits(d.io_dtype, bf16 && d.multipass, k);
    }
    if (!d.multipass) return kSingleTraits[k];
    // HELIX_FORCE_BACKEND=s... pins the fp32 path (reference caps.mm:82-86).
    if (const char* f = std::getenv("HELIX_FORCE_BACKEND"))
        if (f[0] == 's') return pick_traits(0, k, d);
    const bool want_bf16 = d.backend == HELIX_BACKEND_AUTO || d.backend == HELIX_BACKEND_MPP;
    if (want_bf16 && d.multipass) {
        // HELIX_BF16_PASSC=walk|tile overrides the choice between the
        // chunk-walking Pass C (state in registers, no per-chunk scratch) and
        // the chunk-parallel one.
        if (const char* v = std::getenv("HELIX_BF16_PASSC")) {
            if (v[0] == 'w') return pick_traits(2, k, d);
            if (v[0] == 't') return pick_traits(1, k, d);
        }
        return pick_traits(prefer_walk(d) ? 2 : 1, k, d);
    }
    return pick_traits(0, k, d);
}

// The walk's prologue loads up to segs_per_group segment aggregates per
// workgroup, four at a time; past four segments the second round of loads
// costs more than Pass B's own launch (config 2, 8 segments: 149 vs 142 us;
// configs 4a/4b, 4 segments: 701 vs 712 and 767 vs 782 us).
constexpr int kFuseBMaxSegs = 4;

bool fuse_b_on(const HelixMatmulTraits& tr, const MultipassPlan& plan) {
    if (!tr.walk_fuse_b || plan.n_groups != 1) return false;
    if (const char* v = std::getenv("HELIX_FUSE_B")) {
        if (v[0] == '0') return false;
        if (v[0] == '1') return true;
    }
    return plan.segs_per_group <= kFuseBMaxSegs;
}

size_t scratch_budget_bytes() {
    // Default sized for MI355X's 288 GB: a 64-head 8K-token prefill keeps all
    // of its chunks in one group. $HELIX_SCRATCH_MB=1 forces many groups.
    return (size_t)env_long("HELIX_SCRATCH_MB", 2048) << 20;
}

namespace {

// Chunks per segment for a group of `cpg` chunks: enough segments that Pass A
// has ~kTargetWgA workgroups, and no more (a longer walk keeps more of the
// chunk recurrence in registers and shortens Pass B), up to kMaxSegLen (past
// that the walks get too long to fill the chip: at config 4a, 64-chunk
// segments took 1.03 ms and 16-chunk ones 0.95 ms).
constexpr long kMaxSegLen = 16;

int choose_seg_len(const helix_scan_desc& d, int cpg) {
    if (const char* v = std::getenv("HELIX_SEG_LEN")) {
        const long x = std::strtol(v, nullptr, 10);
        if (x > 0) return (int)std::min<long>(x, cpg);
    }
    const long n_pslab = (d.head_dim + HELIX_HD - 1) / HELIX_HD;
    const long items = (long)d.n_seq * d.n_head * n_pslab;
    const long segs = std::max<long>(1, (kTargetWgA + items - 1) / items);
    const long len = std::min<long>((cpg + segs - 1) / segs, kMaxSegLen);
    return (int)std::max<long>(1, std::min<long>(len, cpg));
}

// The bf16 path walks segments in Pass C (no per-chunk state in scratch):
// with the 16 x 16 walk and Pass A's bf16 copies of B and C it is faster
// than the chunk-parallel Pass C at every shape measured, short segments
// included (one MI355X, total scan: config 1 66 vs 72 us, config 2 161 vs
// 211, config 3 89 vs 100, config 4a 786 vs 952, config 4b 859 vs 937; L=512
// 42 vs 48; d_state 256 at L=4096 H=32 G=1 128 vs 146; d_state 64 127 vs
// 135). At d_state 256 it needs the copies: the walk on the caller's B and C
// measured slower there (460 vs 427 us at L=8192 H=64 G=8).
bool prefer_walk(const helix_scan_desc& d) {
    return d.d_state <= 128 || (walk16_on() && bccopy_on(d));
}

void layout(const helix_scan_desc& d, bool bf16_state, bool walk, bool bccopy, bool rec, int np, int cpg,
            MultipassPlan* pl) {
    // State scratch is stored as padded slab tiles of 64 x np (helix_params.h).
    const size_t n_pslab = (size_t)(d.head_dim + HELIX_HD - 1) / HELIX_HD;
    const size_t state = (size_t)d.n_seq * d.n_head * n_pslab * 64 * (size_t)np;
    pl->chunks_per_group = cpg;
    pl->seg_len = choose_seg_len(d, cpg);
    pl->segs_per_group = (cpg + pl->seg_len - 1) / pl->seg_len;
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
    pl->rec_elems = rec ? (size_t)d.n_seq * (size_t)cpg * d.n_head * HELIX_CS * 4 : 0;
    pl->off_rec = off; off += align256(pl->rec_elems * sizeof(float));
    pl->total_bytes = off;
}

}  // namespace

MultipassPlan plan_multipass(const helix_scan_desc& d, const HelixMatmulTraits& tr) {
    const bool bf16_state = tr.bf16_state;
    MultipassPlan pl;
    if (d.n_tok <= 0 || d.n_seq <= 0 || d.n_head <= 0 || d.head_dim <= 0 || d.d_state <= 0 ||
        d.n_group <= 0)
        return pl;
    pl.n_chunks = (d.n_tok + HELIX_CS - 1) / HELIX_CS;

    const size_t budget = scratch_budget_bytes();
    const size_t state = (size_t)d.n_seq * d.n_head * ((d.head_dim + HELIX_HD - 1) / HELIX_HD) * 64 *
                         (size_t)tr.np;
    // A walking Pass C keeps no per-chunk state; only segment aggregates
    // (about one state per seg_len chunks) count against the budget.
    const size_t bc_chunk = tr.bccopy ? (size_t)d.n_seq * HELIX_CS * d.n_group * d.d_state * 2 * 2 : 0;
    const size_t rec_chunk = tr.rec_kind ? (size_t)d.n_seq * d.n_head * HELIX_CS * 16 : 0;
    const size_t per_chunk = (tr.walk ? state : state * (bf16_state ? 2 : 4)) + bc_chunk + rec_chunk;
    long cpg = per_chunk ? (long)(budget / per_chunk) : 1;
    cpg = std::max<long>(1, std::min<long>(cpg, pl.n_chunks));
    for (;;) {
        layout(d, bf16_state, tr.walk, tr.bccopy, tr.rec_kind != 0, tr.np, (int)cpg, &pl);
        if (pl.total_bytes <= budget || cpg == 1) break;
        cpg = std::max<long>(1, cpg - std::max<long>(1, cpg / 8));
    }
    pl.n_groups = (pl.n_chunks + pl.chunks_per_group - 1) / pl.chunks_per_group;

    // Pass C head blocks: share C.B^T over as many heads as possible while
    // keeping ~kTargetWgC workgroups per group launch.
    const int hpg = d.n_head / std::max(1, d.n_group);
    const long base = (long)d.n_seq * pl.chunks_per_group * d.n_group;
    long want_blocks = std::max<long>(1, (kTargetWgC + base - 1) / base);
    if (const char* v = std::getenv("HELIX_HBLK")) {
        const long x = std::strtol(v, nullptr, 10);
        if (x > 0) want_blocks = (hpg + x - 1) / x;
    }
    want_blocks = std::min<long>(want_blocks, hpg);
    pl.hblk = (int)((hpg + want_blocks - 1) / want_blocks);
    pl.n_hblk = (hpg + pl.hblk - 1) / pl.hblk;
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
    if (d.n_head > kMaxYZ || zA > kMaxYZ || d.n_seq > kMaxYZ || (long)d.n_head > kMaxYZ) {
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
    if (d->d_state > HELIX_N_MAX) return false;
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
    if (helix::rt::select_traits(ctx, *d).k_single) return 0;
    return helix::rt::plan_multipass(*d, helix::rt::select_traits(ctx, *d)).total_bytes;
}

extern "C" helix_backend helix_ctx_select_backend(helix_ctx* ctx, const helix_scan_desc* d) {
    if (!ctx || !d) return HELIX_BACKEND_REF;
    if (d->backend == HELIX_BACKEND_SGMMA) return HELIX_BACKEND_SGMMA;
    return helix::rt::select_traits(ctx, *d).backend;
}

extern "C" const char* helix_ctx_backend_desc(helix_ctx* ctx, const helix_scan_desc* d) {
    if (!ctx || !d) return "unavailable (null context)";
    if (!helix_scan_supported(ctx, d)) return "declined (shape unsupported)";
    return helix::rt::select_traits(ctx, *d).name;
}
