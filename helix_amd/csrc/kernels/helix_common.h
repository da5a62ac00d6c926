// helix_common.h -- device helpers shared by the gfx950 HELIX kernels.
//
// Wave64 conventions used throughout:
//   lane = threadIdx.x & 63, wave = threadIdx.x >> 6 (4 waves per workgroup)
//   lo = lane & 31, hi = lane >> 5
//
// MFMA operand/result layouts (CDNA3/CDNA4 ISA):
//   v_mfma_f32_32x32x2_f32   A[i][k]: lane holds A[lo][hi]
//                            B[k][j]: lane holds B[hi][lo]
//                            D[i][j]: lane, reg r holds D[8*(r/4) + 4*hi + r%4][lo]
//   v_mfma_f32_32x32x16_bf16 A[i][k]: lane holds A[lo][8*hi + e], e = 0..7
//                            B[k][j]: lane holds B[8*hi + e][lo]
//                            D as above
// Every kernel output depends on these layouts, so the device parity suite
// (tests/test_gpu_parity.py) checks them end to end.
#ifndef HELIX_COMMON_H
#define HELIX_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "helix_params.h"

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

#define HELIX_DEV static __device__ __forceinline__

HELIX_DEV int lane_id() { return threadIdx.x & 63; }
HELIX_DEV int wave_id() { return threadIdx.x >> 6; }

// softplus with the v > 20 shortcut the reference and ggml use
// (reference src/kernels/helix_common.h:14-16). log1p keeps full relative
// precision for the strongly negative dt of long-memory models. Both sides are
// formed and one selected (the log1p side on min(v, 20), so it is the same
// value as before for every v <= 20): a branch here would split the chunk loops
// that form the decay preamble among their MFMAs.
HELIX_DEV float helix_softplus(float v) {
    const float s = log1pf(expf(fminf(v, 20.0f)));
    return v > 20.0f ? v : s;
}

HELIX_DEV float helix_dt(const HelixScanParams& p, float raw) {
    return fminf(fmaxf(helix_softplus(raw), p.dt_min), p.dt_max);
}

// Lane-shifted copy of a double by a DPP move on each 32-bit half; lanes
// without a source (and rows outside ROW_MASK) receive 0.
template <int CTRL, int ROW_MASK>
HELIX_DEV double dpp_f64(double v) {
    const long long u = __builtin_bit_cast(long long, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)u, CTRL, ROW_MASK, 0xf, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(u >> 32), CTRL, ROW_MASK, 0xf, true);
    return __builtin_bit_cast(double, ((long long)hi << 32) | (unsigned int)lo);
}

// Inclusive prefix sum over the 64 lanes of a wave, in fp64: the intra-chunk
// decays are exp(Lcum_t - Lcum_j), and with |A*dt| summing to a few hundred
// per chunk an fp32 prefix would lose the low digits that the difference of
// two nearby prefixes needs. Six DPP steps, no LDS: row_shr 1, 2, 4, 8 scan
// each row of 16 lanes; row_bcast:15 adds row 0's total to row 1 and row 2's
// to row 3; row_bcast:31 adds the total of rows 0-1 to rows 2 and 3.
HELIX_DEV double wave_incl_sum(double v) {
    v += dpp_f64<0x111, 0xf>(v);   // row_shr:1
    v += dpp_f64<0x112, 0xf>(v);   // row_shr:2
    v += dpp_f64<0x114, 0xf>(v);   // row_shr:4
    v += dpp_f64<0x118, 0xf>(v);   // row_shr:8
    v += dpp_f64<0x142, 0xa>(v);   // row_bcast:15 -> rows 1, 3
    v += dpp_f64<0x143, 0xc>(v);   // row_bcast:31 -> rows 2, 3
    return v;
}

// Per-chunk decay preamble, computed redundantly by every wave so no LDS or
// barrier is needed: lane t owns token t of the chunk.
//   dtv  = clamp(softplus(dt_t))          (0 for t >= tlen)
//   lcum = sum_{j<=t} A_h * dtv_j         fp64; A_h*dtv is exact in fp64.
//                                         Constant past tlen since dtv = 0.
//   lend = lcum at the chunk's last token
// Padded rows therefore carry Lcum[tlen-1], which keeps every intra-chunk
// exponent Lcum_t - Lcum_j <= 0 for j <= t (reference helix_common.h:110-120).
struct ChunkDecay {
    float  dtv;
    double lcum;
    double lend;
};

HELIX_DEV ChunkDecay chunk_decay(const HelixScanParams& p, const float* __restrict__ dt_h,
                                 int t0, int tlen, float A_h) {
    const int lane = lane_id();
    ChunkDecay r;
    r.dtv = 0.0f;
    if (lane < tlen) r.dtv = helix_dt(p, dt_h[(long long)(t0 + lane) * p.s_dt[0]]);
    r.lcum = wave_incl_sum((double)A_h * (double)r.dtv);
    r.lend = __shfl(r.lcum, 63, 64);
    return r;
}

// exp of a (small, non-positive in practice) fp64 log-decay difference.
HELIX_DEV float exp_diff(double a, double b) { return expf((float)(a - b)); }

// The same through the hardware base-2 exponential (v_exp_f32, about 1 ulp):
// the difference is scaled by log2(e) in fp64, so the only fp32 rounding
// before the exponential is that of the final argument.
HELIX_DEV float exp2_diff(double a, double b) {
    return __builtin_amdgcn_exp2f((float)((a - b) * 1.4426950408889634074));
}

// MI355X hands the workgroups of a launch to its 8 XCDs round-robin (linear
// id i runs on XCD i % 8), and each XCD has its own L2. This maps the linear
// id to a logical id so that a contiguous run of logical ids shares one XCD:
// work items that read the same data (chunks of one segment, heads of one
// group) then share an L2 instead of each XCD fetching its own copy.
// A bijection on [0, total); the ragged tail past a multiple of 8 is kept.
HELIX_DEV unsigned xcd_logical_id(unsigned linear, unsigned total) {
    constexpr unsigned kXcd = 8;
    const unsigned per = total / kXcd;
    if (linear >= per * kXcd) return linear;
    return (linear % kXcd) * per + linear / kXcd;
}

// Wave-uniform broadcast of lane `src`'s value (src must be wave-uniform).
// Call it where every lane executes (never inside a divergent branch or one
// arm of a divergent ?:): under a partial exec mask the compiler may read the
// lane from a register copy that was only written for the active lanes.
HELIX_DEV float bcast(float v, int src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}
HELIX_DEV double bcast(double v, int src) {
    const long long u = __builtin_bit_cast(long long, v);
    const int lo32 = __builtin_amdgcn_readlane((int)(u & 0xffffffffLL), src);
    const int hi32 = __builtin_amdgcn_readlane((int)(u >> 32), src);
    return __builtin_bit_cast(double, ((long long)hi32 << 32) | (unsigned int)lo32);
}

HELIX_DEV f32x16 mfma_f32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

HELIX_DEV f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Row of MFMA result register r for this lane (column is lo).
HELIX_DEV int acc_row(int r, int hi) { return 8 * (r >> 2) + 4 * hi + (r & 3); }

HELIX_DEV f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.0f;
    return z;
}

// Offset of one head's slab tile in the state scratch (see helix_params.h).
HELIX_DEV long long state_tile_off(const HelixScanParams& p, int h, int slab) {
    return ((long long)h * p.n_pslab + slab) * (long long)(64 * p.np);
}

// Slab tile layout (helix_params.h): 16-byte (fp32) or 8-byte (bf16) units of
// four consecutive state indices n for one p, in the order of the MFMA result
// registers of R[n][p] (M = n, N = p):
//   unit(pt, nt, r4, lane) = ((pt * NT + nt) * 4 + r4) * 64 + lane
//   holds p = pt*32 + lane%32, n = nt*32 + 8*r4 + 4*(lane/32) + 0..3,
// i.e. result registers 4 r4 .. 4 r4 + 3 of tile (nt, pt).
HELIX_DEV int tile_unit(int NT, int pt, int nt, int r4, int lane) {
    return ((pt * NT + nt) * 4 + r4) * 64 + lane;
}

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
HELIX_DEV __bf16 to_bf16(float v) { return (__bf16)v; }

// a * b with 0 * x = 0 for every x, NaN and infinity included
// (v_mul_legacy_f32); otherwise the IEEE product. For a weight that is exactly
// zero on padding rows whose loaded value is not under the kernel's control.
HELIX_DEV float mul_legacy(float a, float b) {
    float r;
    asm("v_mul_legacy_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// Raw buffer access. The resource (base and byte range) sits in four SGPRs,
// the lane's byte offset is one 32-bit VGPR, and a compile-time byte offset
// goes to the instruction's soffset/immediate fields, so a run of loads from
// one wave-uniform region costs no per-load address VGPRs (flat/global loads
// need a 64-bit VGPR address each once offsets exceed the 4 KiB immediate).
// `base` must be wave-uniform. Raw buffer range checking (stride 0) returns 0
// for a read at or past `bytes` and drops such a write; the checked offset is
// the lane's offset plus the scalar offset (measured on gfx950: a read whose
// scalar offset alone passes the range returns 0).
typedef __amdgpu_buffer_rsrc_t helix_rsrc;

HELIX_DEV helix_rsrc make_rsrc(const void* base, unsigned bytes) {
    // Dword 3 = 0x00020000: DATA_FORMAT 32, the value gfx9-family untyped
    // buffer instructions are used with.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// The same with the base and range read from the first active lane: for a
// resource built from values the compiler cannot prove wave-uniform (a select
// on a wave-uniform flag, for one), which it would otherwise address through a
// waterfall loop around every access.
HELIX_DEV helix_rsrc make_rsrc_u(const void* base, unsigned bytes) {
    const unsigned long long a = reinterpret_cast<unsigned long long>(base);
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)a);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32));
    return make_rsrc(reinterpret_cast<const void*>(((unsigned long long)hi << 32) | lo),
                     __builtin_amdgcn_readfirstlane(bytes));
}
HELIX_DEV float buf_f32(helix_rsrc r, int voff, int soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
HELIX_DEV __bf16 buf_bf16(helix_rsrc r, int voff, int soff) {
    return __builtin_bit_cast(__bf16, __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0));
}
// Element load from a buffer of T (float or __bf16); offsets in elements.
template <typename T>
HELIX_DEV T buf_elem(helix_rsrc r, int vidx, int sidx) {
    if constexpr (sizeof(T) == 4)
        return buf_f32(r, vidx * 4, sidx * 4);
    else
        return buf_bf16(r, vidx * 2, sidx * 2);
}
// Bit casts through a by-value parameter. __builtin_bit_cast applied in place
// to an element of an ext_vector_type lvalue (v[k]) reads element 0 with this
// compiler; passing the element as an argument makes it a plain value first.
HELIX_DEV float as_f32(unsigned v) { return __builtin_bit_cast(float, v); }
HELIX_DEV unsigned as_u32(float v) { return __builtin_bit_cast(unsigned, v); }

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// One tile unit (four state values) as fp32, from an fp32 or bf16 tile.
// `unit` is the unit index; bf16 units are 8 bytes, fp32 units 16.
template <typename T>
HELIX_DEV f32x4 buf_unit(helix_rsrc r, int vunit, int sunit) {
    f32x4 o;
    if constexpr (sizeof(T) == 4) {
        o = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, vunit * 16, sunit * 16, 0));
    } else {
        const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(r, vunit * 8, sunit * 8, 0);
        o[0] = __builtin_bit_cast(float, w[0] << 16);
        o[1] = __builtin_bit_cast(float, w[0] & 0xffff0000u);
        o[2] = __builtin_bit_cast(float, w[1] << 16);
        o[3] = __builtin_bit_cast(float, w[1] & 0xffff0000u);
    }
    return o;
}
// Raw 16-byte unit of an fp32 tile or 8-byte unit of a bf16 tile, kept as
// loaded (no conversion, so the load has no consumer until it is used).
template <typename T> struct RawUnit { typedef u32x4 type; };
template <> struct RawUnit<__bf16> { typedef u32x2 type; };

template <typename T>
HELIX_DEV typename RawUnit<T>::type buf_unit_raw(helix_rsrc r, int vunit, int sunit) {
    if constexpr (sizeof(T) == 4)
        return __builtin_amdgcn_raw_buffer_load_b128(r, vunit * 16, sunit * 16, 0);
    else
        return __builtin_amdgcn_raw_buffer_load_b64(r, vunit * 8, sunit * 8, 0);
}
HELIX_DEV f32x4 unit_to_f32(u32x4 w) { return __builtin_bit_cast(f32x4, w); }
HELIX_DEV f32x4 unit_to_f32(u32x2 w) {
    f32x4 o;
    o[0] = __builtin_bit_cast(float, w[0] << 16);
    o[1] = __builtin_bit_cast(float, w[0] & 0xffff0000u);
    o[2] = __builtin_bit_cast(float, w[1] << 16);
    o[3] = __builtin_bit_cast(float, w[1] & 0xffff0000u);
    return o;
}

// Store four values as one tile unit of T (fp32: 16 bytes; bf16: rounded,
// 8 bytes). Values go in by value: a bit cast of a vector element in place
// reads element 0 with this compiler.
template <typename T>
HELIX_DEV void buf_store_unit(helix_rsrc r, float v0, float v1, float v2, float v3, int vunit, int sunit) {
    if constexpr (sizeof(T) == 4) {
        u32x4 w;
        w[0] = __builtin_bit_cast(unsigned, v0);
        w[1] = __builtin_bit_cast(unsigned, v1);
        w[2] = __builtin_bit_cast(unsigned, v2);
        w[3] = __builtin_bit_cast(unsigned, v3);
        __builtin_amdgcn_raw_buffer_store_b128(w, r, vunit * 16, sunit * 16, 0);
    } else {
        u32x2 w;
        w[0] = (unsigned)__builtin_bit_cast(unsigned short, to_bf16(v0)) |
               ((unsigned)__builtin_bit_cast(unsigned short, to_bf16(v1)) << 16);
        w[1] = (unsigned)__builtin_bit_cast(unsigned short, to_bf16(v2)) |
               ((unsigned)__builtin_bit_cast(unsigned short, to_bf16(v3)) << 16);
        __builtin_amdgcn_raw_buffer_store_b64(w, r, vunit * 8, sunit * 8, 0);
    }
}

// ---- bf16x6: fp32 values as three bf16 parts --------------------------------
// v = v0 + v1 + v2 with v0 = bf16(v), v1 = bf16(v - v0), v2 = bf16(v - v0 - v1)
// (round to nearest even; each residual is exact in fp32 and the three 8-bit
// significands cover fp32's 24). A product a.b accumulated from the six terms
// a0 b0 + a0 b1 + a1 b0 + a0 b2 + a1 b1 + a2 b0 is accurate to about 2^-24
// relative: the dropped terms are below that (bf16x6 in Henry, Tang,
// Heinecke, "Leveraging the bfloat16 Artificial Intelligence Datatype For
// Higher-Precision Computations", ARITH 2019).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Round-to-nearest-even bf16 pair (element 0 in the low half), one
// v_cvt_pk_bf16_f32, and its exact fp32 values.
HELIX_DEV unsigned pk_bf16(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf16x2));
}
HELIX_DEV float pk_lo(unsigned w) { return __builtin_bit_cast(float, w << 16); }
HELIX_DEV float pk_hi(unsigned w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// a - lo(w) and a - hi(w) for a packed bf16 pair w, each one v_dot2_f32_bf16:
// w . (-1, 0) + a. Where w is a's own bf16 rounding (or that of a residual of
// it) the difference is exactly representable in fp32, and the bf16 products
// are exact, so the result is exact: the same value as unpacking the half and
// subtracting, in one operation instead of two. The (-1, 0) and (0, -1) pairs
// reach the instruction in a scalar register: the compiler would otherwise
// encode the first as the inline constant -1.0, which the hardware applies as
// the fp32 bit pattern 0xbf800000, i.e. the pair (0, -1) (measured).
HELIX_DEV unsigned bf16_pair_reg(unsigned k) {
    asm("" : "+s"(k));
    return k;
}
HELIX_DEV float sub_lo(float a, unsigned w) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w),
                                           __builtin_bit_cast(bf16x2, bf16_pair_reg(0x0000bf80u)), a, false);
}
HELIX_DEV float sub_hi(float a, unsigned w) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w),
                                           __builtin_bit_cast(bf16x2, bf16_pair_reg(0xbf800000u)), a, false);
}

// Three-way bf16 split of the pair (a, b), each part packed as a pair:
// 7 VALU operations for two values.
HELIX_DEV void split3_pair(float a, float b, unsigned& w0, unsigned& w1, unsigned& w2) {
    w0 = pk_bf16(a, b);
    const float ra = sub_lo(a, w0), rb = sub_hi(b, w0);
    w1 = pk_bf16(ra, rb);
    w2 = pk_bf16(sub_lo(ra, w1), sub_hi(rb, w1));
}

// Two-way bf16 split of the pair (a, b): v = v0 + v1 + e with |e| <= 2^-18 |v|,
// 4 VALU operations for two values. Three products a0b0 + a0b1 + a1b0 leave
// out terms of at most 3 * 2^-18 of |ab| (about 1.1e-5).
HELIX_DEV void split2_pair(float a, float b, unsigned& w0, unsigned& w1) {
    w0 = pk_bf16(a, b);
    w1 = pk_bf16(sub_lo(a, w0), sub_hi(b, w0));
}

// Six-product MFMA of split operands a[3] x b[3], smallest terms first.
HELIX_DEV f32x16 mfma_x6(const bf16x8 (&a)[3], const bf16x8 (&b)[3], f32x16 acc) {
    acc = mfma_bf16(a[2], b[0], acc);
    acc = mfma_bf16(a[1], b[1], acc);
    acc = mfma_bf16(a[0], b[2], acc);
    acc = mfma_bf16(a[1], b[0], acc);
    acc = mfma_bf16(a[0], b[1], acc);
    acc = mfma_bf16(a[0], b[0], acc);
    return acc;
}

// Split planes in LDS: [3][ROWS][NCH * 8] bf16, rows of NCH 16-byte chunks,
// chunk c of row r stored at chunk position c ^ f(r):
//   NCH = 8  (128-byte rows): f(r) = ((r >> 1) ^ (r >> 4)) & 7. Row bases
//            alternate between two bank halves; over 16 consecutive rows f
//            takes every value once per parity, and over rows 4l + k
//            (l < 16) every value twice.
//   NCH = 16 (256-byte rows, all starting at bank 0): f(r) = r & 15.
// Either way the 16-byte reads of an MFMA operand (16 consecutive rows, one
// chunk each) cover all 64 banks once per 16 lanes.
template <int ROWS, int NCH>
HELIX_DEV int x6_off(int k, int r, int c) {
    static_assert(NCH == 8 || NCH == 16, "rows of 8 or 16 chunks");
    const int f = NCH == 8 ? (((r >> 1) ^ (r >> 4)) & 7) : (r & 15);
    return ((k * ROWS + r) * NCH + (c ^ f)) * 8;
}

// The three planes' chunk c of row r, as MFMA operands.
template <int ROWS, int NCH>
HELIX_DEV void x6_read(const __bf16* planes, int r, int c, bf16x8 (&o)[3]) {
#pragma unroll
    for (int k = 0; k < 3; ++k) o[k] = *reinterpret_cast<const bf16x8*>(&planes[x6_off<ROWS, NCH>(k, r, c)]);
}

// Split eight fp32 values and store them as chunk c of row r (three planes).
template <int ROWS, int NCH>
HELIX_DEV void x6_write8(__bf16* planes, int r, int c, const float* v) {
    u32x4 q0, q1, q2;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        unsigned w0, w1, w2;
        split3_pair(v[2 * e], v[2 * e + 1], w0, w1, w2);
        q0[e] = w0;
        q1[e] = w1;
        q2[e] = w2;
    }
    *reinterpret_cast<u32x4*>(&planes[x6_off<ROWS, NCH>(0, r, c)]) = q0;
    *reinterpret_cast<u32x4*>(&planes[x6_off<ROWS, NCH>(1, r, c)]) = q1;
    *reinterpret_cast<u32x4*>(&planes[x6_off<ROWS, NCH>(2, r, c)]) = q2;
}

// Eight fp32 values as the three split planes of one MFMA operand.
HELIX_DEV void x6_split8(const float (&v)[8], bf16x8 (&o)[3]) {
    u32x4 q0, q1, q2;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        unsigned w0, w1, w2;
        split3_pair(v[2 * e], v[2 * e + 1], w0, w1, w2);
        q0[e] = w0;
        q1[e] = w1;
        q2[e] = w2;
    }
    o[0] = __builtin_bit_cast(bf16x8, q0);
    o[1] = __builtin_bit_cast(bf16x8, q1);
    o[2] = __builtin_bit_cast(bf16x8, q2);
}

// LDS transpose read of 16-bit elements (ds_read_b64_tr_b16): every lane
// names 8 bytes (four elements); lane l of each 16-lane group receives, as
// element r (r = 0..3), element l % 4 of the 8 bytes named by lane
// 4 r + l / 4 of its group. With lane 4 r + q naming row k_r, columns
// c0 + 4 q .. c0 + 4 q + 3 of a row-major array, lane l gets column c0 + l of
// rows k_0 .. k_3: a K-major operand read from rows that run along the other
// index.
typedef short i16x4 __attribute__((ext_vector_type(4)));
HELIX_DEV u32x2 lds_read_tr16(const __bf16* p) {
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)p);
    return __builtin_bit_cast(u32x2, v);
}

// Split eight fp32 values v[0..7] into NS bf16 planes (NS = 3: split3_pair,
// NS = 2: split2_pair) and store them as chunk c of row r.
template <int ROWS, int NS>
HELIX_DEV void stage_split8(__bf16* planes, int r, int c, const float* v) {
    u32x4 q[NS];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        unsigned w[3];
        if constexpr (NS == 3)
            split3_pair(v[2 * e], v[2 * e + 1], w[0], w[1], w[2]);
        else
            split2_pair(v[2 * e], v[2 * e + 1], w[0], w[1]);
#pragma unroll
        for (int k = 0; k < NS; ++k) q[k][e] = w[k];
    }
#pragma unroll
    for (int k = 0; k < NS; ++k) *reinterpret_cast<u32x4*>(&planes[x6_off<ROWS, 8>(k, r, c)]) = q[k];
}

// Raw-register form of an element of T: a float stays a float, a bf16 stays
// its 16 bits zero-extended in a 32-bit register. Loads into this form carry
// no data dependence (nothing packs two 16-bit results into one register), so
// a run of prefetch loads stays in flight until the value is used.
template <typename T> struct RawReg { typedef float type; };
template <> struct RawReg<__bf16> { typedef unsigned type; };

template <typename T>
HELIX_DEV typename RawReg<T>::type buf_raw(helix_rsrc r, int vidx, int sidx) {
    if constexpr (sizeof(T) == 4)
        return buf_f32(r, vidx * 4, sidx * 4);
    else
        return (unsigned)__builtin_amdgcn_raw_buffer_load_b16(r, vidx * 2, sidx * 2, 0);
}
HELIX_DEV float raw_to_f32(float v) { return v; }
HELIX_DEV float raw_to_f32(unsigned bits) { return __builtin_bit_cast(float, bits << 16); }

// ---- caller storage types (helix_scan_desc.io_dtype) --------------------------
// x, B, C and y are stored as IO = float, __bf16 or _Float16; dt, A and the
// states are always fp32. Loads widen to fp32 exactly; stores round to
// nearest even. Offsets are in elements.
template <typename IO>
HELIX_DEV float io_f32(unsigned short bits) {
    if constexpr (__is_same(IO, __bf16))
        return __builtin_bit_cast(float, (unsigned)bits << 16);
    else
        return (float)__builtin_bit_cast(_Float16, bits);
}
template <typename IO>
HELIX_DEV float io_load(helix_rsrc r, int vidx, int sidx) {
    if constexpr (sizeof(IO) == 4)
        return buf_f32(r, vidx * 4, sidx * 4);
    else
        return io_f32<IO>(__builtin_bit_cast(unsigned short,
                                             __builtin_amdgcn_raw_buffer_load_b16(r, vidx * 2, sidx * 2, 0)));
}
// An element kept in its storage form from its load to its use: fp32 stays a
// float, a 16-bit type stays its loaded bits until io_widen. A loader that
// widened at the load would make each load's consumer the next instruction,
// and the loads would wait for each other one by one.
template <typename IO> struct IoWord { typedef float type; };
template <> struct IoWord<__bf16> { typedef unsigned type; };
template <> struct IoWord<_Float16> { typedef unsigned type; };
template <typename IO>
HELIX_DEV typename IoWord<IO>::type io_load_word(helix_rsrc r, int vidx, int sidx) {
    if constexpr (sizeof(IO) == 4)
        return buf_f32(r, vidx * 4, sidx * 4);
    else
        return (unsigned)__builtin_bit_cast(unsigned short,
                                            __builtin_amdgcn_raw_buffer_load_b16(r, vidx * 2, sidx * 2, 0));
}
template <typename IO>
HELIX_DEV float io_widen(typename IoWord<IO>::type w) {
    if constexpr (sizeof(IO) == 4)
        return w;
    else
        return io_f32<IO>((unsigned short)w);
}
// Cache policy of a buffer access (the instruction's aux operand, gfx950 bits:
// 1 sc0, 2 nt, 16 sc1): 0 is the default. y is written once and never read
// back by the scan, so its stores carry HELIX_NT = nt | sc1: non-temporal,
// which keeps y from displacing the inputs still being read (15-25% faster
// than the default on the walking Pass C at config 2), at device scope, which
// measured a further 5% on the walks (bf16 61.1 -> 58.3 us, fp32 155.5 ->
// 147.9 us at config 2). The walk that reads Pass A's bf16 copies of B and C
// (many heads per group, all reading the copies through L2) stores with nt
// alone, HELIX_NT_L2: there the device-scope bit cost 7% (config 4a walk
// 342 -> 366 us; 4b unchanged). sc1 without nt, or with sc0, measured slower
// than the default; the same bits on loads or on the scratch stores gave
// nothing.
#define HELIX_NT 18
#define HELIX_NT_L2 2
template <typename IO, int AUX = 0>
HELIX_DEV void io_store(helix_rsrc r, float v, int voff_bytes, int soff_bytes) {
    if constexpr (sizeof(IO) == 4) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, voff_bytes, soff_bytes, AUX);
    } else {
        const IO h = (IO)v;
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, h), r, voff_bytes, soff_bytes,
                                              AUX);
    }
}
// One element of y at (voff, soff) of resource r: stored with HELIX_NT, or,
// with ACC (HelixScanParams::y_acc: fp32 storage, the second and later blocks
// of state indices of a d_state above HELIX_N_MAX), added to the value y
// holds first. Callers test y_acc once around a run of stores
// (with_y_acc), so the common path has no branch per store.
// 16-bit y is stored with nt alone: with the device-scope bit its 2-byte
// stores made the bf16-storage walk 67% slower (config 2: 51 -> 86 us).
template <typename IO, bool ACC, int AUX = HELIX_NT>
HELIX_DEV void y_store(helix_rsrc r, float v, int voff_bytes, int soff_bytes) {
    if constexpr (ACC && sizeof(IO) == 4)
        v += __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff_bytes, soff_bytes, 0));
    io_store<IO, sizeof(IO) == 4 ? AUX : HELIX_NT_L2>(r, v, voff_bytes, soff_bytes);
}
// f(std::bool_constant<p.y_acc>{}).
template <typename F>
HELIX_DEV void with_y_acc(const HelixScanParams& p, F&& f) {
    if (p.y_acc)
        f(std::true_type{});
    else
        f(std::false_type{});
}
// Eight consecutive elements starting at byte offset voff, widened to fp32:
// two 16-byte loads for fp32, one for 16-bit storage.
template <typename IO>
HELIX_DEV void io_load8(helix_rsrc r, int voff, float (&o)[8]) {
    if constexpr (sizeof(IO) == 4) {
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
        const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            o[e] = as_f32(a[e]);
            o[4 + e] = as_f32(b[e]);
        }
    } else {
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const unsigned w = a[e];
            o[2 * e] = io_f32<IO>((unsigned short)(w & 0xffffu));
            o[2 * e + 1] = io_f32<IO>((unsigned short)(w >> 16));
        }
    }
}

// Element store of v, as T (float, or rounded to __bf16); offsets in elements.
template <typename T>
HELIX_DEV void buf_store_elem(helix_rsrc r, float v, int vidx, int sidx) {
    if constexpr (sizeof(T) == 4)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, vidx * 4, sidx * 4, 0);
    else
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, to_bf16(v)), r, vidx * 2,
                                              sidx * 2, 0);
}

// Branch- and mask-free selects. A compare feeding a select or a guarded
// store is a 64-bit lane mask in SGPRs; when the compare is loop-invariant
// the optimizer hoists it and keeps the masks of every row live across the
// loop. These forms keep the condition in a VGPR instead.
//   keep_if_le(v, a, b)  = a <= b ? v : 0.0f
HELIX_DEV float keep_if_le(float v, int a, int b) {
    const unsigned m = (unsigned)((b - a) >> 31);          // all ones iff a > b
    return __builtin_bit_cast(float, __builtin_bit_cast(unsigned, v) & ~m);
}
//   pick_hi(a, b, hi) = hi ? b : a, as a bitwise select (hi is 0 or 1)
HELIX_DEV double pick_hi(double a, double b, int hi) {
    const unsigned long long m = 0ull - (unsigned long long)hi;
    const unsigned long long ua = __builtin_bit_cast(unsigned long long, a);
    const unsigned long long ub = __builtin_bit_cast(unsigned long long, b);
    return __builtin_bit_cast(double, (ua & ~m) | (ub & m));
}
//   keep_if_lt2(v, a, la, b, lb) = (a < la && b < lb) ? v : 0.0f
HELIX_DEV float keep_if_lt2(float v, int a, int la, int b, int lb) {
    const unsigned bad = (unsigned)(((la - 1 - a) | (lb - 1 - b)) >> 31);
    return __builtin_bit_cast(float, __builtin_bit_cast(unsigned, v) & ~bad);
}
//   keep_if_lt(v, a, la) = a < la ? v : 0.0f
HELIX_DEV float keep_if_lt(float v, int a, int la) {
    const unsigned bad = (unsigned)((la - 1 - a) >> 31);
    return __builtin_bit_cast(float, __builtin_bit_cast(unsigned, v) & ~bad);
}
// Byte offset for a raw buffer store, or one past any range (>= 2^31, which
// the resource's range check drops) when the lane's element is not valid.
// valid iff a < la && b < lb.
HELIX_DEV int store_off_if_lt(int off, int a, int la, int b, int lb) {
    const unsigned bad = (unsigned)(((la - 1 - a) | (lb - 1 - b)) >> 31);   // all ones iff invalid
    return (int)((unsigned)off | (bad & 0x80000000u));
}

// A wave-uniform value the optimizer must treat as produced here. Applied to a
// stride inside a loop, it keeps the products formed from it (one per row of
// a staged tile) from being hoisted out of the loop as dozens of SGPRs that
// stay live across it and spill; they are recomputed by the scalar unit
// instead, which costs no vector issue slots.
HELIX_DEV int sgpr_fresh(int v) {
    asm volatile("" : "+s"(v));
    return v;
}

// The same for a per-lane value: expressions built on it inside a loop are
// recomputed there instead of being hoisted out as dozens of loop-invariant
// VGPRs (one per unrolled load address) that would stay live across the loop.
HELIX_DEV int vgpr_fresh(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Load of a wave-uniform element through the scalar unit (s_load, counted by
// lgkmcnt): reading through the constant address space tells the compiler the
// data does not change during the kernel (an input, or what an earlier launch
// wrote). A vector load would join the in-order vmcnt queue, so waiting for
// it would also wait for every load issued before it.
HELIX_DEV float sload_f32(const float* p, long long i) {
    return ((const __attribute__((address_space(4))) float*)p)[i];
}
HELIX_DEV int sload_i32(const int* p, long long i) {
    return ((const __attribute__((address_space(4))) int*)p)[i];
}

// This thread's wave index, as a wave-uniform (SGPR) value: everything derived
// from it (row offsets, branch conditions) then stays scalar.
HELIX_DEV int wave_uniform() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// The decay record of token t = lane of chunk c (group-local) of head h, as
// the walking Pass C uses it: {dt_t, Lcum_t log2(e)} (HELIX_REC_WALK_BYTES),
// with dt zero past tlen (padded tokens carry Lcum_{tlen-1}). Pass A forms
// dt_t and Lcum_t (fp64) for its own GEMM; storing them once per (seq, chunk,
// head) spares the walk's four waves per head recomputing the softplus and the
// fp64 scan every chunk. The walk forms exp(L_end - Lcum_t), exp(Lcum_t) and
// exp(L_end) from the fp32 log2 values with v_exp_f32 (Lcum_63 = L_end): a
// few ulps of a value that then rounds to a bf16 operand, for half the bytes
// of storing the exponentials too.
HELIX_DEV u32x2 walk_record(float dtv, double lcum) {
    return u32x2{__builtin_bit_cast(unsigned, dtv), __builtin_bit_cast(unsigned, (float)(lcum * 1.4426950408889634074))};
}
HELIX_DEV void store_decay_record(const HelixScanParams& p, const HelixScanBuffers& b, int seq, int c, int h,
                                  int lane, float dtv, double lcum) {
    const char* rec = reinterpret_cast<const char*>(b.pre) +
                      (((long long)seq * p.cpg + c) * p.n_head + h) * (HELIX_CS * HELIX_REC_WALK_BYTES);
    const helix_rsrc r = make_rsrc(rec, HELIX_CS * HELIX_REC_WALK_BYTES);
    __builtin_amdgcn_raw_buffer_store_b64(walk_record(dtv, lcum), r, lane * HELIX_REC_WALK_BYTES, 0, 0);
}

// The fp32 path's form of the record (its Pass C forms the intra-chunk decays
// from fp64 differences of Lcum): {dt_t, exp(Lcum_t), Lcum_t as fp64}.
HELIX_DEV void store_decay_record64(const HelixScanParams& p, const HelixScanBuffers& b, int seq, int c, int h,
                                    int lane, float dtv, double lcum) {
    const float e = expf((float)lcum);
    const unsigned long long u = __builtin_bit_cast(unsigned long long, lcum);
    const float* rec = b.pre + (((long long)seq * p.cpg + c) * p.n_head + h) * (HELIX_CS * 4);
    const helix_rsrc r = make_rsrc(rec, HELIX_CS * 16u);
    const u32x4 w = {__builtin_bit_cast(unsigned, dtv), __builtin_bit_cast(unsigned, e), (unsigned)u,
                     (unsigned)(u >> 32)};
    __builtin_amdgcn_raw_buffer_store_b128(w, r, lane * 16, 0, 0);
}

// The single pass run as the three passes without scratch
// (HelixScanParams::ytile): the tile of (seq, head h, P slab, segment s),
// Pass A's aggregate D_s and then the start state Pass B writes over it, lies
// in y's rows of segment s, in the slab's own columns: unit u (four floats of
// the tile, helix_params.h order) at row u / (pw / 4), columns 4 (u % (pw / 4))
// .. + 3 of the slab (pw its width, a multiple of 8; y's channel stride is 1).
// The segment's log-decay takes the unit after the tile, in slab 0. Only the
// walk of that (head, slab) over those rows writes these columns afterwards,
// and it has read its start state before (the encoder checks that every
// segment has the rows and that y overlaps no input).
HELIX_DEV long long ytile_base(const HelixScanParams& p, int seq, int h, int slab, int seg) {
    return seq * p.seq_y + (long long)seg * p.seg_len * HELIX_CS * p.s_y[0] + h * p.s_y[1] + (long long)slab * HELIX_HD;
}
// Float offset of tile unit u from ytile_base.
HELIX_DEV long long ytile_unit(const HelixScanParams& p, int u, int pw) {
    const int upr = pw >> 2;
    return (long long)(u / upr) * p.s_y[0] + 4 * (u % upr);
}
// Float offset in y of the log-decay of segment seg of (seq, h).
HELIX_DEV long long ytile_segld(const HelixScanParams& p, int seq, int h, int seg) {
    return ytile_base(p, seq, h, 0, seg) + ytile_unit(p, 16 * p.np, min(HELIX_HD, p.head_dim));
}

#endif  // HELIX_COMMON_H
