// attn_common.h -- fixed-point attention arithmetic shared by the attention
// kernels and the layer engine (internal to the library).
//
// Products, bank sums, Q2.14 probabilities and the rounding of scores and
// PV values follow golden_tiled_flash_attention_q2_14 (raw-payload
// semantics, reference host/host_qwen_8x64.cpp:3609-3738 ==
// kernel/control_cache_8x64.cpp:5491-5765).  K / V operands are Q8.8
// values staged clamped to [-2048, 2048]; a staged 2048 marks a value that
// saturates in Q4.12, whose product is corrected by c(x) =
// floor((8 - x) / 16).  Rows are kept with every 8-element group in the
// bank-paired order [0 4 1 5 2 6 3 7], so dword j of a group holds
// elements j and j + 4 of bank j.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fixed_point.h"

namespace llm {
namespace {

constexpr int TILE = 64;

typedef short s16x2 __attribute__((ext_vector_type(2)));
// Register staging types: native vectors (plain loads and stores, no
// aggregate copies).
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int32_t dot2(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s16x2, a),
                                  __builtin_bit_cast(s16x2, b), c, false);
}

// Slot of element u (0..7) of a group in the bank-paired order, and back.
__device__ __forceinline__ uint32_t paired(uint32_t e) {
    const uint32_t u = e & 7u;
    return (e & ~7u) | (u < 4 ? 2 * u : 2 * (u - 4) + 1);
}
__device__ __forceinline__ uint32_t slot_pos(uint32_t j) {
    return (j >> 1) + 4 * (j & 1);
}

__device__ __forceinline__ int32_t clamp_k(int32_t v) {
    return v < -2048 ? -2048 : (v > 2048 ? 2048 : v);
}
// c(x) = floor((8 - x) / 16): correction of a product with 32767.
__device__ __forceinline__ int32_t sat_corr(int32_t x) { return (8 - x) >> 4; }

// Both int16 halves clamped to [-2048, 2048] (v_pk_max_i16 / v_pk_min_i16).
__device__ __forceinline__ uint32_t clamp_word(uint32_t w) {
    const s16x2 lo = {-2048, -2048}, hi = {2048, 2048};
    const s16x2 v = __builtin_bit_cast(s16x2, w);
    return __builtin_bit_cast(uint32_t,
                              __builtin_elementwise_min(__builtin_elementwise_max(v, lo), hi));
}
// 1 in each half of a clamped word that holds 2048 (a saturating value):
// in [-2048, 2048] that is the one value with bit 11 set and bit 15 clear.
__device__ __forceinline__ uint32_t sat_mask(uint32_t w) {
    return (w >> 11) & ~(w >> 15) & 0x00010001u;
}
// Clamped chunk; `any` collects the saturation masks of its words, so
// that after a row any != 0 tells whether a value saturated.  (A running
// packed maximum of the clamped words compared with 2048 would be fewer
// operations, but its reduction has been observed to compile to the
// maximum of one word per chunk and miss values in the others.)
__device__ __forceinline__ v4u clamp4(v4u v, uint32_t& any) {
    v4u r;
    r.x = clamp_word(v.x);
    r.y = clamp_word(v.y);
    r.z = clamp_word(v.z);
    r.w = clamp_word(v.w);
    any |= sat_mask(r.x) | sat_mask(r.y) | sat_mask(r.z) | sat_mask(r.w);
    return r;
}

// rnd(v * f, 16) for 0 <= f <= 2^16, exactly, in full-rate 24-bit
// products: with v = 2^16 h + l (l the low 16 bits), rnd(v f, 16) = h f +
// ((l f + 2^15) >> 16); |h f| <= 2^31, l f + 2^15 < 2^32, and the result
// lies within |v| (a dependent 64-bit multiply-add costs ~100 cycles).
__device__ __forceinline__ int32_t rnd16_mul(int32_t v, int32_t f) {
    const uint32_t lo = (__umul24((uint32_t)v & 0xffffu, (uint32_t)f) + 32768u) >> 16;
    return __mul24(v >> 16, f) + (int32_t)lo;
}
// rnd(v, s) of an int32 in 32-bit arithmetic: floor(v / 2^s) plus the
// carry of the dropped bits and the half.
__device__ __forceinline__ int32_t rnd32(int32_t v, int s) {
    return (v >> s) + (int32_t)((((uint32_t)v & ((1u << s) - 1u)) + (1u << (s - 1))) >> s);
}
__device__ __forceinline__ int16_t sat16_32(int32_t v) {
    return (int16_t)(v < INT16_MIN ? INT16_MIN : (v > INT16_MAX ? INT16_MAX : v));
}

__device__ __forceinline__ int16_t prob(const int16_t* exp14, int32_t x) {
    x = fx_sat16(x);
    x = x < -2048 ? -2048 : x;
    return exp14[x + 2048];
}

// Workgroup barrier that orders LDS only: a __syncthreads() fences every
// address space and so waits for the workgroup's outstanding global loads
// (the next tile's prefetch) as well.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Wavefront reductions over DPP row operations; the result is uniform.
template <int CTRL, int ROWS>
__device__ __forceinline__ int32_t dpp(int32_t old, int32_t v) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWS, 0xf, false);
}
__device__ __forceinline__ int32_t wave_max(int32_t v) {
    v = max(v, dpp<0xb1, 0xf>(v, v));   // quad_perm [1 0 3 2]
    v = max(v, dpp<0x4e, 0xf>(v, v));   // quad_perm [2 3 0 1]
    v = max(v, dpp<0x141, 0xf>(v, v));  // row_half_mirror
    v = max(v, dpp<0x140, 0xf>(v, v));  // row_mirror
    v = max(v, dpp<0x142, 0xa>(v, v));  // row_bcast:15 -> rows 1, 3
    v = max(v, dpp<0x143, 0xc>(v, v));  // row_bcast:31 -> rows 2, 3
    return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ int32_t wave_sum(int32_t v) {
    v += dpp<0xb1, 0xf>(0, v);
    v += dpp<0x4e, 0xf>(0, v);
    v += dpp<0x141, 0xf>(0, v);
    v += dpp<0x140, 0xf>(0, v);
    v += dpp<0x142, 0xa>(0, v);
    v += dpp<0x143, 0xc>(0, v);
    return __builtin_amdgcn_readlane(v, 63);
}
// Maximum of `first` and the values of the lanes below each lane (lane 0:
// first alone): the lanes shifted up by one (wave_shr:1, lane 0 takes
// `first`), then an inclusive scan within rows of 16 (row_shr 1, 2, 4, 8;
// lanes without a source keep INT32_MIN) and across them (row_bcast).
__device__ __forceinline__ int32_t wave_prefix_max_excl(int32_t v, int32_t first) {
    v = __builtin_amdgcn_update_dpp(first, v, 0x138, 0xf, 0xf, false);  // wave_shr:1
    v = max(v, dpp<0x111, 0xf>(INT32_MIN, v));  // row_shr:1
    v = max(v, dpp<0x112, 0xf>(INT32_MIN, v));  // row_shr:2
    v = max(v, dpp<0x114, 0xf>(INT32_MIN, v));  // row_shr:4
    v = max(v, dpp<0x118, 0xf>(INT32_MIN, v));  // row_shr:8
    v = max(v, dpp<0x142, 0xa>(INT32_MIN, v));  // row_bcast:15 -> rows 1, 3
    v = max(v, dpp<0x143, 0xc>(INT32_MIN, v));  // row_bcast:31 -> rows 2, 3
    return v;
}

// (x0, x1) rotated by the Q8.8 table entry (c, s) (host:4765-4788).  The
// table holds quantised cos / sin, |c|, |s| <= 256, so the sums fit int32.
__device__ __forceinline__ void rope_pair(int32_t x0, int32_t x1, int32_t c,
                                          int32_t s, int32_t& y0, int32_t& y1) {
    y0 = fx_sat16((x0 * c - x1 * s + 128) >> 8);
    y1 = fx_sat16((x1 * c + x0 * s + 128) >> 8);
}

__device__ __forceinline__ int32_t half16(const v2u& v, uint32_t j) {
    const uint32_t w = j < 2 ? v.x : v.y;
    return (int16_t)((j & 1) ? (w >> 16) : (w & 0xffff));
}
__device__ __forceinline__ int32_t half16(const v4u& v, uint32_t j) {
    const uint32_t w = j < 2 ? v.x : (j < 4 ? v.y : (j < 6 ? v.z : v.w));
    return (int16_t)((j & 1) ? (w >> 16) : (w & 0xffff));
}

// Score (Q8.8) of the query qg (bank-paired; c(q) in cg) against the K row
// held in kr (bank-paired, clamped).
template <int D>
__device__ __forceinline__ int16_t row_score(const int16_t* qg, const int16_t* cg,
                                             const v4u* kr, bool corr, int64_t scale) {
    int32_t b0 = 0, b1 = 0, b2 = 0, b3 = 0;
#pragma unroll
    for (int c = 0; c < D / 8; c++) {
        const v4u qv = *(const v4u*)(qg + 8 * c);
        b0 = dot2(kr[c].x, qv.x, b0);
        b1 = dot2(kr[c].y, qv.y, b1);
        b2 = dot2(kr[c].z, qv.z, b2);
        b3 = dot2(kr[c].w, qv.w, b3);
    }
    if (corr) {
#pragma unroll
        for (int c = 0; c < D / 8; c++) {
            const v4u cv = *(const v4u*)(cg + 8 * c);
            b0 = dot2(sat_mask(kr[c].x), cv.x, b0);
            b1 = dot2(sat_mask(kr[c].y), cv.y, b1);
            b2 = dot2(sat_mask(kr[c].z), cv.z, b2);
            b3 = dot2(sat_mask(kr[c].w), cv.w, b3);
        }
    }
    // +2^31 (one saturating bank) wraps to INT32_MIN
    const int64_t t64 = (int64_t)(b0 == INT32_MIN ? INT32_MAX : b0) +
                        (b1 == INT32_MIN ? INT32_MAX : b1) +
                        (b2 == INT32_MIN ? INT32_MAX : b2) +
                        (b3 == INT32_MIN ? INT32_MAX : b3);
    int32_t t = fx_sat32(t64);
    t = fx_sat32(fx_rnd((int64_t)t * scale, 16));
    return fx_sat16(fx_rnd(t, 8));
}

// Q8.8 PV tile value of one query head (probabilities pg, c(p) cg) against
// the V^T row held in vr: banks, x fm(1/64).
__device__ __forceinline__ int32_t row_pv(const int16_t* pg, const int16_t* cg,
                                          const v4u* vr, bool corr) {
    int32_t b0 = 0, b1 = 0, b2 = 0, b3 = 0;
#pragma unroll
    for (int c = 0; c < TILE / 8; c++) {
        const v4u pv = *(const v4u*)(pg + 8 * c);
        b0 = dot2(vr[c].x, pv.x, b0);
        b1 = dot2(vr[c].y, pv.y, b1);
        b2 = dot2(vr[c].z, pv.z, b2);
        b3 = dot2(vr[c].w, pv.w, b3);
    }
    if (corr) {
#pragma unroll
        for (int c = 0; c < TILE / 8; c++) {
            const v4u cv = *(const v4u*)(cg + 8 * c);
            b0 = dot2(sat_mask(vr[c].x), cv.x, b0);
            b1 = dot2(sat_mask(vr[c].y), cv.y, b1);
            b2 = dot2(sat_mask(vr[c].z), cv.z, b2);
            b3 = dot2(sat_mask(vr[c].w), cv.w, b3);
        }
    }
    int32_t t = fx_sat32((int64_t)b0 + b1 + b2 + b3);
    t = fx_sat32(fx_rnd((int64_t)t * 1024, 16));
    return fx_sat16(fx_rnd(t, 8));
}


}  // namespace
}  // namespace llm
