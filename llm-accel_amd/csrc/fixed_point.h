// fixed_point.h -- raw-integer ap_fixed arithmetic used by the kernels.
//
// Formats (include/datatypes.hpp:8-15 of the reference): Q8.8 activations
// and gammas, Q4.12 weights, Q16.16 accumulators, Q2.14 probabilities, all
// AP_RND (round half toward +inf) and AP_SAT.  rnd(v, s) drops s fraction
// bits with AP_RND: floor(v / 2^s + 1/2).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define FX_HD __host__ __device__ __forceinline__

FX_HD int64_t fx_rnd(int64_t v, int s) {
    return (v + ((int64_t)1 << (s - 1))) >> s;
}
FX_HD int32_t fx_sat32(int64_t v) {
    return v > INT32_MAX ? INT32_MAX : (v < INT32_MIN ? INT32_MIN : (int32_t)v);
}
FX_HD int16_t fx_sat16(int64_t v) {
    return v > INT16_MAX ? INT16_MAX : (v < INT16_MIN ? INT16_MIN : (int16_t)v);
}
// Q8.8 -> Q4.12 (golden_weight_t(fm)): exact shift, saturating at +-8.
FX_HD int32_t fx_fm_to_wt(int32_t x) { return fx_sat16((int64_t)x * 16); }

// Projection narrowing (host/host_qwen_8x64.cpp:3126-3138, fused MAC
// kernel/mm_stream_8x64_fused_mac.cpp:89-96 + compute_core convert :10-39):
// raw Q28.20 exact sum -> Q16.16 -> Q8.8, each AP_RND + AP_SAT.
FX_HD int16_t fx_narrow_projection(int64_t acc) {
    return fx_sat16(fx_rnd(fx_sat32(fx_rnd(acc, 4)), 8));
}

// golden_recip / cu_recip_approx (host:537-576, compute_stream.cpp:15-48):
// power-of-two seed, three Newton steps est = fm(est * (2 - safe * est)).
FX_HD int16_t fx_recip(int32_t x) {
    int32_t safe = x < 0 ? 0 : x;  // fm(2^-12) is raw 0
    int32_t est = safe >= 16384 ? 4
                : safe >= 8192 ? 8
                : safe >= 4096 ? 16
                : safe >= 2048 ? 32
                : safe >= 1024 ? 64
                : safe >= 512 ? 128
                : safe >= 256 ? 256
                : safe >= 128 ? 512
                : safe >= 64 ? 1024
                : safe >= 32 ? 2048 : 4096;
    for (int i = 0; i < 3; i++) {
        int64_t d = ((int64_t)2 << 16) - (int64_t)safe * est;
        est = fx_sat16(fx_rnd((int64_t)est * d, 16));
    }
    return (int16_t)(est < 0 ? 0 : (est > 16384 ? 16384 : est));
}

// golden_rsqrt / cu_rsqrt_approx (host:621-656, compute_stream.cpp:57-86)
// on a Q16.16 argument.  refine = accum(1.5 - 0.5*safe*est^2) is exact at
// 48 fraction bits before its single rounding, so it needs 128 bits.
FX_HD int16_t fx_rsqrt(int32_t v) {
    int64_t safe = v < 16 ? 16 : v;  // accum(2^-12) = raw 16
    int32_t est = safe >= ((int64_t)64 << 16) ? 32
                : safe >= ((int64_t)16 << 16) ? 64
                : safe >= ((int64_t)4 << 16) ? 128
                : safe >= ((int64_t)1 << 16) ? 256
                : safe >= 16384 ? 512
                : safe >= 4096 ? 1024 : 2048;
    for (int i = 0; i < 3; i++) {
        int32_t square = fx_sat32((int64_t)est * est);
        __int128 t = ((__int128)98304 << 32) -
                     (__int128)32768 * safe * (__int128)square;
        t = (t + ((__int128)1 << 31)) >> 32;
        int32_t refine = t > INT32_MAX ? INT32_MAX
                       : (t < INT32_MIN ? INT32_MIN : (int32_t)t);
        est = fx_sat16(fx_rnd((int64_t)est * refine, 16));
    }
    return (int16_t)(est < 0 ? 0 : (est > 8192 ? 8192 : est));
}

// Per-row RMSNorm gain (golden_rmsnorm host:3162-3197, stream_rmsnorm
// compute_stream.cpp:227-288) from the row's saturating sum of squares.
FX_HD int16_t fx_rmsnorm_gain(int64_t sum_sq, uint32_t cols) {
    int32_t s = sum_sq > INT32_MAX ? INT32_MAX : (int32_t)sum_sq;
    int16_t inv_elems = fx_recip(fx_sat16((int64_t)cols * 256));
    int32_t mean = fx_sat32(fx_rnd((int64_t)s * inv_elems * 256, 16));
    return fx_rsqrt(mean);  // + accum(1e-6), which is raw 0
}

// fx_silu in two steps: the table index its argument selects, then the
// value from that entry.
FX_HD int32_t fx_silu_index(int32_t x) {
    const int32_t c = x >= 0 ? (-x < -2048 ? -2048 : -x) : (x < -2048 ? -2048 : x);
    return c + 2048;
}
FX_HD int16_t fx_silu_entry(int32_t x, int32_t e) {
    const int32_t r = fx_recip(256 + e);
    if (x >= 0) return fx_sat16(fx_rnd((int64_t)x * r, 8));
    return fx_sat16(fx_rnd((int64_t)x * e * r, 16));
}
// golden_silu (host:658-668) with the Q8.8 exp table e8[x + 2048],
// x in [-2048, 0].
FX_HD int16_t fx_silu(int32_t x, const int16_t* e8) {
    if (x >= 0) {
        int32_t nx = -x < -2048 ? -2048 : -x;
        int32_t e = e8[nx + 2048];
        int32_t r = fx_recip(256 + e);
        return fx_sat16(fx_rnd((int64_t)x * r, 8));
    }
    int32_t cx = x < -2048 ? -2048 : x;
    int32_t e = e8[cx + 2048];
    int32_t r = fx_recip(256 + e);
    return fx_sat16(fx_rnd((int64_t)x * e * r, 16));
}

// fm(accum(1) / max(sum, 2^-12)) (host:3726-3730, ctrl:4093-4099): the
// ap_fixed quotient floor(2^32 / b) (16 fraction bits) rounded to Q8.8 is
// floor(2^24 / b + 1/2) = floor((2^25 + b) / (2b)), which saturates for
// b <= 512 and otherwise fits 32-bit unsigned division.
FX_HD int16_t fx_inv_sum(int32_t sum) {
    const uint32_t b = sum < 16 ? 16u : (uint32_t)sum;
    if (b <= 512) return INT16_MAX;
    return (int16_t)(((1u << 25) + b) / (2u * b));
}
