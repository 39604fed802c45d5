// proj_common.h -- projection arithmetic shared by the projection kernels
// and the fused attention-sublayer kernel (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_common.h"
#include "coherent.h"
#include "fixed_point.h"
#include "kernels.h"

namespace llm {
namespace {

__device__ __forceinline__ int64_t dot2_wide(uint32_t a, uint32_t b) {
    int32_t a0 = (int16_t)(a & 0xffff), a1 = (int16_t)(a >> 16);
    int32_t b0 = (int16_t)(b & 0xffff), b1 = (int16_t)(b >> 16);
    return (int64_t)(a0 * b0) + (int64_t)(a1 * b1);
}

// All-ones when `keep`, else zero, as a per-lane value the compiler cannot
// turn back into a branch: a wave-uniform select would let it sink the
// loads that feed the masked value into a conditional block, one memory
// round trip after another.
__device__ __forceinline__ uint32_t lane_mask(bool keep) {
    uint32_t m = keep ? 0xffffffffu : 0u;
    asm volatile("" : "+v"(m));
    return m;
}
__device__ __forceinline__ uint4 and4(uint4 v, uint32_t m) {
    return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
}

// The activations of lane (i, j) of a 4-row weight block -- columns
// 8j .. 8j + 7 of a 128-column k-step -- from the step's 256 bytes loaded
// once per wavefront (lane l holds columns 2l, 2l + 1 in `w`) and spread
// through the LDS crossbar (ds_bpermute, no LDS memory): one 4-byte load
// per lane instead of a 16-byte load that the four lanes of each column
// group would repeat (decode down 8.3 -> 8.0 us).  Every lane of the
// wavefront must be active.
__device__ __forceinline__ uint4 spread8(uint32_t w, int j) {
    return make_uint4((uint32_t)__builtin_amdgcn_ds_bpermute(16 * j, (int)w),
                      (uint32_t)__builtin_amdgcn_ds_bpermute(16 * j + 4, (int)w),
                      (uint32_t)__builtin_amdgcn_ds_bpermute(16 * j + 8, (int)w),
                      (uint32_t)__builtin_amdgcn_ds_bpermute(16 * j + 12, (int)w));
}

// One input normalised with a constant gain: rnd(x * gg, 16), gg = gain *
// gamma (int32), in 32-bit arithmetic: with gg = 2^16 gh + gl (0 <= gl <
// 2^16), floor((x gg + 2^15) / 2^16) = x gh + floor((x gl + 2^15) / 2^16)
// exactly, |x gl + 2^15| < 2^31 for int16 x and |x gh| <= 2^30.  Both
// products have 24-bit operands (x 16 bits, gh and gl within 17), so they
// use the full-rate 24-bit multiply.
__device__ __forceinline__ int32_t norm1(int32_t x, int32_t gg) {
    const int32_t gh = gg >> 16, gl = gg & 0xffff;
    const int32_t y = __mul24(x, gh) + ((__mul24(x, gl) + 32768) >> 16);
    return y < -32768 ? -32768 : (y > 32767 ? 32767 : y);
}
// Eight inputs normalised with a constant gain: rnd(x * gain * gamma, 16);
// columns >= cols have gamma 0 (the caller zeroes g there).  The gain is
// below 2^23 (the host guarantees it), so gain * gamma is a 24-bit product.
__device__ __forceinline__ uint4 norm8(uint4 x, uint4 g, int32_t gain) {
    uint32_t w[4] = {x.x, x.y, x.z, x.w};
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int32_t lo = norm1((int16_t)(w[i] & 0xffff), __mul24(gain, (int16_t)(gw[i] & 0xffff)));
        const int32_t hi = norm1((int16_t)(w[i] >> 16), __mul24(gain, (int16_t)(gw[i] >> 16)));
        w[i] = (uint32_t)(uint16_t)lo | ((uint32_t)hi << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// Sum of v over the 16 lanes of a DPP row (lanes 16i..16i+15), in lane
// 16i + 15: an inclusive scan by row shifts of 1, 2, 4, 8 (lanes shifted
// in from outside the row read 0).
__device__ __forceinline__ int64_t row16_sum(int64_t v) {
#define ROW_SHR_ADD(n)                                                                   \
    {                                                                                    \
        const uint32_t lo = __builtin_amdgcn_update_dpp(0u, (uint32_t)v, 0x110 + n, 0xf, 0xf, true); \
        const uint32_t hi = __builtin_amdgcn_update_dpp(0u, (uint32_t)((uint64_t)v >> 32), 0x110 + n, 0xf, 0xf, true); \
        v += (int64_t)(((uint64_t)hi << 32) | lo);                                         \
    }
    ROW_SHR_ADD(1) ROW_SHR_ADD(2) ROW_SHR_ADD(4) ROW_SHR_ADD(8)
#undef ROW_SHR_ADD
    return v;
}

// Epilogue operands that do not depend on the sums (residual, norm
// gammas), fetched when the kernel starts so that the epilogue waits on no
// memory round trip.
struct EpiIn {
    int32_t res, g0, g1;
};
template <int EPI>
__device__ __forceinline__ EpiIn epi_fetch(const ProjArgs& a, uint32_t r, uint32_t n) {
    EpiIn e{0, 0, 0};
    if (EPI == EPI_RESID) {
        e.res = a.res[(size_t)r * a.ldr + n];
        if (a.norm_out) e.g0 = a.norm_gamma[n];
        if (a.final_out) e.g1 = a.final_gamma[n];
    }
    return e;
}

// Corrections of output (r, n) of a 12-bit copy with out-of-range weights
// (ProjArgs::corr0 / corr1): the row's slot words, and the activations at
// their columns -- as the kernel uses them: normalised on load for
// EPI_STORE_NORM_IN.  corr_slots runs when the kernel starts; corr_inputs
// in the epilogue, for rows that have a correction (XCOH: activations
// written by other workgroups of the same launch, read device-coherently).
struct CorrIn {
    uint32_t e[kCorrSlots];
    int32_t x[kCorrSlots];
};
__device__ __forceinline__ void corr_slots(const uint32_t* corr, uint32_t n, CorrIn& c) {
    const uint4 s = *(const uint4*)(corr + (size_t)kCorrSlots * n);
    c.e[0] = s.x, c.e[1] = s.y, c.e[2] = s.z, c.e[3] = s.w;
}
template <int EPI, bool XCOH>
__device__ __forceinline__ void corr_inputs(const ProjArgs& a, uint32_t r, CorrIn& c) {
#pragma unroll
    for (int j = 0; j < (int)kCorrSlots; j++) {
        const uint32_t k = c.e[j] >> 16;
        const int16_t* px = a.x + (size_t)r * a.ldx + k;
        int32_t x = XCOH ? ld_coherent(px) : *px;
        if (EPI == EPI_STORE_NORM_IN) x = norm1(x, __mul24(a.in_gain, a.in_gamma[k]));
        c.x[j] = x;
    }
}
// The exact correction sum_j x_j * delta_j (0 for unused words).
__device__ __forceinline__ int64_t corr_sum(const CorrIn& c) {
    int64_t s = 0;
#pragma unroll
    for (int j = 0; j < (int)kCorrSlots; j++) s += (int64_t)c.x[j] * (int16_t)(c.e[j] & 0xffffu);
    return s;
}

// fx_narrow_projection with its second rounding in 32-bit arithmetic.
__device__ __forceinline__ int16_t narrow16(int64_t acc) {
    return sat16_32(rnd32(fx_sat32(fx_rnd(acc, 4)), 8));
}
// fx_silu_entry from a packed table word w = e | recip(256 + e) << 16 (the
// reciprocal formed on the host by the same Newton steps), its products in
// 32-bit arithmetic: x r <= 2^15 * 2^14, and x e r as norm1(r, x e) with
// |x e| <= 2^23 (e <= 256).
__device__ __forceinline__ int16_t silu_packed(int32_t x, uint32_t w) {
    const int32_t e = (int32_t)(w & 0xffffu), r = (int32_t)(w >> 16);
    if (x >= 0) return sat16_32(rnd32(x * r, 8));
    return (int16_t)norm1(r, x * e);
}
// Sum of N int64 values as a tree (depth log2 N instead of a chain of N
// dependent 64-bit additions).
template <int N, typename F>
__device__ __forceinline__ int64_t tree_sum64(F get) {
    int64_t v[N];
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = get(i);
#pragma unroll
    for (int n = N; n > 1; n = (n + 1) / 2)
#pragma unroll
        for (int i = 0; i < n / 2; i++) v[i] += v[n - 1 - i];
    return v[0];
}

// Output (r, n) of a projection from its exact sums (gate and up for
// EPI_SILU): the reference's narrowing, then the epilogue.
// COH: the output is read by other workgroups of the same launch, so it is
// written with a device-coherent store.
template <int EPI, bool COH = false>
__device__ __forceinline__ void proj_out(const ProjArgs& a, uint32_t r, uint32_t n,
                                         int64_t t0, int64_t t1, const EpiIn& ei) {
    int16_t y = narrow16(t0);
    if (EPI == EPI_RESID) {
        y = sat16_32((int32_t)y + ei.res);
        // rnd(y gain gamma, 16) with the (int16) gain: norm1's exact split
        if (a.norm_out)
            a.norm_out[(size_t)r * a.ldn + n] = (int16_t)norm1(y, __mul24(a.norm_gain, ei.g0));
        if (a.final_out)
            a.final_out[(size_t)r * a.ldn + n] = (int16_t)norm1(y, __mul24(a.norm_gain, ei.g1));
    } else if (EPI == EPI_SILU) {
        const int16_t up = narrow16(t1);
        const int16_t sg = silu_packed(y, a.silu8[fx_silu_index(y)]);
        y = sat16_32(rnd32((int32_t)sg * up, 8));
    }
    if (COH)
        st_coherent(&a.out[(size_t)r * a.ldo + n], y);
    else
        a.out[(size_t)r * a.ldo + n] = y;
}


// The SiLU epilogue of lanes 0..NL-1 of wavefront 0 (the calling lanes; at
// most 64), output (r, n) of lane et: the table entries through the scalar
// cache, one uniform load per lane, which do not queue behind the vector
// loads of the weight stream (a lane's dependent table load did).
template <int NL>
__device__ __forceinline__ void silu_out_scalar(const ProjArgs& a, uint32_t r, uint32_t n,
                                                int64_t t0, int64_t t1, int et) {
    static_assert(NL <= 64, "lanes of wavefront 0");
    const int16_t y = narrow16(t0);
    const int16_t up = narrow16(t1);
    const int32_t ix = fx_silu_index(y);  // 0..2048
    typedef const __attribute__((address_space(4))) uint32_t* ctab;
    const ctab tab = (ctab)(const void*)a.silu8;
    uint32_t w = 0;
#pragma unroll
    for (int l = 0; l < NL; l++) {
        uint32_t il = __builtin_amdgcn_readlane(ix, l);
        il = il > 2048u ? 2048u : il;  // a lane past the matrix holds anything
        const uint32_t wl = tab[il];
        w = et == l ? wl : w;
    }
    const int16_t sg = silu_packed(y, w);
    a.out[(size_t)r * a.ldo + n] = sat16_32(rnd32((int32_t)sg * up, 8));
}

// NB consecutive 4-row blocks NB b .. NB b + NB - 1 of a projection inside
// a fused launch, on WPB wavefronts that each hold at most SPW k-steps of
// every block (SPW no larger than the widening interval: the int32 sums
// widen once).  Lane (i, j) owns row i and columns 8j..8j+7 of a step, as
// in the projection kernel; the blocks share the activation loads.  The
// weight loads (and the norm gammas and epilogue operands) are issued
// first; then wait() runs and only then the activations are loaded --
// with device-coherent loads when XCOH, for activations another workgroup
// of the same launch wrote.  Steps past a wavefront's last repeat its last
// address and blocks past the matrix its last block; both are masked at
// use, so that no branch separates a load from its use.  red: LDS of
// NB * WPB * 4 * RT int64.  LW: the int32 sums widen once at the end (4:
// the matrix's widening interval covers SPW steps), after every step (1)
// or every product is widened (0).  P12: the weights are read from the
// 12-bit copy a.p0 instead (layout and sums as proj_p12_kernel; int32
// sums, SPW <= 32); CORR: that copy carries corrections (a.corr0; a
// variant of its own, so that the common one holds no code or registers
// for them).  Returns false when wait() gave up (uniform over the
// workgroup).
template <int RT, int EPI, int WPB, int SPW, bool XCOH, bool OCOH, int LW, int NB = 1,
          bool P12 = false, bool CORR = false, typename Wait>
__device__ __forceinline__ bool proj_block(const ProjArgs& a, uint32_t b, int64_t* red,
                                           Wait&& wait) {
    static_assert(EPI != EPI_SILU, "one matrix per block");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane >> 4, j = lane & 15;
    const int et = threadIdx.x;
    const uint32_t nblocks = (a.n + 3) / 4;
    // epilogue thread et < 4 RT NB: block et / (4 RT), output row et % RT
    const uint32_t eb = NB * b + et / (4 * RT), en = eb * 4 + (et % (4 * RT)) / RT, er = et % RT;
    const bool eout = et < 4 * RT * NB && er < a.rows && en < a.n;
    EpiIn ei{0, 0, 0};
    if (eout) ei = epi_fetch<EPI>(a, er, en);
    CorrIn cr = {};  // correction slots of a 12-bit copy (zero without)
    static_assert(!CORR || P12, "corrections belong to a 12-bit copy");
    if (CORR && a.corr0 && eout) corr_slots(a.corr0, en, cr);  // a role's matrix may have none
    const uint32_t S = a.steps;
    const uint32_t s0 = wave * S / WPB, s1 = (wave + 1) * S / WPB;
    const uint32_t cnt = s1 - s0;  // <= SPW (the launcher's choice)
    static_assert(!P12 || SPW <= 32, "int32 sums of the 12-bit products");
    uint4 wv[NB][SPW], gv[SPW];
    uint2 lv[NB][SPW];     // P12: low bytes of the lane's 8 columns
    uint32_t hv[NB][SPW];  // P12: their high nibbles
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        const uint32_t bb = NB * b + nb < nblocks ? NB * b + nb : nblocks - 1;
        if constexpr (P12) {
            const uint8_t* pp = a.p0 + (size_t)(bb * S + s0) * kP12Step;
#pragma unroll
            for (int u = 0; u < SPW; u++) {
                const uint32_t du = cnt == 0 ? 0 : ((uint32_t)u < cnt ? u : cnt - 1);
                lv[nb][u] = *(const uint2*)(pp + (size_t)du * kP12Step + 8 * lane);
                hv[nb][u] = *(const uint32_t*)(pp + (size_t)du * kP12Step + 512 + 4 * lane);
            }
        } else {
            const int16_t* wp = a.w0 + ((size_t)(bb * S + s0) * 4 + i) * 128 + j * 8;
#pragma unroll
            for (int u = 0; u < SPW; u++) {
                const uint32_t du = cnt == 0 ? 0 : ((uint32_t)u < cnt ? u : cnt - 1);
                wv[nb][u] = *(const uint4*)(wp + (size_t)du * 512);
            }
        }
    }
    // EPI_STORE_NORM_IN: lane l normalises columns 2l, 2l + 1 of each of
    // the wavefront's steps and rows (once per wavefront, not once per row
    // of the block), shared through LDS
    constexpr bool NIN = EPI == EPI_STORE_NORM_IN;
    uint32_t g2[SPW];
#pragma unroll
    for (int u = 0; u < SPW; u++) {
        const uint32_t du = cnt == 0 ? 0 : ((uint32_t)u < cnt ? u : cnt - 1);
        if (NIN) g2[u] = *(const uint32_t*)(a.in_gamma + (s0 + du) * 128 + 2 * lane);
    }
    (void)gv;
    if (!wait()) return false;
    uint4 xv[SPW][RT];
    if constexpr (NIN) {
        uint32_t x2[SPW][RT];
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const uint32_t du = cnt == 0 ? 0 : ((uint32_t)u < cnt ? u : cnt - 1);
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const int16_t* px = a.x + (size_t)r * a.ldx + (size_t)(s0 + du) * 128 + 2 * lane;
                x2[u][r] = XCOH ? ld_coherent((const uint32_t*)px) : *(const uint32_t*)px;
            }
        }
        // a wavefront's LDS operations complete in order: no barrier
        __shared__ uint32_t xs[WPB][SPW][RT][64];
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const int32_t glo = __mul24(a.in_gain, (int16_t)(g2[u] & 0xffff));
            const int32_t ghi = __mul24(a.in_gain, (int16_t)(g2[u] >> 16));
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const int32_t lo16 = norm1((int16_t)(x2[u][r] & 0xffff), glo);
                const int32_t hi16 = norm1((int16_t)(x2[u][r] >> 16), ghi);
                xs[wave][u][r][lane] = (uint32_t)(uint16_t)lo16 | ((uint32_t)hi16 << 16);
            }
        }
#pragma unroll
        for (int u = 0; u < SPW; u++)
#pragma unroll
            for (int r = 0; r < RT; r++) xv[u][r] = *(const uint4*)&xs[wave][u][r][4 * j];
    } else {
        // 16 bytes per lane (not spread8: after the wait the spreading's LDS
        // round trip lies on the launch's critical path, measured +0.3 us
        // for the fused sublayer)
        const int16_t* xp = a.x + (size_t)s0 * 128 + j * 8;
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const uint32_t du = cnt == 0 ? 0 : ((uint32_t)u < cnt ? u : cnt - 1);
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const int16_t* px = xp + (size_t)r * a.ldx + du * 128;
                xv[u][r] = XCOH ? ld_coherent16(px) : *(const uint4*)px;
            }
        }
    }
    int32_t part[NB][RT];
    int64_t wide[NB][RT];
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int r = 0; r < RT; r++) part[nb][r] = 0, wide[nb][r] = 0;
    if constexpr (P12) {
        // w + 2048 = 256 h + l: sum w x = 256 sum h x + sum l x - 2048 sum x;
        // steps past the wavefront's last carry zero activations
        int32_t ph[NB][RT], sx[RT];
#pragma unroll
        for (int r = 0; r < RT; r++) {
            sx[r] = 0;
#pragma unroll
            for (int nb = 0; nb < NB; nb++) ph[nb][r] = 0;
        }
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const uint32_t keep = lane_mask((uint32_t)u < cnt);
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const uint4 x = and4(xv[u][r], keep);
                sx[r] = dot2(0x00010001u, x.x, sx[r]);
                sx[r] = dot2(0x00010001u, x.y, sx[r]);
                sx[r] = dot2(0x00010001u, x.z, sx[r]);
                sx[r] = dot2(0x00010001u, x.w, sx[r]);
#pragma unroll
                for (int nb = 0; nb < NB; nb++) {
                    const uint2 l8 = lv[nb][u];
                    const uint32_t h4 = hv[nb][u];
                    int32_t p = part[nb][r], q = ph[nb][r];
                    p = dot2(__builtin_amdgcn_perm(0u, l8.x, 0x0c010c00u), x.x, p);
                    p = dot2(__builtin_amdgcn_perm(0u, l8.x, 0x0c030c02u), x.y, p);
                    p = dot2(__builtin_amdgcn_perm(0u, l8.y, 0x0c010c00u), x.z, p);
                    p = dot2(__builtin_amdgcn_perm(0u, l8.y, 0x0c030c02u), x.w, p);
                    q = dot2(h4 & 0x000f000fu, x.x, q);
                    q = dot2((h4 >> 4) & 0x000f000fu, x.y, q);
                    q = dot2((h4 >> 8) & 0x000f000fu, x.z, q);
                    q = dot2((h4 >> 12) & 0x000f000fu, x.w, q);
                    part[nb][r] = p;
                    ph[nb][r] = q;
                }
            }
        }
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
#pragma unroll
            for (int r = 0; r < RT; r++)
                wide[nb][r] = 256 * (int64_t)ph[nb][r] - 2048 * (int64_t)sx[r];
    } else {
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const uint32_t keep = lane_mask((uint32_t)u < cnt);
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const uint4 x = xv[u][r];
#pragma unroll
                for (int nb = 0; nb < NB; nb++) {
                    const uint4 w = and4(wv[nb][u], keep);
                    if (LW == 0) {
                        wide[nb][r] += dot2_wide(w.x, x.x) + dot2_wide(w.y, x.y) +
                                       dot2_wide(w.z, x.z) + dot2_wide(w.w, x.w);
                    } else {
                        int32_t p = part[nb][r];
                        p = dot2(w.x, x.x, p);
                        p = dot2(w.y, x.y, p);
                        p = dot2(w.z, x.z, p);
                        p = dot2(w.w, x.w, p);
                        part[nb][r] = p;
                        if (LW == 1) wide[nb][r] += p, part[nb][r] = 0;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int r = 0; r < RT; r++) {
            int64_t acc = wide[nb][r] + part[nb][r];
            acc = row16_sum(acc);
            if (j == 15) red[((nb * WPB + wave) * 4 + i) * RT + r] = acc;
        }
    lds_barrier();
    if (eout) {
        const int nb = et / (4 * RT), ii = (et % (4 * RT)) / RT;
        int64_t tot = tree_sum64<WPB>(
            [&](int w) { return red[((nb * WPB + w) * 4 + ii) * RT + er]; });
        if (CORR && (cr.e[0] | cr.e[1] | cr.e[2] | cr.e[3]) != 0) {
            // this row's activations at its correction columns
            corr_inputs<EPI, XCOH>(a, er, cr);
            tot += corr_sum(cr);
        }
        proj_out<EPI, OCOH>(a, er, en, tot, tot, ei);
    }
    return true;
}

}  // namespace
}  // namespace llm
