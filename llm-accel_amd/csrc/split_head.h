// split_head.h -- the split-head attention of one (row, query head) on
// head_dim / 32 wavefronts, shared by the attention kernels and the
// decode stack kernel (internal to the library).  Arithmetic as in
// attention.hip: golden_tiled_flash_attention_q2_14, raw-payload
// semantics (reference host/host_qwen_8x64.cpp:3609-3738).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attention.h"
#include "attn_common.h"
#include "coherent.h"
#include "fixed_point.h"

namespace llm {
namespace {

// Offset of a cache page: tile `tile` of KV head h of the layer the
// arguments point at.
template <int D>
__device__ __forceinline__ size_t page_off(const AttnArgs& a, uint32_t h,
                                           uint32_t tile) {
    return ((size_t)h * a.tiles + tile) * TILE * D;
}

// Half-word j (0..7) of a 16-byte chunk replaced by v.
__device__ __forceinline__ v4u put_half(v4u w, uint32_t j, int32_t v) {
    const uint32_t sh = 16 * (j & 1), msk = 0xffffu << sh, val = (uint32_t)(uint16_t)v << sh;
    if (j / 2 == 0) w.x = (w.x & ~msk) | val;
    else if (j / 2 == 1) w.y = (w.y & ~msk) | val;
    else if (j / 2 == 2) w.z = (w.z & ~msk) | val;
    else w.w = (w.w & ~msk) | val;
    return w;
}

// ---------------------------------------------------------------------
// Split-head path: D / 32 wavefronts per (row, query head), for the
// contexts of the fused path.  Wavefront w owns head elements
// [32 w, 32 w + 32).  QK: lane p forms the four bank partial sums of its
// position over the wavefront's 32 elements (8 products per bank, far from
// wrapping), the partials of all wavefronts meet in LDS (one barrier per
// tile; the buffer alternates with the tile's parity) and every wavefront
// completes the same bank sums, scores, softmax state and probabilities,
// which it keeps in its own LDS slice.  PV: lane (e, half) sums the 32
// positions of one half of the tile for element 32 w + e; the halves meet
// across lanes e and e + 32.  A bank sum taken in pieces is the same
// integer mod 2^32 as the sequential chain, so the +2^31 case reads the
// same.  Cache rows of the next tile are loaded while a tile is computed.
// ---------------------------------------------------------------------
// Per-wavefront LDS scratch of the slice transposes: K [64][40], V^T
// [32][72] (int16; rows padded against bank conflicts).
constexpr int KSROW = 40, VSROW = 72, SLICE_SCRATCH = 64 * KSROW;

template <int D>
struct __attribute__((aligned(16))) SplitSmem {
    static constexpr int NWH = D / 32;
    int16_t q[D], cq[D];                  // rotated query, c(q), bank-paired
    int16_t kc[8][D];                     // the block's K rows after RoPE, bank-paired
    int16_t vc[8][D];                     // the block's V rows
    int16_t p[NWH][TILE], cp[NWH][TILE];  // per wavefront: probabilities, c(p)
    v4u part[2][NWH][TILE];               // QK bank partials (int32), by tile parity
    int16_t e14[2056];                    // Q2.14 exp table
    int16_t scr[NWH][SLICE_SCRATCH];      // per wavefront: slice transposes
};

// A wavefront's share of one tile as loaded: four K chunks and four V^T
// chunks per lane (see slice_load).
struct SplitRegs {
    v4u k[4], v[4];
};

// A wavefront's slices of one tile: its 32 head elements of the K rows
// of all 64 positions, and its 32 V^T rows (all 64 positions), read with
// coalesced 16-byte loads (the page clamped to one in bounds), loaded
// unconditionally: a load under a branch makes the compiler wait for every
// outstanding load where the branch joins, which would stall on the next
// step's prefetch.  Positions that are not cached are masked where the
// rows are used.
//   K: load c, lane l = position 16 c + l / 4, elements 8 (l % 4) ..
//   V: load c, lane l = V^T row 8 c + l / 8, positions 8 (l % 8) ..
template <int D, bool SKIP = false>
__device__ __forceinline__ void slice_load(const AttnArgs& a, uint32_t h, uint32_t tile,
                                           uint32_t w, uint32_t lane, SplitRegs& R) {
    // SKIP: a tile that holds no cached position (the block's first rows
    // at the start of the context) reads nothing, every value would be
    // masked (not in the fused launch, where the branch costs more than
    // the loads it saves)
    if (SKIP && tile * TILE >= a.pos0) {
#pragma unroll
        for (int c = 0; c < 4; c++) R.k[c] = R.v[c] = v4u{0, 0, 0, 0};
        return;
    }
    const uint32_t tp = tile < a.tiles ? tile : a.tiles - 1;
    const int16_t* kp = a.kcache + page_off<D>(a, h, tp) + 32 * w + 8 * (lane & 3);
    const int16_t* vp = a.vcache + page_off<D>(a, h, tp) + (size_t)32 * w * TILE + 8 * lane;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        R.k[c] = *(const v4u*)(kp + (size_t)(16 * c + (lane >> 2)) * D);
        R.v[c] = *(const v4u*)(vp + 512 * c);
    }
}
// The K row (this wavefront's 32 elements) of position `lane`.  LDS
// operations of one wavefront complete in order, so no barrier.
__device__ __forceinline__ void slice_k_rows(int16_t* scr, const SplitRegs& R, uint32_t lane,
                                             v4u* kr) {
#pragma unroll
    for (int c = 0; c < 4; c++)
        *(v4u*)(scr + (16 * c + (lane >> 2)) * KSROW + 8 * (lane & 3)) = R.k[c];
#pragma unroll
    for (int c = 0; c < 4; c++) kr[c] = *(const v4u*)(scr + lane * KSROW + 8 * c);
}
// V^T row 32 w + lane % 32 (this wavefront's), positions of half lane / 32.
__device__ __forceinline__ void slice_v_rows(int16_t* scr, const SplitRegs& R, uint32_t lane,
                                             v4u* vr) {
#pragma unroll
    for (int c = 0; c < 4; c++)
        *(v4u*)(scr + (8 * c + (lane >> 3)) * VSROW + 8 * (lane & 7)) = R.v[c];
#pragma unroll
    for (int c = 0; c < 4; c++)
        vr[c] = *(const v4u*)(scr + (lane & 31) * VSROW + 32 * (lane >> 5) + 8 * c);
}

// Attention of row t, query head g on D / 32 wavefronts (one workgroup).
// FUSED: the q / k / v rows are written by other workgroups of the same
// launch; every load that does not depend on them (exp table, RoPE rows,
// the first tile's cache slices) is issued, then wait() runs, then those
// rows are read with device-coherent loads, and the output row is written
// with device-coherent stores.  Returns false when wait() gave up.
template <int D, bool FUSED, typename Wait>
__device__ __forceinline__ bool split_head_body(const AttnArgs& a, uint32_t t, uint32_t g,
                                                SplitSmem<D>& sm, Wait&& wait) {
    static_assert(D % 32 == 0, "split-head path: head_dim a multiple of 32");
    constexpr uint32_t NTH = D * 2;  // D / 32 wavefronts
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63, w = tid >> 6;
    const uint32_t h = g / a.group;
    const uint32_t n = a.pos0 + t + 1, own = n - 1;
    const uint32_t ntiles = (n + TILE - 1) / TILE;
    const int64_t scale = (int64_t)a.qk_scale << 8;

    // ---- staging loads (indices clamped: every load is issued), then the
    // first tile's slices, then the staging writes ----
    constexpr int NE = (257 + NTH - 1) / NTH;          // exp table pieces per thread
    constexpr int NK = (8 * (D / 2) + NTH - 1) / NTH;  // block K items per thread
    constexpr int NV = (8 * D + NTH - 1) / NTH;        // block V elements per thread
    v4u ex[NE];
#pragma unroll
    for (int u = 0; u < NE; u++) {
        const uint32_t c = tid + NTH * u;
        ex[u] = *(const v4u*)(a.exp14 + 8 * (c < 257 ? c : 256));
    }
    const uint32_t qc = tid < D / 2 ? tid : 0;
    const int16_t* qrow = a.qkv + (size_t)t * a.ldqkv + (size_t)g * D;
    const int16_t* qrope = a.rope + (size_t)own * D;
    const int32_t qcs = qrope[qc], qsn = qrope[D / 2 + qc];
    const uint32_t nk = (t + 1) * (D / 2), nv = (t + 1) * D;
    int32_t kx[NK][4];
#pragma unroll
    for (int u = 0; u < NK; u++) {
        const uint32_t i = tid + NTH * u < nk ? tid + NTH * u : 0;
        const uint32_t r = i / (D / 2), c = i % (D / 2);
        const int16_t* kr = a.rope + (size_t)(a.pos0 + r) * D;
        kx[u][2] = kr[c];
        kx[u][3] = kr[D / 2 + c];
    }
    SplitRegs regs;
    slice_load<D, !FUSED>(a, h, 0, w, lane, regs);
    if (FUSED && !wait()) return false;
    // the block's q / k / v rows
    auto ld_row = [&](const int16_t* p) -> int32_t { return FUSED ? ld_coherent(p) : *p; };
    const int32_t qx0 = ld_row(qrow + qc), qx1 = ld_row(qrow + D / 2 + qc);
#pragma unroll
    for (int u = 0; u < NK; u++) {
        const uint32_t i = tid + NTH * u < nk ? tid + NTH * u : 0;
        const uint32_t r = i / (D / 2), c = i % (D / 2);
        const int16_t* krow = a.qkv + (size_t)r * a.ldqkv + (size_t)a.num_heads * D +
                              (size_t)h * D;
        kx[u][0] = ld_row(krow + c);
        kx[u][1] = ld_row(krow + D / 2 + c);
    }
    int16_t vx[NV];
#pragma unroll
    for (int u = 0; u < NV; u++) {
        const uint32_t i = tid + NTH * u < nv ? tid + NTH * u : 0;
        vx[u] = (int16_t)ld_row(a.qkv + (size_t)(i / D) * a.ldqkv +
                                (size_t)(a.num_heads + a.num_kv_heads) * D + (size_t)h * D + i % D);
    }
#pragma unroll
    for (int u = 0; u < NE; u++) {
        const uint32_t c = tid + NTH * u;
        if (c < 257) *(v4u*)(sm.e14 + 8 * c) = ex[u];
    }
    if (tid < D / 2) {
        int32_t y0, y1;
        rope_pair(qx0, qx1, qcs, qsn, y0, y1);
        sm.q[paired(tid)] = (int16_t)y0;
        sm.q[paired(D / 2 + tid)] = (int16_t)y1;
        sm.cq[paired(tid)] = (int16_t)sat_corr(y0);
        sm.cq[paired(D / 2 + tid)] = (int16_t)sat_corr(y1);
    }
#pragma unroll
    for (int u = 0; u < NK; u++) {
        const uint32_t i = tid + NTH * u;
        if (i < nk) {
            const uint32_t r = i / (D / 2), c = i % (D / 2);
            int32_t y0, y1;
            rope_pair(kx[u][0], kx[u][1], kx[u][2], kx[u][3], y0, y1);
            sm.kc[r][paired(c)] = (int16_t)y0;
            sm.kc[r][paired(D / 2 + c)] = (int16_t)y1;
        }
    }
#pragma unroll
    for (int u = 0; u < NV; u++) {
        const uint32_t i = tid + NTH * u;
        if (i < nv) sm.vc[i / D][i % D] = vx[u];
    }
    lds_barrier();

    const uint32_t el = lane & 31, hh = lane >> 5, e = 32 * w + el;
    int32_t m = INT16_MIN, sum = 0, acc = 0;
    for (uint32_t tile = 0; tile < ntiles; tile++) {
        const SplitRegs cur = regs;
        // the next tile's slices (a repeat of this tile's on the last one)
        slice_load<D, !FUSED>(a, h, tile + 1 < ntiles ? tile + 1 : tile, w, lane, regs);
        // ---- QK partials over this wavefront's elements ----
        const uint32_t p = tile * TILE + lane;
        const bool valid = p < n;
        const bool blk = p >= a.pos0 && p <= own;  // K row of this block
        const bool cached = p < a.pos0;
        const int16_t* kb = sm.kc[blk ? p - a.pos0 : 0] + 32 * w;
        v4u kr[4];
        slice_k_rows(sm.scr[w], cur, lane, kr);
        uint32_t mk = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const v4u kv = blk ? *(const v4u*)(kb + 8 * c) : kr[c];
            kr[c] = clamp4(blk || cached ? kv : v4u{0, 0, 0, 0}, mk);
        }
        const bool kcorr = __any(mk != 0);
        int32_t b0 = 0, b1 = 0, b2 = 0, b3 = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const v4u qv = *(const v4u*)(sm.q + 32 * w + 8 * c);
            b0 = dot2(kr[c].x, qv.x, b0);
            b1 = dot2(kr[c].y, qv.y, b1);
            b2 = dot2(kr[c].z, qv.z, b2);
            b3 = dot2(kr[c].w, qv.w, b3);
        }
        if (kcorr) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const v4u cv = *(const v4u*)(sm.cq + 32 * w + 8 * c);
                b0 = dot2(sat_mask(kr[c].x), cv.x, b0);
                b1 = dot2(sat_mask(kr[c].y), cv.y, b1);
                b2 = dot2(sat_mask(kr[c].z), cv.z, b2);
                b3 = dot2(sat_mask(kr[c].w), cv.w, b3);
            }
        }
        sm.part[tile & 1][w][lane] = v4u{(uint32_t)b0, (uint32_t)b1, (uint32_t)b2, (uint32_t)b3};
        lds_barrier();  // every wavefront's partials
        uint32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;  // bank sums mod 2^32
#pragma unroll
        for (int ww = 0; ww < SplitSmem<D>::NWH; ww++) {
            const v4u pv = sm.part[tile & 1][ww][lane];
            s0 += pv.x;
            s1 += pv.y;
            s2 += pv.z;
            s3 += pv.w;
        }
        // +2^31 (one saturating bank) wraps to INT32_MIN
        const int64_t t64 = (int64_t)((int32_t)s0 == INT32_MIN ? INT32_MAX : (int32_t)s0) +
                            ((int32_t)s1 == INT32_MIN ? INT32_MAX : (int32_t)s1) +
                            ((int32_t)s2 == INT32_MIN ? INT32_MAX : (int32_t)s2) +
                            ((int32_t)s3 == INT32_MIN ? INT32_MAX : (int32_t)s3);
        int32_t ts32 = fx_sat32(t64);
        ts32 = rnd16_mul(ts32, (int32_t)scale);  // scale = qk_scale << 8 <= 2^16
        const int32_t s = valid ? sat16_32(rnd32(ts32, 8)) : INT16_MIN;
        // ---- softmax state (the same in every wavefront) ----
        const int32_t wm = wave_max(s);
        const int32_t mn = wm > m ? wm : m;
        const int32_t old = prob(sm.e14, m - mn);
        const int32_t pr = valid ? prob(sm.e14, s - mn) : 0;
        sm.p[w][paired(lane)] = (int16_t)pr;
        sm.cp[w][paired(lane)] = (int16_t)sat_corr(pr);
        const int32_t tsum = wave_sum(pr);  // <= 64 * 16384
        // (old << 2 <= 2^16; sum and its terms are non-negative, so the
        // saturation of the rounded sum is that of nested saturating adds)
        sum = __builtin_elementwise_add_sat(rnd16_mul(sum, old << 2), tsum << 2);
        m = mn;
        if (old != 16384) acc = rnd16_mul(acc, old << 2);
        // ---- PV over half hh of the tile for element e ----
        v4u vr[4];
        slice_v_rows(sm.scr[w], cur, lane, vr);
#pragma unroll
        for (int c = 0; c < 4; c++)  // chunks holding no cached position: zero
            vr[c] = tile * TILE + 32 * hh + 8 * c < a.pos0 ? vr[c] : v4u{0, 0, 0, 0};
        // the block's V rows in this tile go to their own slots (slots
        // beyond the context meet probability 0)
        for (uint32_t r = 0; r <= t; r++) {
            const uint32_t pp = a.pos0 + r;
            if (pp / TILE != tile) continue;
            const uint32_t slot = paired(pp % TILE);
            if (slot / 32 != hh) continue;
#pragma unroll
            for (int c = 0; c < 4; c++)
                if ((slot % 32) / 8 == (uint32_t)c) vr[c] = put_half(vr[c], slot % 8, sm.vc[r][e]);
        }
        uint32_t mv = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) vr[c] = clamp4(vr[c], mv);
        const bool vcorr = __any(mv != 0);
        b0 = b1 = b2 = b3 = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const v4u pv = *(const v4u*)(sm.p[w] + 32 * hh + 8 * c);
            b0 = dot2(vr[c].x, pv.x, b0);
            b1 = dot2(vr[c].y, pv.y, b1);
            b2 = dot2(vr[c].z, pv.z, b2);
            b3 = dot2(vr[c].w, pv.w, b3);
        }
        if (vcorr) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const v4u cv = *(const v4u*)(sm.cp[w] + 32 * hh + 8 * c);
                b0 = dot2(sat_mask(vr[c].x), cv.x, b0);
                b1 = dot2(sat_mask(vr[c].y), cv.y, b1);
                b2 = dot2(sat_mask(vr[c].z), cv.z, b2);
                b3 = dot2(sat_mask(vr[c].w), cv.w, b3);
            }
        }
        // the two halves of each bank (PV banks never leave the range)
        b0 += __shfl_xor(b0, 32, 64);
        b1 += __shfl_xor(b1, 32, 64);
        b2 += __shfl_xor(b2, 32, 64);
        b3 += __shfl_xor(b3, 32, 64);
        int32_t tv = fx_sat32((int64_t)b0 + b1 + b2 + b3);
        tv = sat16_32(rnd32(rnd32(tv, 6), 8));  // rnd(tv 2^10, 16) = rnd(tv, 6)
        acc = __builtin_elementwise_add_sat(acc, tv * 256);
    }
    const int32_t inv = fx_inv_sum(sum);
    if (hh == 0) {
        const int16_t y = sat16_32(rnd16_mul(acc, inv));  // 0 <= inv < 2^15
        int16_t* po = a.out + (size_t)t * a.ldo + (size_t)g * D + e;
        if (FUSED)
            st_coherent(po, y);
        else
            *po = y;
    }
    if (g % a.group == 0) {  // this row's K (rotated, paired) and V into the cache
        const uint32_t tile = own / TILE, slot = own % TILE;
        if (tid < D / 8)
            *(v4u*)(a.kcache + page_off<D>(a, h, tile) + slot * D + 8 * tid) =
                *(const v4u*)(sm.kc[t] + 8 * tid);
        if (tid < D) a.vcache[page_off<D>(a, h, tile) + tid * TILE + paired(slot)] = sm.vc[t][tid];
    }
    return true;
}

}  // namespace
}  // namespace llm
