// attention_gqa.hip -- long-context attention with the query heads of a
// GQA group sharing each K / V page (head_dim 64 or 128, at most 8 query
// heads per KV head).  Arithmetic as in attention.hip (the reference's
// golden_tiled_flash_attention_q2_14, raw-payload semantics,
// host/host_qwen_8x64.cpp:3609-3738; the controller gives each compute
// unit one KV head and runs the whole query group against each 64-position
// tile, kernel/control_cache_8x64.cpp:5604-5748).  Three steps, in one
// launch when the grid is resident (attention_gqa_fused_kernel: the tiles'
// maxima and sums handed to the scan's workgroups as epoch-tagged words),
// else in two or three launches:
//   (1) scores: one workgroup per (row, KV head, tile) stages the tile's K
//       rows in LDS once and forms the scores and tile maxima of all G query
//       heads; the K row of each row's own position is appended;
//   (2) PV: one workgroup per (row, KV head, tile) stages the tile's V^T in
//       LDS once and, for every head, forms the probabilities under the
//       running max after the tile (the maximum of the tile maxima up to
//       it), their sum and the rounded PV value of every element; the V row
//       is appended;
//   (3) scan: one workgroup per (row, query head, 32 elements) runs the
//       per-tile rounding recurrence.  The running max rises at a few tiles only
//       ("events"); between two events the recurrence only adds exact
//       int32 terms, so each such run is summed in parallel and the
//       sequential part is one step per event, taken only when no partial
//       sum of the run can reach the int32 bounds (else the run goes tile
//       by tile).
// Scratch (s_scores, s_tmax, s_tsum, s_tval) is indexed (row, KV head,
// tile, head in group) as in the other split paths.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attention.h"
#include "attn_common.h"
#include "coherent.h"
#include "fixed_point.h"
#include "split_head.h"

namespace llm {
namespace {

constexpr uint32_t GNT = 256;    // threads per workgroup
constexpr uint32_t GMAXG = 8;    // query heads per KV head
constexpr uint32_t GMAXT = 1024; // tiles per context (scan)
constexpr uint32_t GSLOTS = 32;  // runs the scan sums in parallel (more: tile by tile)
constexpr uint32_t GSE = 32;     // elements per scan workgroup

// Block rows [r0, r0 + nrow) of a row's block that fall in `tile`.
struct GqaRows {
    uint32_t r0, nrow;
};
__device__ __forceinline__ GqaRows gqa_rows(const AttnArgs& a, uint32_t tile, uint32_t own) {
    GqaRows r;
    const uint32_t lo = tile * TILE, hi = tile * TILE + TILE - 1;
    r.r0 = lo > a.pos0 ? lo - a.pos0 : 0;
    r.nrow = hi >= a.pos0 ? (own < hi ? own : hi) - a.pos0 + 1 - r.r0 : 0;
    return r;
}

// Workgroup -> (row, KV head, tile); false for padding or a tile beyond
// the row's context.
struct GqaWg {
    uint32_t t, h, tile;
};
__device__ __forceinline__ bool gqa_wg(const AttnArgs& a, GqaWg& w) {
    const uint32_t L = blockIdx.x;
    w.h = L % a.num_kv_heads;
    const uint32_t rt = L / a.num_kv_heads;
    w.t = rt / a.grid_tiles;
    w.tile = rt % a.grid_tiles;
    return w.t < a.grid_rows && w.tile * TILE < a.pos0 + w.t + 1;
}

template <int D>
struct __attribute__((aligned(16))) GqaScoresSmem {
    int16_t q[GMAXG][D], cq[GMAXG][D];  // rotated queries of the group, c(q)
    int16_t kv[8][D];                   // the block's K rows after RoPE
    int16_t k[TILE][D + 8];             // the tile's K rows, clamped (rows padded)
    uint32_t sat;                       // a staged K value saturates
};

// Scores of a (row, KV head, tile) workgroup: lane = position, heads w and
// w + 4.  FUSED keeps them (and the tile maxima) in sc / mt for the PV phase
// of the same workgroup and publishes the maxima as tagged words; else they
// go to s_scores.  The maxima go to s_tmax either way (the scan reads them).
template <int D>
struct GqaScoresLoads {
    static constexpr uint32_t HD = D / 2, C8 = D / 8;
    static constexpr int KC = TILE * C8 / GNT;               // K chunks per thread
    static constexpr int QP = (GMAXG * HD + GNT - 1) / GNT;  // query pairs per thread
    static constexpr int NK = (8 * HD + GNT - 1) / GNT;      // block K pairs per thread
    v4u kc[KC];
    int32_t qx[QP][4], kx[NK][4];
};
// The scores phase's loads (indices clamped: every load is issued): the
// tile's K page, the group's query rows and the block's K rows in the tile
// with their RoPE rows.
template <int D>
__device__ __forceinline__ void gqa_scores_loads(const AttnArgs& a, const GqaWg& wg,
                                                 GqaScoresLoads<D>& L) {
    constexpr uint32_t HD = D / 2, C8 = D / 8;
    const uint32_t t = wg.t, h = wg.h, tile = wg.tile, tid = threadIdx.x;
    const uint32_t own = a.pos0 + t, G = a.group;
    const uint32_t tp = tile < a.tiles ? tile : a.tiles - 1;
    const int16_t* kpage = a.kcache + page_off<D>(a, h, tp);
#pragma unroll
    for (int u = 0; u < GqaScoresLoads<D>::KC; u++) {
        const uint32_t i = tid + GNT * u;
        L.kc[u] = *(const v4u*)(kpage + (i / C8) * D + 8 * (i % C8));
    }
#pragma unroll
    for (int u = 0; u < GqaScoresLoads<D>::QP; u++) {
        const uint32_t i = tid + GNT * u < G * HD ? tid + GNT * u : 0;
        const uint32_t gi = i / HD, c = i % HD;
        const int16_t* qrow = a.qkv + (size_t)t * a.ldqkv + (size_t)(h * G + gi) * D;
        const int16_t* rp = a.rope + (size_t)own * D;
        L.qx[u][0] = qrow[c];
        L.qx[u][1] = qrow[HD + c];
        L.qx[u][2] = rp[c];
        L.qx[u][3] = rp[HD + c];
    }
    const GqaRows tr = gqa_rows(a, tile, own);
    const uint32_t nk = tr.nrow * HD;
#pragma unroll
    for (int u = 0; u < GqaScoresLoads<D>::NK; u++) {
        const uint32_t i = tid + GNT * u < nk ? tid + GNT * u : 0;
        const uint32_t r = tr.r0 + i / HD, c = i % HD;
        const int16_t* krow = a.qkv + (size_t)r * a.ldqkv + (size_t)a.num_heads * D +
                              (size_t)h * D;
        const int16_t* kr = a.rope + (size_t)(a.pos0 + r) * D;
        L.kx[u][0] = krow[c];
        L.kx[u][1] = krow[HD + c];
        L.kx[u][2] = kr[c];
        L.kx[u][3] = kr[HD + c];
    }
}

// Scores of a (row, KV head, tile) workgroup from its loads: lane =
// position, heads w and w + 4.  FUSED keeps them (and the tile maxima) in
// sc / mt for the PV phase of the same workgroup and publishes the maxima
// as tagged words; else they go to s_scores.  The maxima go to s_tmax
// either way (the scan reads them).
template <int D, bool FUSED>
__device__ __forceinline__ void gqa_scores_body(const AttnArgs& a, const GqaWg& wg,
                                                GqaScoresSmem<D>& sm,
                                                const GqaScoresLoads<D>& L, int32_t (&sc)[2],
                                                int32_t (&mt)[2]) {
    static_assert(D == 64 || D == 128, "GQA tile path: head_dim 64 or 128");
    constexpr uint32_t HD = D / 2, C8 = D / 8;
    constexpr int KC = GqaScoresLoads<D>::KC, QP = GqaScoresLoads<D>::QP,
                  NK = GqaScoresLoads<D>::NK;
    const uint32_t t = wg.t, h = wg.h, tile = wg.tile, tid = threadIdx.x;
    const uint32_t n = a.pos0 + t + 1, own = n - 1, G = a.group;
    const uint32_t lane = tid & 63, w = tid >> 6;
    const int64_t scale = (int64_t)a.qk_scale << 8;
    const v4u* kc = L.kc;
    const int32_t(*qx)[4] = L.qx;
    const int32_t(*kx)[4] = L.kx;
    const GqaRows tr = gqa_rows(a, tile, own);
    const uint32_t nk = tr.nrow * HD;
    // ---- the group's queries and the block's K rows, rotated ----
    if (tid == 0) sm.sat = 0;
#pragma unroll
    for (int u = 0; u < QP; u++) {
        const uint32_t i = tid + GNT * u;
        if (i < G * HD) {
            const uint32_t gi = i / HD, c = i % HD;
            int32_t y0, y1;
            rope_pair(qx[u][0], qx[u][1], qx[u][2], qx[u][3], y0, y1);
            sm.q[gi][paired(c)] = (int16_t)y0;
            sm.q[gi][paired(HD + c)] = (int16_t)y1;
            sm.cq[gi][paired(c)] = (int16_t)sat_corr(y0);
            sm.cq[gi][paired(HD + c)] = (int16_t)sat_corr(y1);
        }
    }
#pragma unroll
    for (int u = 0; u < NK; u++) {
        const uint32_t i = tid + GNT * u;
        if (i < nk) {
            const uint32_t r = tr.r0 + i / HD, c = i % HD;
            int32_t y0, y1;
            rope_pair(kx[u][0], kx[u][1], kx[u][2], kx[u][3], y0, y1);
            sm.kv[r][paired(c)] = (int16_t)y0;
            sm.kv[r][paired(HD + c)] = (int16_t)y1;
        }
    }
    lds_barrier();
    // ---- the tile's K rows: cached positions from the page, the block's
    // positions from its rotated rows, later positions 0; clamped ----
    uint32_t any = 0;
#pragma unroll
    for (int u = 0; u < KC; u++) {
        const uint32_t i = tid + GNT * u, p = i / C8, c8 = i % C8;
        const uint32_t pos = tile * TILE + p;
        v4u v = pos < a.pos0 ? kc[u]
              : (pos <= own ? *(const v4u*)(sm.kv[pos - a.pos0] + 8 * c8) : v4u{0, 0, 0, 0});
        *(v4u*)(&sm.k[p][8 * c8]) = clamp4(v, any);
    }
    if (any) sm.sat = 1;
    lds_barrier();
    const bool kcorr = sm.sat != 0;
    // ---- scores: lane = position, heads w and w + 4 ----
    const uint32_t pos = tile * TILE + lane;
    const bool valid = pos < n;
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
        const uint32_t gi = w + 4 * kk;
        if (gi >= G) break;
        int32_t b0 = 0, b1 = 0, b2 = 0, b3 = 0;
#pragma unroll
        for (int c = 0; c < (int)C8; c++) {
            const v4u kv = *(const v4u*)(&sm.k[lane][8 * c]);
            const v4u qv = *(const v4u*)(sm.q[gi] + 8 * c);
            b0 = dot2(kv.x, qv.x, b0);
            b1 = dot2(kv.y, qv.y, b1);
            b2 = dot2(kv.z, qv.z, b2);
            b3 = dot2(kv.w, qv.w, b3);
        }
        if (kcorr) {
#pragma unroll
            for (int c = 0; c < (int)C8; c++) {
                const v4u kv = *(const v4u*)(&sm.k[lane][8 * c]);
                const v4u cv = *(const v4u*)(sm.cq[gi] + 8 * c);
                b0 = dot2(sat_mask(kv.x), cv.x, b0);
                b1 = dot2(sat_mask(kv.y), cv.y, b1);
                b2 = dot2(sat_mask(kv.z), cv.z, b2);
                b3 = dot2(sat_mask(kv.w), cv.w, b3);
            }
        }
        // +2^31 (one saturating bank) wraps to INT32_MIN
        const int64_t t64 = (int64_t)(b0 == INT32_MIN ? INT32_MAX : b0) +
                            (b1 == INT32_MIN ? INT32_MAX : b1) +
                            (b2 == INT32_MIN ? INT32_MAX : b2) +
                            (b3 == INT32_MIN ? INT32_MAX : b3);
        int32_t ts = fx_sat32(t64);
        ts = rnd16_mul(ts, (int32_t)scale);  // scale = qk_scale << 8 <= 2^16
        const int32_t s = valid ? sat16_32(rnd32(ts, 8)) : INT16_MIN;
        const size_t base = (((size_t)t * a.num_kv_heads + h) * a.max_tiles + tile) * G + gi;
        const int32_t mx = wave_max(s);
        if (FUSED) {
            sc[kk] = s;
            mt[kk] = mx;
            if (lane == 0) {
                a.s_tmax[base] = (int16_t)mx;
                st_coherent(&a.s_gmax32[base], (int32_t)((a.epoch << 16) | (uint16_t)mx));
            }
        } else {
            a.s_scores[base * TILE + lane] = (int16_t)s;
            if (lane == 0) a.s_tmax[base] = (int16_t)mx;
        }
    }
    if (own / TILE == tile && tid < C8)  // this row's K into the cache
        *(v4u*)(a.kcache + page_off<D>(a, h, tile) + (own % TILE) * D + 8 * tid) =
            *(const v4u*)(sm.kv[t] + 8 * tid);
}

template <int D>
__global__ __launch_bounds__(GNT) void attention_gqa_scores_kernel(AttnArgs a) {
    __shared__ GqaScoresSmem<D> sm;
    GqaWg wg;
    if (!gqa_wg(a, wg)) return;
    int32_t sc[2], mt[2];
    GqaScoresLoads<D> L;
    gqa_scores_loads<D>(a, wg, L);
    gqa_scores_body<D, false>(a, wg, sm, L, sc, mt);
}

template <int D>
struct __attribute__((aligned(16))) GqaPvSmem {
    int16_t vt[D][TILE + 8];            // V^T of the tile (positions bank-paired), padded
    int16_t vb[8][D];                   // the block's V rows
    int16_t p[GMAXG][TILE], cp[GMAXG][TILE];  // probabilities, c(p), bank-paired
    int16_t e14[2056];                  // Q2.14 exp table
    int32_t mrun[GMAXG];                // running max before the tile, per head
    int32_t tsum[GMAXG];                // the tile's probability sums (SCAN)
    int16_t tv[GMAXG][D];               // the tile's values, staged (SCAN)
};

// One-launch GQA path: a context of at most kGqaFusedMaxTiles tiles, so that
// the maxima of the tiles before any tile (tile x G <= GNT x GPW words) are
// polled GPW words per thread.
constexpr uint32_t kGqaFusedMaxTiles = 257;
constexpr int GPW = (kGqaFusedMaxTiles - 1) * GMAXG / GNT;

// PV of a (row, KV head, tile) workgroup.  FUSED: the scores and tile
// maxima come from the same workgroup's scores phase (sci, mti), and the
// earlier tiles' maxima are awaited as tagged words (bounded); ok (LDS,
// 1 on entry) is cleared by a wavefront whose wait gave up, and the
// workgroup then returns false.
template <int D>
struct GqaPvLoads {
    static constexpr uint32_t VC = D * TILE / 8 / GNT;  // V^T chunks per thread
    static constexpr int NE = (257 + GNT - 1) / GNT;    // exp table pieces per thread
    static constexpr int NV = (8 * D + GNT - 1) / GNT;  // block V values per thread
    v4u ex[NE];
    v4u vc[VC];
    int16_t vx[NV];
};
// The PV phase's loads that depend on nothing computed (indices clamped:
// every load is issued): the exp table, the tile's V page, the block's V
// rows in the tile.
template <int D>
__device__ __forceinline__ void gqa_pv_loads(const AttnArgs& a, const GqaWg& wg,
                                             GqaPvLoads<D>& L) {
    const uint32_t t = wg.t, h = wg.h, tile = wg.tile, tid = threadIdx.x;
    const uint32_t own = a.pos0 + t;
#pragma unroll
    for (int u = 0; u < GqaPvLoads<D>::NE; u++) {
        const uint32_t c = tid + GNT * u;
        L.ex[u] = *(const v4u*)(a.exp14 + 8 * (c < 257 ? c : 256));
    }
    const uint32_t tp = tile < a.tiles ? tile : a.tiles - 1;
    const int16_t* vpage = a.vcache + page_off<D>(a, h, tp);
#pragma unroll
    for (int u = 0; u < (int)GqaPvLoads<D>::VC; u++) {
        const uint32_t i = tid + GNT * u;  // row i / 8, slots 8 (i % 8) ..
        L.vc[u] = *(const v4u*)(vpage + (i / 8) * TILE + 8 * (i % 8));
    }
    const GqaRows tr = gqa_rows(a, tile, own);
    const uint32_t nv = tr.nrow * D;
#pragma unroll
    for (int u = 0; u < GqaPvLoads<D>::NV; u++) {
        const uint32_t i = tid + GNT * u < nv ? tid + GNT * u : 0;
        L.vx[u] = a.qkv[(size_t)(tr.r0 + i / D) * a.ldqkv +
                        (size_t)(a.num_heads + a.num_kv_heads) * D + (size_t)h * D + i % D];
    }
}

template <int D, bool FUSED, bool SCAN = false>
__device__ __forceinline__ bool gqa_pv_body(const AttnArgs& a, const GqaWg& wg,
                                            GqaPvSmem<D>& sm, const GqaPvLoads<D>& L,
                                            const int32_t (&sci)[2],
                                            const int32_t (&mti)[2], uint32_t& ok_all) {
    static_assert(D == 64 || D == 128, "GQA tile path: head_dim 64 or 128");
    constexpr uint32_t VC = D * TILE / 8 / GNT;        // V^T chunks per thread
    constexpr int NE = (257 + GNT - 1) / GNT;          // exp table pieces per thread
    constexpr int NV = (8 * D + GNT - 1) / GNT;        // block V values per thread
    constexpr uint32_t NHS = GNT / D;                  // heads a PV pass covers at once
    const uint32_t t = wg.t, h = wg.h, tile = wg.tile, tid = threadIdx.x;
    const uint32_t n = a.pos0 + t + 1, own = n - 1, G = a.group;
    const uint32_t lane = tid & 63, w = tid >> 6;
    const size_t rh = (size_t)t * a.num_kv_heads + h;

    // ---- loads (issued by the caller: FUSED at the start of the launch) ----
    const v4u* ex = L.ex;
    const v4u* vc = L.vc;
    const int16_t* vx = L.vx;
    const GqaRows tr = gqa_rows(a, tile, own);
    const uint32_t nv = tr.nrow * D;
    // scores and this tile's maxima of heads w and w + 4 (lane = position)
    int32_t sc[2], mt[2];
    if (FUSED) {
        sc[0] = sci[0], sc[1] = sci[1], mt[0] = mti[0], mt[1] = mti[1];
    } else {
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            const uint32_t gi = w + 4 * kk < G ? w + 4 * kk : 0;
            const size_t base = (rh * a.max_tiles + tile) * G + gi;
            sc[kk] = a.s_scores[base * TILE + lane];
            mt[kk] = a.s_tmax[base];
        }
    }
    // maxima of the tiles before this one, (tile, head) pairs over threads
    constexpr int NPM = FUSED ? GPW : 4;
    int32_t pm[NPM];
    const uint32_t npm = tile * G;
    if (FUSED) {
        // the tagged words of the earlier tiles (contiguous: [0, tile) x G),
        // every one read until it carries this launch's epoch; a wavefront
        // waits for its own words, one that gives up clears sm.ok
        const int32_t* gm = a.s_gmax32 + rh * a.max_tiles * G;
        const TagWait tw{(uint64_t)wall_clock64(), a.wait_limit, a.abort, a.host_abort};
        bool waited = true;
        while (true) {
            bool ok = true;
#pragma unroll
            for (int u = 0; u < NPM; u++) {
                const uint32_t i = tid + GNT * u;
                const uint32_t wd = (uint32_t)ld_coherent(&gm[i < npm ? i : 0]);
                ok = ok && (i >= npm || tag_ok(wd, 16, a.epoch));
                pm[u] = i < npm ? (int32_t)(int16_t)(wd & 0xffffu) : INT16_MIN;
            }
            if (__all(ok)) break;
            if (!tw.keep_waiting()) {
                waited = false;
                break;
            }
        }
        if (!waited) ok_all = 0;
    } else {
#pragma unroll
        for (int u = 0; u < NPM; u++) {
            const uint32_t i = tid + GNT * u < npm ? tid + GNT * u : 0;
            pm[u] = npm ? a.s_tmax[(rh * a.max_tiles + i / G) * G + i % G] : INT16_MIN;
        }
    }
    // ---- staging ----
    if (tid < GMAXG) sm.mrun[tid] = INT16_MIN;
#pragma unroll
    for (int u = 0; u < NE; u++) {
        const uint32_t c = tid + GNT * u;
        if (c < 257) *(v4u*)(sm.e14 + 8 * c) = ex[u];
    }
    // slot groups holding no cached position: 0 (the block's positions are
    // written next, later ones meet probability 0)
#pragma unroll
    for (int u = 0; u < (int)VC; u++) {
        const uint32_t i = tid + GNT * u, e = i / 8, c8 = i % 8;
        *(v4u*)(&sm.vt[e][8 * c8]) = tile * TILE + 8 * c8 < a.pos0 ? vc[u] : v4u{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < NV; u++) {
        const uint32_t i = tid + GNT * u;
        if (i < nv) sm.vb[tr.r0 + i / D][i % D] = vx[u];
    }
    lds_barrier();
    if (FUSED && ok_all == 0) return false;  // uniform: read after the barrier
#pragma unroll
    for (int u = 0; u < NPM; u++) {
        const uint32_t i = tid + GNT * u;
        if (i < npm)
            __hip_atomic_fetch_max(&sm.mrun[i % G], pm[u], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (!FUSED) {
        for (uint32_t i = tid + GNT * NPM; i < npm; i += GNT)  // beyond 128 tiles x 8 heads
            __hip_atomic_fetch_max(&sm.mrun[i % G],
                                   (int32_t)a.s_tmax[(rh * a.max_tiles + i / G) * G + i % G],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    // the block's V rows into their slots
    for (uint32_t i = tid; i < nv; i += GNT) {
        const uint32_t r = tr.r0 + i / D, e = i % D;
        sm.vt[e][paired((a.pos0 + r) % TILE)] = sm.vb[r][e];
    }
    lds_barrier();
    // ---- probabilities under the running max after this tile ----
    const bool valid = tile * TILE + lane < n;
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
        const uint32_t gi = w + 4 * kk;
        if (gi >= G) break;
        const int32_t m0 = sm.mrun[gi];
        const int32_t mn = mt[kk] > m0 ? mt[kk] : m0;
        const int32_t pr = valid ? prob(sm.e14, sc[kk] - mn) : 0;
        sm.p[gi][paired(lane)] = (int16_t)pr;
        sm.cp[gi][paired(lane)] = (int16_t)sat_corr(pr);
        const int32_t tsum = wave_sum(pr);  // <= 64 * 16384
        if (lane == 0) {
            if (SCAN)
                sm.tsum[gi] = tsum;
            else
                a.s_tsum[(rh * a.max_tiles + tile) * G + gi] = tsum;
        }
    }
    lds_barrier();
    // ---- PV: element e, heads e_set + NHS k ----
    const uint32_t e = tid % D;
    v4u vr[TILE / 8];
    uint32_t mv = 0;
#pragma unroll
    for (int c = 0; c < TILE / 8; c++) vr[c] = clamp4(*(const v4u*)(&sm.vt[e][8 * c]), mv);
    const bool vcorr = __any(mv != 0);
    for (uint32_t gi = tid / D; gi < G; gi += NHS) {
        int32_t b0 = 0, b1 = 0, b2 = 0, b3 = 0;
#pragma unroll
        for (int c = 0; c < TILE / 8; c++) {
            const v4u pv = *(const v4u*)(sm.p[gi] + 8 * c);
            b0 = dot2(vr[c].x, pv.x, b0);
            b1 = dot2(vr[c].y, pv.y, b1);
            b2 = dot2(vr[c].z, pv.z, b2);
            b3 = dot2(vr[c].w, pv.w, b3);
        }
        if (vcorr) {
#pragma unroll
            for (int c = 0; c < TILE / 8; c++) {
                const v4u cv = *(const v4u*)(sm.cp[gi] + 8 * c);
                b0 = dot2(sat_mask(vr[c].x), cv.x, b0);
                b1 = dot2(sat_mask(vr[c].y), cv.y, b1);
                b2 = dot2(sat_mask(vr[c].z), cv.z, b2);
                b3 = dot2(sat_mask(vr[c].w), cv.w, b3);
            }
        }
        int32_t tv = fx_sat32((int64_t)b0 + b1 + b2 + b3);
        tv = sat16_32(rnd32(rnd32(tv, 6), 8));  // rnd(tv 2^10, 16) = rnd(tv, 6)
        if (SCAN)
            sm.tv[gi][e] = (int16_t)tv;
        else
            a.s_tval[((rh * a.max_tiles + tile) * G + gi) * D + e] = (int16_t)tv;
    }
    if (own / TILE == tile && tid < D)  // this row's V into the cache
        a.vcache[page_off<D>(a, h, tile) + tid * TILE + paired(own % TILE)] = sm.vb[t][tid];
    if (SCAN) {
        // the tile's G x D values (contiguous in s_tval) go out in 8-byte
        // device-coherent stores; once they are performed (every wavefront
        // waited for its stores) the sums go out tagged: a scan workgroup
        // that sees a sum's epoch reads the values after
        lds_barrier();
        uint64_t* dst = (uint64_t*)(a.s_tval + (rh * a.max_tiles + tile) * G * D);
        const uint64_t* src = (const uint64_t*)&sm.tv[0][0];
        for (uint32_t i = tid; i < G * D / 4; i += GNT) st_coherent(dst + i, src[i]);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid < G)
            st_coherent(&a.s_gsum64[(rh * a.max_tiles + tile) * G + tid],
                        ((uint64_t)a.epoch << 32) | (uint32_t)sm.tsum[tid]);
    }
    return true;
}

template <int D>
__global__ __launch_bounds__(GNT) void attention_gqa_pv_kernel(AttnArgs a) {
    __shared__ GqaPvSmem<D> sm;
    GqaWg wg;
    if (!gqa_wg(a, wg)) return;
    const int32_t none[2] = {0, 0};
    uint32_t unused = 1;
    GqaPvLoads<D> L;
    gqa_pv_loads<D>(a, wg, L);
    gqa_pv_body<D, false>(a, wg, sm, L, none, none, unused);
}

// 16 bytes of tile values read with device-coherent loads.
__device__ __forceinline__ v4u ld_coherent_v4(const int16_t* p) {
    const uint4 u = ld_coherent16(p);
    return v4u{u.x, u.y, u.z, u.w};
}

// Run r of the scan: tiles [a0, a0 + len) (len 0: empty), the rescale
// factor of its event (<< 2; r >= 1) and the running max before its tiles.
struct GqaRun {
    int64_t old;
    int32_t a0, len, mb, pad;
};

struct __attribute__((aligned(16))) GqaScanSmem {
    int32_t tm[GMAXT];          // tile maxima
    int32_t ts[GMAXT];          // tile sums
    int16_t run[GMAXT];         // run of each tile (0: before the first event)
    int16_t ev[GMAXT];          // tile of event k (run k + 1 starts there)
    int32_t rsum[GSLOTS][GSE];  // per run, per element: sum of the tile values
    int32_t rts[GSLOTS];        // per run: sum of the tile sums
    GqaRun ri[GSLOTS];          // per run: its tiles, rescale factor and running max
    int16_t e14[2056];
    int32_t nev, sum;
};

// The per-tile recurrence of the accumulator of one element over tiles
// [j0, j1) (the reference's order), from running max m.
template <bool FUSED>
__device__ __forceinline__ int32_t acc_tiles_seq(const AttnArgs& a, const GqaScanSmem& sm,
                                                 size_t tv0, uint32_t G, uint32_t D,
                                                 uint32_t j0, uint32_t j1, int32_t m,
                                                 int32_t acc) {
    for (uint32_t jb = j0; jb < j1; jb += 16) {
        int32_t tvv[16];  // sixteen tiles' values in flight
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const uint32_t j = jb + u < j1 ? jb + u : j0;
            const int16_t* src = a.s_tval + tv0 + (size_t)j * G * D;
            tvv[u] = FUSED ? ld_coherent(src) : *src;
        }
#pragma unroll
        for (int u = 0; u < 16; u++) {  // no early exit: tvv stays in registers
            const uint32_t j = jb + u;
            if (j < j1) {
                const int32_t tmv = sm.tm[j];
                if (tmv > m) {  // (the factor is at most 2^16)
                    acc = rnd16_mul(acc, (int32_t)prob(sm.e14, m - tmv) << 2);
                    m = tmv;
                }
                acc = __builtin_elementwise_add_sat(acc, tvv[u] * 256);
            }
        }
    }
    return acc;
}
// The same for the sum of the probabilities.
__device__ __forceinline__ int32_t sum_tiles_seq(const GqaScanSmem& sm, uint32_t j0,
                                                 uint32_t j1, int32_t m, int32_t sum) {
    for (uint32_t j = j0; j < j1; j++) {
        const int32_t tmv = sm.tm[j], tsk = sm.ts[j];
        if (tmv > m) {  // non-negative terms: nested saturating additions
            const int32_t old = (int32_t)prob(sm.e14, m - tmv) << 2;
            sum = __builtin_elementwise_add_sat(rnd16_mul(sum, old), tsk << 2);
            m = tmv;
        } else {
            sum = __builtin_elementwise_add_sat(sum, tsk << 2);
        }
    }
    return sum;
}

// The scan of workgroup `bid` (row, query head, 32 elements).  FUSED: a
// workgroup of the one-launch GQA kernel; the tile maxima and sums are
// awaited as tagged words (bounded; a wavefront that gives up clears
// ok_all and the workgroup returns) and the tile values read with
// device-coherent loads after their sums were seen.
template <int D, bool FUSED>
__device__ __forceinline__ void gqa_scan_body(const AttnArgs& a, GqaScanSmem& sm, uint32_t bid,
                                              uint32_t& ok_all) {
    static_assert(D == 64 || D == 128, "GQA tile path: head_dim 64 or 128");
    static_assert(kGqaFusedMaxTiles <= 2 * GNT, "two tagged words per thread");
    constexpr uint32_t ES = D / GSE;                // workgroups per (row, head)
    constexpr uint32_t C8 = GSE / 8, NSL = GNT / C8;  // element octets, tile slices
    constexpr int TVB = 8;                          // tile-value loads in flight per thread
    constexpr int NU = FUSED ? 2 : (int)(GMAXT / GNT);  // tiles per thread (maxima, sums)
    static_assert((kGqaFusedMaxTiles + NSL - 1) / NSL <= (uint32_t)TVB,
                  "FUSED: a thread's slice of tiles fits one batch of value loads");
    const uint32_t es = bid % ES, tg = bid / ES;
    const uint32_t t = tg / a.num_heads, g = tg % a.num_heads;
    if (t >= a.grid_rows) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t n = a.pos0 + t + 1, G = a.group, h = g / G, gi = g % G;
    const uint32_t ntiles = (n + TILE - 1) / TILE;  // <= GMAXT (the launcher's check)
    const size_t rh = (size_t)t * a.num_kv_heads + h;
    const size_t tv_base = (rh * a.max_tiles * G + gi) * D + GSE * es;  // + j G D + e
    // ---- every load that does not depend on another is issued first: tile
    // maxima and sums, the exp table, this thread's first tile values ----
    int32_t tmr[NU], tsr[NU];
    if (!FUSED) {
#pragma unroll
        for (int u = 0; u < NU; u++) {
            const uint32_t j = tid + GNT * u < ntiles ? tid + GNT * u : 0;
            tmr[u] = a.s_tmax[(rh * a.max_tiles + j) * G + gi];
            tsr[u] = a.s_tsum[(rh * a.max_tiles + j) * G + gi];
        }
    }
    const v4u exr = *(const v4u*)(a.exp14 + 8 * (tid < 257 ? tid : 256));
    const v4u exr2 = *(const v4u*)(a.exp14 + 8 * 256);
    const uint32_t oc = tid % C8, sl = tid / C8;
    const uint32_t per = (ntiles + NSL - 1) / NSL;
    const uint32_t j0 = sl * per, j1 = j0 + per < ntiles ? j0 + per : ntiles;
    const size_t tw0 = (rh * a.max_tiles) * G + gi;  // tagged word of tile j: tw0 + j G
    v4u ld[TVB];
    if (!FUSED) {
#pragma unroll
        for (int u = 0; u < TVB; u++) {
            const uint32_t j = j0 + u < j1 ? j0 + u : (j0 < j1 ? j0 : 0);
            ld[u] = *(const v4u*)(a.s_tval + tv_base + (size_t)j * G * D + 8 * oc);
        }
    } else {
        // the tile maxima, each read until it carries this launch's epoch
        const TagWait tw{(uint64_t)wall_clock64(), a.wait_limit, a.abort, a.host_abort};
        while (true) {
            bool ok = true;
#pragma unroll
            for (int u = 0; u < NU; u++) {
                const uint32_t j = tid + GNT * u;
                const uint32_t wd = (uint32_t)ld_coherent(&a.s_gmax32[tw0 + (size_t)(j < ntiles ? j : 0) * G]);
                ok = ok && (j >= ntiles || tag_ok(wd, 16, a.epoch));
                tmr[u] = (int32_t)(int16_t)(wd & 0xffffu);
            }
            if (__all(ok)) break;
            if (!tw.keep_waiting()) {
                ok_all = 0;
                break;
            }
        }
    }
#pragma unroll
    for (int u = 0; u < NU; u++) {
        const uint32_t j = tid + GNT * u;
        if (j < ntiles) {
            sm.tm[j] = tmr[u];
            if (!FUSED) sm.ts[j] = tsr[u];
        }
    }
    if (tid < 257) *(v4u*)(sm.e14 + 8 * tid) = exr;
    if (tid == 0) *(v4u*)(sm.e14 + 8 * 256) = exr2;
    for (uint32_t i = tid; i < GSLOTS * GSE; i += GNT) (&sm.rsum[0][0])[i] = 0;
    if (tid < GSLOTS) sm.rts[tid] = 0;
    lds_barrier();
    if (FUSED && ok_all == 0) return;  // uniform: read after the barrier
    // ---- events (wavefront 0): tiles whose maximum exceeds every earlier
    // one and the initial -128.0; run of a tile = events at or before it.
    // Lane L holds tiles [L T, L T + T).
    if (tid < 64) {
        const uint32_t T = (ntiles + 63) / 64;
        const uint32_t b0 = lane * T, b1 = b0 + T < ntiles ? b0 + T : ntiles;
        int32_t v = INT32_MIN;
        for (uint32_t j = b0; j < b1; j++) v = sm.tm[j] > v ? sm.tm[j] : v;
#pragma unroll
        for (uint32_t off = 1; off < 64; off <<= 1) {
            const int32_t o = __shfl_up(v, off, 64);
            if (lane >= off) v = o > v ? o : v;
        }
        const int32_t before = __shfl_up(v, 1, 64);
        int32_t m = lane && before > INT16_MIN ? before : INT16_MIN;  // running max before b0
        uint32_t mask = 0, cnt = 0;
        for (uint32_t j = b0; j < b1; j++) {
            if (sm.tm[j] > m) {
                m = sm.tm[j];
                mask |= 1u << (j - b0);
                cnt++;
            }
        }
        uint32_t c = cnt;
#pragma unroll
        for (uint32_t off = 1; off < 64; off <<= 1) {
            const uint32_t o = __shfl_up(c, off, 64);
            if (lane >= off) c += o;
        }
        uint32_t k = c - cnt;  // events before tile b0
        for (uint32_t j = b0; j < b1; j++) {
            if (mask & (1u << (j - b0))) sm.ev[k++] = (int16_t)j;
            sm.run[j] = (int16_t)k;
        }
        if (lane == 63) sm.nev = (int32_t)c;
        // run r's operands (lane r), from the events alone: run r covers
        // tiles [ev[r - 1], ev[r]) (run 0 from tile 0, the last to the
        // end); run r >= 1 starts at event tile ev[r - 1], whose maximum
        // replaces that of the event before it (or -128.0), which is also
        // the running max before the run
        const uint32_t nw = __builtin_amdgcn_readlane(c, 63);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (nw + 1 <= GSLOTS && lane <= nw) {
            const uint32_t a0 = lane == 0 ? 0 : (uint32_t)sm.ev[lane - 1];
            const uint32_t a1 = lane == nw ? ntiles : (uint32_t)sm.ev[lane];
            const int32_t mprev = lane >= 2 ? sm.tm[sm.ev[lane - 2]] : INT16_MIN;
            GqaRun ru;
            ru.old = lane ? (int64_t)prob(sm.e14, mprev - sm.tm[a0]) << 2 : 0;
            ru.a0 = (int32_t)a0;
            ru.len = a1 > a0 ? (int32_t)(a1 - a0) : 0;
            ru.mb = mprev;
            ru.pad = 0;
            sm.ri[lane] = ru;
        }
    }
    int32_t tsl[TVB];  // FUSED: the sums of this thread's slice of tiles
    lds_barrier();  // the events
    if (FUSED) {
        // the sums of this thread's slice of tiles (tagged after the tiles'
        // values were performed; the slice has at most TVB tiles), then the
        // slice's values, while later tiles may still be running
        const TagWait tw{(uint64_t)wall_clock64(), a.wait_limit, a.abort, a.host_abort};
        while (true) {
            bool ok = true;
#pragma unroll
            for (int u = 0; u < TVB; u++) {
                const uint32_t j = j0 + u;
                const uint64_t wd = ld_coherent(&a.s_gsum64[tw0 + (size_t)(j < j1 ? j : 0) * G]);
                ok = ok && (j >= j1 || (uint32_t)(wd >> 32) == a.epoch);
                tsl[u] = (int32_t)(uint32_t)wd;
            }
            if (__all(ok)) break;
            if (!tw.keep_waiting()) {
                ok_all = 0;
                break;
            }
        }
#pragma unroll
        for (int u = 0; u < TVB; u++) {
            const uint32_t j = j0 + u < j1 ? j0 + u : (j0 < j1 ? j0 : 0);
            ld[u] = ld_coherent_v4(a.s_tval + tv_base + (size_t)j * G * D + 8 * oc);
        }
        if (oc == 0) {
#pragma unroll
            for (int u = 0; u < TVB; u++)
                if (j0 + u < j1) sm.ts[j0 + u] = tsl[u];
        }
    }
    const uint32_t nev = (uint32_t)sm.nev;
    const bool parallel = nev + 1 <= GSLOTS;
    if (parallel) {
        // ---- per run: sums of the tile values (this thread's slice of
        // consecutive tiles, flushed into LDS when the run changes), tile
        // sums and lengths, and the rescale factor of its event ----
        int32_t part[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int32_t cur = j0 < j1 ? sm.run[j0] : 0;
        for (uint32_t jb = j0; jb < j1; jb += TVB) {
            if (jb != j0) {
#pragma unroll
                for (int u = 0; u < TVB; u++) {
                    const uint32_t j = jb + u < j1 ? jb + u : j0;
                    const int16_t* src = a.s_tval + tv_base + (size_t)j * G * D + 8 * oc;
                    ld[u] = FUSED ? ld_coherent_v4(src) : *(const v4u*)src;
                }
            }
#pragma unroll
            for (int u = 0; u < TVB; u++) {  // no early exit: ld stays in registers
                const uint32_t j = jb + u;
                if (j < j1) {
                    const int32_t r = sm.run[j];
                    if (r != cur) {
#pragma unroll
                        for (int q = 0; q < 8; q++) {
                            atomicAdd(&sm.rsum[cur][8 * oc + q], part[q]);
                            part[q] = 0;
                        }
                        cur = r;
                    }
                    const uint32_t wv[4] = {ld[u].x, ld[u].y, ld[u].z, ld[u].w};
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        part[2 * q] += (int16_t)(wv[q] & 0xffff);
                        part[2 * q + 1] += (int16_t)(wv[q] >> 16);
                    }
                }
            }
        }
        if (j0 < j1) {
#pragma unroll
            for (int q = 0; q < 8; q++) atomicAdd(&sm.rsum[cur][8 * oc + q], part[q]);
        }
        if (oc == 0) {  // the slice's tile sums into their runs
            if (FUSED) {
#pragma unroll
                for (int u = 0; u < TVB; u++)
                    if (j0 + u < j1) atomicAdd(&sm.rts[sm.run[j0 + u]], tsl[u]);
            } else {
                for (uint32_t j = j0; j < j1; j++) atomicAdd(&sm.rts[sm.run[j]], sm.ts[j]);
            }
        }
        lds_barrier();
        if (FUSED && ok_all == 0) return;  // uniform: read after the barrier
        // ---- the sum of the probabilities, once per workgroup (lane 0 of
        // the second wavefront, beside the elements' chains); the next
        // run's operands are read while a run is computed ----
        if (tid == 64) {
            int32_t sum = 0;
            GqaRun nx = sm.ri[0];
            int32_t tsn = sm.rts[0];
            for (uint32_t r = 0; r <= nev; r++) {
                const GqaRun cu = nx;
                const int32_t ts = tsn;
                const uint32_t rn = r < nev ? r + 1 : r;
                nx = sm.ri[rn];
                tsn = sm.rts[rn];
                if (cu.len == 0) continue;
                const int64_t sumr = r ? rnd16_mul(sum, (int32_t)cu.old) : sum;
                const int64_t t4 = (int64_t)ts << 2;
                if (sumr + t4 <= INT32_MAX)
                    sum = (int32_t)(sumr + t4);
                else
                    sum = sum_tiles_seq(sm, cu.a0, cu.a0 + cu.len, cu.mb, sum);
            }
            sm.sum = sum;
        }
    } else {
        if (FUSED) {
            lds_barrier();  // every slice's sums
            if (ok_all == 0) return;
        }
        if (tid == 64) sm.sum = sum_tiles_seq(sm, 0, ntiles, INT16_MIN, 0);
    }
    // ---- the accumulator, one element per thread: one step per run when
    // no partial sum of the run can reach the int32 bounds (tile values
    // << 8 are within 2^23 in magnitude), else the run tile by tile ----
    int32_t acc = 0;
    if (tid < GSE) {
        const size_t tv0 = tv_base + tid;
        if (!parallel) {
            acc = acc_tiles_seq<FUSED>(a, sm, tv0, G, D, 0, ntiles, INT16_MIN, 0);
        } else {
            GqaRun nx = sm.ri[0];
            int32_t rsn = sm.rsum[0][tid];
            for (uint32_t r = 0; r <= nev; r++) {
                const GqaRun cu = nx;
                const int32_t rs = rsn;
                const uint32_t rn = r < nev ? r + 1 : r;
                nx = sm.ri[rn];
                rsn = sm.rsum[rn][tid];
                if (cu.len == 0) continue;
                const int32_t accr = r ? rnd16_mul(acc, (int32_t)cu.old) : acc;
                const int64_t aa = accr < 0 ? -(int64_t)accr : accr;
                if (aa + ((int64_t)cu.len << 23) <= INT32_MAX)
                    acc = accr + rs * 256;
                else
                    acc = acc_tiles_seq<FUSED>(a, sm, tv0, G, D, cu.a0, cu.a0 + cu.len, cu.mb, acc);
            }
        }
    }
    lds_barrier();  // the sum
    if (tid < GSE)
        a.out[(size_t)t * a.ldo + (size_t)g * D + GSE * es + tid] =
            sat16_32(rnd16_mul(acc, fx_inv_sum(sm.sum)));
}

template <int D>
__global__ __launch_bounds__(GNT) void attention_gqa_scan_kernel(AttnArgs a) {
    __shared__ GqaScanSmem sm;
    uint32_t unused = 1;
    gqa_scan_body<D, false>(a, sm, blockIdx.x, unused);
}

template <int D, bool SCAN>
union GqaFusedSmem {
    GqaScoresSmem<D> s;
    GqaPvSmem<D> p;
};
template <int D>
union GqaFusedSmem<D, true> {
    GqaScoresSmem<D> s;
    GqaPvSmem<D> p;
    GqaScanSmem c;
};

// Scores and PV in one launch (at most kGqaFusedMaxTiles tiles; launched
// only when the whole grid fits on the device at once, so that the tiles a
// workgroup waits for are all running): the scores phase publishes the
// tile's tagged maxima, the PV phase issues its loads, then waits for the
// earlier tiles' maxima.  SCAN: the scan's workgroups follow the tiles'
// in the same grid; the tiles publish their sums tagged after their
// values, and each scan workgroup forms its events as soon as the maxima
// are in, while the tiles' PV phases run.
template <int D, bool SCAN>
__global__ __launch_bounds__(GNT) void attention_gqa_fused_kernel(AttnArgs a) {
    __shared__ GqaFusedSmem<D, SCAN> sm;
    __shared__ uint32_t ok_all;
    if (SCAN) {
        const uint32_t tile_wgs = a.grid_rows * a.grid_tiles * a.num_kv_heads;
        if (blockIdx.x >= tile_wgs) {
            if (threadIdx.x == 0) ok_all = 1;
            __syncthreads();
            if constexpr (SCAN) gqa_scan_body<D, true>(a, sm.c, blockIdx.x - tile_wgs, ok_all);
            return;
        }
    }
    GqaWg wg;
    if (!gqa_wg(a, wg)) return;
    if (threadIdx.x == 0) ok_all = 1;  // ordered by the scores phase's barriers
    // both phases' loads first (the V page arrives while the scores are
    // computed: loads complete in order, the K page's first)
    GqaScoresLoads<D> LS;
    gqa_scores_loads<D>(a, wg, LS);
    GqaPvLoads<D> LP;
    gqa_pv_loads<D>(a, wg, LP);
    int32_t sc[2], mt[2];
    gqa_scores_body<D, true>(a, wg, sm.s, LS, sc, mt);
    __syncthreads();  // the scores phase's LDS use ends
    gqa_pv_body<D, true, SCAN>(a, wg, sm.p, LP, sc, mt, ok_all);
}

// Workgroups of the one-launch GQA kernel the device holds at once (the
// per-CU occupancy of the gfx950 code object, queried once under C++'s
// thread-safe initialisation of a local static).
template <int D, bool SCAN>
uint32_t gqa_fused_capacity(uint32_t cus) {
    static const int per_cu = [] {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nb, reinterpret_cast<const void*>(&attention_gqa_fused_kernel<D, SCAN>), GNT,
                0) != hipSuccess)
            nb = 0;
        return nb;
    }();
    return (uint32_t)per_cu * cus;
}

template <int D>
hipError_t launch_gqa_d(const AttnArgs& a, uint32_t rows, uint32_t tiles, hipStream_t st) {
    AttnArgs g = a;
    g.grid_rows = rows;
    g.grid_tiles = tiles;
    const uint32_t grid = rows * tiles * a.num_kv_heads;
    const uint32_t scan_grid = rows * a.num_heads * (D / GSE);
    const bool one = a.epoch && a.s_gmax32 && tiles <= kGqaFusedMaxTiles;
    hipError_t e;
    // The one-launch kernels, cooperatively when a.coop: a grid the device
    // cannot hold at once is refused and the next variant is taken.
    auto coop_launch = [&](const void* fn, uint32_t n) -> hipError_t {
        void* args[] = {&g};
        const hipError_t r = hipLaunchCooperativeKernel(fn, dim3(n), dim3(GNT), args, 0, st);
        if (r == hipErrorCooperativeLaunchTooLarge) (void)hipGetLastError();
        return r;
    };
    if (one && a.s_gsum64 && grid + scan_grid <= gqa_fused_capacity<D, true>(a.cus)) {
        if (!a.coop) {
            attention_gqa_fused_kernel<D, true><<<grid + scan_grid, GNT, 0, st>>>(g);
            return hipGetLastError();
        }
        e = coop_launch(reinterpret_cast<const void*>(&attention_gqa_fused_kernel<D, true>),
                        grid + scan_grid);
        if (e != hipErrorCooperativeLaunchTooLarge) return e;
    }
    bool one_done = false;
    if (one && grid <= gqa_fused_capacity<D, false>(a.cus)) {
        if (!a.coop) {
            attention_gqa_fused_kernel<D, false><<<grid, GNT, 0, st>>>(g);
            e = hipGetLastError();
        } else {
            e = coop_launch(reinterpret_cast<const void*>(&attention_gqa_fused_kernel<D, false>),
                            grid);
        }
        if (e != hipSuccess && e != hipErrorCooperativeLaunchTooLarge) return e;
        one_done = e == hipSuccess;
    }
    if (!one_done) {
        attention_gqa_scores_kernel<D><<<grid, GNT, 0, st>>>(g);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        attention_gqa_pv_kernel<D><<<grid, GNT, 0, st>>>(g);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    attention_gqa_scan_kernel<D><<<scan_grid, GNT, 0, st>>>(g);
    return hipGetLastError();
}

}  // namespace

bool attention_gqa_ok(const AttnArgs& a, uint32_t rows) {
    const uint32_t tiles = (a.pos0 + rows + TILE - 1) / TILE;
    return (a.head_dim == 64 || a.head_dim == 128) && a.group >= 1 && a.group <= GMAXG &&
           a.num_heads == a.group * a.num_kv_heads && rows >= 1 && rows <= 8 &&
           tiles <= GMAXT && tiles <= a.max_tiles && tiles <= a.tiles;
}

hipError_t launch_attention_gqa(const AttnArgs& a, uint32_t rows, hipStream_t st) {
    if (!attention_gqa_ok(a, rows)) return hipErrorInvalidValue;
    const uint32_t tiles = (a.pos0 + rows + TILE - 1) / TILE;
    return a.head_dim == 64 ? launch_gqa_d<64>(a, rows, tiles, st)
                            : launch_gqa_d<128>(a, rows, tiles, st);
}

}  // namespace llm
