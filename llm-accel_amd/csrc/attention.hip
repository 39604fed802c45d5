// attention.hip -- RoPE + KV append + tiled online-softmax attention.
//
// Arithmetic is golden_tiled_flash_attention_q2_14 (raw-payload semantics,
// reference host/host_qwen_8x64.cpp:3609-3738) == the resident controller
// (kernel/control_cache_8x64.cpp:5491-5765): 64-position tiles anchored at
// position 0, QK and PV in four k-mod-4 Q16.16 banks of AP_RND-narrowed
// Q8.8 x Q4.12 products, Q2.14 probabilities, per-tile rounding of the
// running sum and accumulator.
//
// Exact integer form of one product.  The K (or V) operand is a Q8.8 value
// k converted to Q4.12 with saturation at +-8:
//   k in [-2048, 2047]:  16k exactly, so rnd(q * 16k, 4) = q * k;
//   k <= -2048:          -32768 = 16 * -2048, so the product is q * -2048;
//   k >= 2048:           32767, and rnd(q * 32767, 4) = 2048 q + c(q) with
//                        c(q) = floor((8 - q) / 16).
// So product = q * clamp(k, -2048, 2048) + [k >= 2048] * c(q).  The staged
// operand is clamp(k, -2048, 2048); a staged value equals 2048 exactly when
// k >= 2048, so the mask is recovered from the staged value itself.  A bank
// sum is one v_dot2_i32_i16 chain over the clamped operand plus, only in
// tiles that hold a value >= 2048, a second chain of the 0/1 mask against
// precomputed c(q).  Rows are staged with each 8-element group permuted to
// [0 4 1 5 2 6 3 7], so dword j of a group holds elements j and j + 4 of
// the same bank (index mod 4 = j).
//
// Bank range.  QK banks hold <= 32 products (head_dim <= 128) in
// [-2^26 + 2048, 2^26], so only the last addition can leave the Q16.16
// range and only at exactly +2^31; the reference saturates that to
// 2^31 - 1.  In 32-bit wrapping arithmetic +2^31 reads as INT32_MIN, a
// value no true bank sum can take, and is mapped back.  PV banks hold <= 16
// products of magnitude <= 2^25 and never leave the range.
//
// Cache layout: pages of 64 positions of one (layer, KV head), page
// (layer * kv_heads + head) * tiles + tile.  K page [64][d] with each row's
// elements in the bank-paired order; V page transposed [d][64] with
// positions in the bank-paired order, so staging a tile is a straight
// 16-byte copy.
//
// A workgroup issues all of its global loads for a tile at once (queries,
// RoPE rows and the exp table ride with the first tile, and the next
// tile's loads are issued before the current tile is computed).  The K / V
// rows a workgroup appends to the cache are parked in LDS and stored after
// its last barrier.
//
// Long contexts: the running max over tiles is a prefix max (exact), so
// tiles are split over workgroups: (A) scores and per-tile maxima, (B)
// probabilities, tile sums and per-tile PV values given the prefix max,
// and a sequential scan of the per-tile rounding recurrence performed by
// the last workgroup of each (row, KV head) to finish (atomic counter, no
// waiting).
#include "attention.h"

#include "attn_common.h"
#include "coherent.h"
#include "fixed_point.h"
#include "proj_common.h"
#include "split_head.h"

namespace llm {

namespace {

constexpr int MAXG = 16;
constexpr uint32_t kHeadPathRows = 2;  // rows per block taking the head path
#ifndef LLM_SPLIT_HEAD_ROWS
#define LLM_SPLIT_HEAD_ROWS 8
#endif
// rows per block taking the split-head path (head_dim a multiple of 32)
constexpr uint32_t kSplitHeadRows = LLM_SPLIT_HEAD_ROWS;
#ifndef LLM_SPLIT_HEAD_MAX_TILES
#define LLM_SPLIT_HEAD_MAX_TILES 4
#endif
// head_dim a multiple of 32: contexts of up to this many tiles take the
// split-head path (one launch, tiles in sequence), longer ones the tile
// path (two launches, tiles in parallel)
constexpr uint32_t kSplitHeadMaxTiles = LLM_SPLIT_HEAD_MAX_TILES;

constexpr int NT = 512;          // threads per workgroup
constexpr int NW = NT / 64;      // wavefronts per workgroup
constexpr int VROW = TILE + 8;   // padded LDS row of the V^T tile (int16)

template <int D>
struct __attribute__((aligned(16))) Smem {
    static constexpr int KROW = D + 8;  // padded LDS row of the K tile
    int16_t q[MAXG * D];     // rotated queries, bank-paired
    int16_t cq[MAXG * D];    // c(q) of every query element
    int16_t p[MAXG * TILE];  // Q2.14 probabilities, positions paired
    int16_t cp[MAXG * TILE]; // c(p)
    int16_t e14[2056];       // Q2.14 exp table, x = -2048..0
    int16_t k[TILE * KROW];  // clamped K tile, rows bank-paired
    int16_t vt[D * VROW];    // clamped V tile transposed
    int16_t app_k[D];        // the appended K row (after RoPE), paired
    int16_t app_v[D];        // the appended V row
    int32_t wflags[NW];      // per wave: bit 0 K tile has a value >= 2048,
                             // bit 1 V tile has one
    uint32_t last;           // this workgroup finishes the scan
};

// Each wave publishes whether its lanes staged a saturating K / V value;
// read back after the barrier that follows.
template <int D>
__device__ __forceinline__ void publish_flags(Smem<D>& sm, uint32_t any_k,
                                              uint32_t any_v) {
    const uint64_t bk = __ballot(any_k != 0), bv = __ballot(any_v != 0);
    if ((threadIdx.x & 63) == 0)
        sm.wflags[threadIdx.x >> 6] = (bk ? 1 : 0) | (bv ? 2 : 0);
}
template <int D>
__device__ __forceinline__ int32_t read_flags(const Smem<D>& sm) {
    int32_t f = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) f |= sm.wflags[w];
    return f;
}

// Four RoPE pairs (elements c..c+3 and c+d/2..c+d/2+3) of one vector.
struct RopeItem {
    v2u x0, x1, cs, sn;
};
template <int D>
__device__ __forceinline__ void issue_rope_item(const int16_t* vec,
                                                const int16_t* rope_row,
                                                uint32_t c, RopeItem& r) {
    r.x0 = *(const v2u*)(vec + c);
    r.x1 = *(const v2u*)(vec + D / 2 + c);
    r.cs = *(const v2u*)(rope_row + c);
    r.sn = *(const v2u*)(rope_row + D / 2 + c);
}


// Registers of one tile's loads.
template <int D>
struct TileLoad {
    static constexpr int KPER = (TILE * (D / 8) + NT - 1) / NT;
    static constexpr int VPER = (D * (TILE / 8) + NT - 1) / NT;
    v4u kpg[KPER];  // cached K rows, 16-byte chunks
    RopeItem kcur;    // current-block K, four RoPE pairs
    v4u vpg[VPER];  // cached V^T rows, 8 paired positions
    v4u vcur;       // current-block V row, 8 elements
};

// One tile of one row: positions [tile * 64, tile * 64 + tl) of which the
// first ncache are in the cache and the rest are rows of this block.
struct TileGeo {
    uint32_t tile, tl, ncache;
};
__device__ __forceinline__ TileGeo tile_geo(const AttnArgs& a, uint32_t n,
                                            uint32_t tile) {
    TileGeo g;
    const uint32_t base = tile * TILE;
    g.tile = tile;
    g.tl = n - base < TILE ? n - base : TILE;
    g.ncache = a.pos0 > base ? (a.pos0 - base < g.tl ? a.pos0 - base : g.tl) : 0;
    return g;
}

template <int D>
__device__ __forceinline__ void issue_k(const AttnArgs& a, uint32_t h, const TileGeo& tg,
                        TileLoad<D>& L) {
    constexpr uint32_t chunks = D / 8, items = D / 8;  // items: 4 pairs
    const int16_t* page = a.kcache + page_off<D>(a, h, tg.tile);
#pragma unroll
    for (int u = 0; u < TileLoad<D>::KPER; u++) {
        const uint32_t idx = threadIdx.x + NT * u;
        if (idx < tg.ncache * chunks)
            L.kpg[u] = *(const v4u*)(page + (idx / chunks) * D + 8 * (idx % chunks));
    }
    const uint32_t idx = threadIdx.x;
    if (idx < (tg.tl - tg.ncache) * items) {
        const uint32_t pos = tg.tile * TILE + tg.ncache + idx / items;
        const int16_t* k = a.qkv + (size_t)(pos - a.pos0) * a.ldqkv +
                           a.num_heads * D + h * D;
        issue_rope_item<D>(k, a.rope + (size_t)pos * D, 4 * (idx % items), L.kcur);
    }
}

template <int D>
__device__ __forceinline__ void issue_v(const AttnArgs& a, uint32_t h, const TileGeo& tg,
                        TileLoad<D>& L) {
    constexpr uint32_t cpr = TILE / 8;  // chunks per V^T row
    const int16_t* page = a.vcache + page_off<D>(a, h, tg.tile);
#pragma unroll
    for (int u = 0; u < TileLoad<D>::VPER; u++) {
        const uint32_t idx = threadIdx.x + NT * u;
        const uint32_t e = idx / cpr, c = idx % cpr;
        if (e < D && 8 * c < tg.ncache)
            L.vpg[u] = *(const v4u*)(page + e * TILE + 8 * c);
    }
    const uint32_t idx = threadIdx.x;
    if (idx < (tg.tl - tg.ncache) * (D / 8)) {
        const uint32_t pos = tg.tile * TILE + tg.ncache + idx / (D / 8);
        L.vcur = *(const v4u*)(a.qkv + (size_t)(pos - a.pos0) * a.ldqkv +
                                 (a.num_heads + a.num_kv_heads) * D + h * D +
                                 8 * (idx % (D / 8)));
    }
}

// K into LDS: cached rows clamped; current rows rotated and clamped; the
// row at absolute position `own` is also parked in app_k (unclamped).
// Returns nonzero when a staged value saturates.
template <int D>
__device__ __forceinline__ uint32_t commit_k(Smem<D>& sm, const TileGeo& tg,
                             const TileLoad<D>& L, uint32_t own) {
    constexpr uint32_t chunks = D / 8, items = D / 8;
    uint32_t any = 0;
#pragma unroll
    for (int u = 0; u < TileLoad<D>::KPER; u++) {
        const uint32_t idx = threadIdx.x + NT * u;
        if (idx < tg.ncache * chunks)
            *(v4u*)(sm.k + (idx / chunks) * Smem<D>::KROW + 8 * (idx % chunks)) =
                clamp4(L.kpg[u], any);
    }
    const uint32_t idx = threadIdx.x;
    if (idx < (tg.tl - tg.ncache) * items) {
        const uint32_t p = tg.ncache + idx / items, c = 4 * (idx % items);
        const bool app = tg.tile * TILE + p == own;
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) {
            int32_t y0, y1;
            rope_pair(half16(L.kcur.x0, j), half16(L.kcur.x1, j),
                      half16(L.kcur.cs, j), half16(L.kcur.sn, j), y0, y1);
            const uint32_t e0 = paired(c + j), e1 = paired(D / 2 + c + j);
            sm.k[p * Smem<D>::KROW + e0] = (int16_t)clamp_k(y0);
            sm.k[p * Smem<D>::KROW + e1] = (int16_t)clamp_k(y1);
            any |= (y0 >= 2048) | (y1 >= 2048);
            if (app) {
                sm.app_k[e0] = (int16_t)y0;
                sm.app_k[e1] = (int16_t)y1;
            }
        }
    }
    return any;
}

// V^T into LDS.  Cached chunks are copied whole, or slot by slot where the
// chunk also holds current positions; current rows go to their own slots,
// so the two writers touch disjoint bytes.  Slots at or beyond the row's
// context keep whatever they hold: their probabilities are 0 and c(0) = 0.
// Returns nonzero when a staged value saturates.
template <int D>
__device__ __forceinline__ uint32_t commit_v(Smem<D>& sm, const TileGeo& tg,
                             const TileLoad<D>& L, uint32_t own) {
    constexpr uint32_t cpr = TILE / 8;
    uint32_t any = 0;
#pragma unroll
    for (int u = 0; u < TileLoad<D>::VPER; u++) {
        const uint32_t idx = threadIdx.x + NT * u;
        const uint32_t e = idx / cpr, c = idx % cpr;
        if (e >= D || 8 * c >= tg.ncache) continue;
        const v4u cl = clamp4(L.vpg[u], any);
        int16_t* dst = sm.vt + e * VROW + 8 * c;
        if (8 * c + 8 <= tg.ncache) {
            *(v4u*)dst = cl;
        } else {
#pragma unroll
            for (uint32_t j = 0; j < 8; j++)
                if (8 * c + slot_pos(j) < tg.ncache) dst[j] = (int16_t)half16(cl, j);
        }
    }
    const uint32_t idx = threadIdx.x;
    if (idx < (tg.tl - tg.ncache) * (D / 8)) {
        const uint32_t p = tg.ncache + idx / (D / 8), c = 8 * (idx % (D / 8));
        const bool app = tg.tile * TILE + p == own;
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) {
            const int32_t v = half16(L.vcur, j);
            sm.vt[(c + j) * VROW + paired(p)] = (int16_t)clamp_k(v);
            any |= v >= 2048;
            if (app) sm.app_v[c + j] = (int16_t)v;
        }
    }
    return any;
}

// Prologue registers: one query item (four RoPE pairs) and the exp table.
struct ProLoad {
    RopeItem q;
    v4u e;
};

template <int D>
__device__ __forceinline__ void issue_prologue(const AttnArgs& a, uint32_t t, uint32_t h,
                               bool queries, bool exp_table, ProLoad& P) {
    constexpr uint32_t items = D / 8;
    const uint32_t tid = threadIdx.x;
    if (exp_table && tid < 257) P.e = *(const v4u*)(a.exp14 + 8 * tid);
    if (queries && tid < a.group * items) {
        const uint32_t pos = a.pos0 + t;
        const int16_t* q = a.qkv + (size_t)t * a.ldqkv +
                           (size_t)(h * a.group + tid / items) * D;
        issue_rope_item<D>(q, a.rope + (size_t)pos * D, 4 * (tid % items), P.q);
    }
}

template <int D>
__device__ __forceinline__ void commit_prologue(const AttnArgs& a, Smem<D>& sm, bool queries,
                                bool exp_table, const ProLoad& P) {
    constexpr uint32_t items = D / 8;
    const uint32_t tid = threadIdx.x;
    if (exp_table && tid < 257) *(v4u*)(sm.e14 + 8 * tid) = P.e;
    if (queries && tid < a.group * items) {
        const uint32_t g = tid / items, c = 4 * (tid % items);
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) {
            int32_t y0, y1;
            rope_pair(half16(P.q.x0, j), half16(P.q.x1, j), half16(P.q.cs, j),
                      half16(P.q.sn, j), y0, y1);
            const uint32_t e0 = g * D + paired(c + j), e1 = g * D + paired(D / 2 + c + j);
            sm.q[e0] = (int16_t)y0;
            sm.q[e1] = (int16_t)y1;
            sm.cq[e0] = (int16_t)sat_corr(y0);
            sm.cq[e1] = (int16_t)sat_corr(y1);
        }
    }
}

template <int D>
__device__ __forceinline__ void load_k_row(const Smem<D>& sm, uint32_t p, v4u* kr) {
#pragma unroll
    for (int c = 0; c < D / 8; c++)
        kr[c] = *(const v4u*)(sm.k + p * Smem<D>::KROW + 8 * c);
}
template <int D>
__device__ __forceinline__ void load_v_row(const Smem<D>& sm, uint32_t e, v4u* vr) {
#pragma unroll
    for (int c = 0; c < TILE / 8; c++) vr[c] = *(const v4u*)(sm.vt + e * VROW + 8 * c);
}

template <int D>
__device__ __forceinline__ void put_prob(Smem<D>& sm, uint32_t g, uint32_t lane,
                                         int32_t pr) {
    sm.p[g * TILE + paired(lane)] = (int16_t)pr;
    sm.cp[g * TILE + paired(lane)] = (int16_t)sat_corr(pr);
}

// The parked K / V rows of position `own` into their cache pages (after
// the workgroup's last barrier).
template <int D>
__device__ __forceinline__ void store_appended(const AttnArgs& a, const Smem<D>& sm, uint32_t h,
                               uint32_t own, bool k, bool v) {
    const uint32_t tile = own / TILE, slot = own % TILE;
    const uint32_t tid = threadIdx.x;
    if (k && tid < D / 8)
        *(v4u*)(a.kcache + page_off<D>(a, h, tile) + slot * D + 8 * tid) =
            *(const v4u*)(sm.app_k + 8 * tid);
    if (v && tid < D)
        a.vcache[page_off<D>(a, h, tile) + tid * TILE + paired(slot)] = sm.app_v[tid];
}

// Running state of the per-tile recurrence of one (query head, element).
struct ScanState {
    int32_t m, sum, acc;
};

// Tiles [j0, j1) of the recurrence, one by one (a chunk in which the
// running max rises, or whose sums could saturate).
template <int D>
__device__ __noinline__ ScanState scan_tiles(const int16_t* s_tval, const int16_t* s_tmax,
                                             const int32_t* s_tsum, const int16_t* e14,
                                             size_t row0, uint32_t G, uint32_t g,
                                             uint32_t e, uint32_t j0, uint32_t j1,
                                             ScanState st) {
    // row0 = (row, head) * max_tiles: tile j of head g at (row0 + j) * G + g
    int32_t tv[kMaxChunkTiles], tmx[kMaxChunkTiles], tsm[kMaxChunkTiles];
#pragma unroll
    for (int v = 0; v < (int)kMaxChunkTiles; v++) {
        if (j0 + v < j1) {
            const size_t base = (row0 + j0 + v) * G + g;
            tv[v] = ld_coherent(&s_tval[base * D + e]);
            tmx[v] = s_tmax[base];
            tsm[v] = ld_coherent(&s_tsum[base]);
        }
    }
#pragma unroll
    for (int v = 0; v < (int)kMaxChunkTiles; v++) {
        if (j0 + v < j1) {
            if (tmx[v] > st.m) {  // the running max moves: rescale
                const int64_t old = (int64_t)prob(e14, st.m - tmx[v]) << 2;
                st.sum = fx_sat32(fx_rnd((int64_t)st.sum * old + ((int64_t)tsm[v] << 18), 16));
                st.acc = fx_sat32(fx_rnd((int64_t)st.acc * old, 16));
                st.m = tmx[v];
            } else {  // factor exp(0) = 1.0: rnd(v * 2^16, 16) = v
                st.sum = fx_sat32((int64_t)st.sum + ((int64_t)tsm[v] << 2));
            }
            st.acc = fx_sat32((int64_t)st.acc + ((int64_t)tv[v] << 8));
        }
    }
    return st;
}

}  // namespace

// ---------------------------------------------------------------------
// Fused path: one workgroup per (row, KV head) walks every tile.
// 512 threads; wave w owns query heads w, w+8; in QK and softmax
// lanes are tile positions, in PV lanes are head elements.  The loads of
// tile i + 1 are in flight while tile i is computed.
// ---------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(NT) void attention_fused_kernel(AttnArgs a) {
    __shared__ Smem<D> sm;
    const uint32_t t = blockIdx.x, h = blockIdx.y;
    const uint32_t G = a.group;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = a.pos0 + t + 1, own = n - 1;
    const uint32_t ntiles = (n + TILE - 1) / TILE;
    const int64_t scale = (int64_t)a.qk_scale << 8;

    ProLoad pl{};
    TileLoad<D> ld;
    issue_prologue<D>(a, t, h, true, true, pl);
    TileGeo tg = tile_geo(a, n, 0);
    issue_k<D>(a, h, tg, ld);
    issue_v<D>(a, h, tg, ld);
    commit_prologue<D>(a, sm, true, true, pl);

    constexpr int GW = MAXG / NW;            // query heads per wave (max)
    constexpr int EW = (D + 63) / 64;        // element chunks per lane
    int32_t m[GW], sum[GW], acc[GW][EW];
#pragma unroll
    for (int i = 0; i < GW; i++) {
        m[i] = INT16_MIN;  // fm(-128)
        sum[i] = 0;
#pragma unroll
        for (int j = 0; j < EW; j++) acc[i][j] = 0;
    }

    for (uint32_t tile = 0; tile < ntiles; tile++) {
        const uint32_t any_k = commit_k<D>(sm, tg, ld, own);
        const uint32_t any_v = commit_v<D>(sm, tg, ld, own);
        publish_flags<D>(sm, any_k, any_v);
        const uint32_t tl = tg.tl;
        __syncthreads();  // tile staged
        const int32_t fl = read_flags<D>(sm);
        const bool kcorr = (fl & 1) != 0, vcorr = (fl & 2) != 0;
        if (tile + 1 < ntiles) {  // next tile's loads overlap this tile
            tg = tile_geo(a, n, tile + 1);
            issue_k<D>(a, h, tg, ld);
            issue_v<D>(a, h, tg, ld);
        }
        {
            v4u kr[D / 8];
            load_k_row<D>(sm, lane, kr);
#pragma unroll
            for (int gi = 0; gi < GW; gi++) {
                const uint32_t g = wave + NW * gi;
                if (g >= G) break;
                const bool valid = lane < tl;
                const int32_t s = valid ? row_score<D>(sm.q + g * D, sm.cq + g * D, kr,
                                                           kcorr, scale)
                                        : INT16_MIN;
                const int32_t wm = wave_max(s);
                const int32_t mn = wm > m[gi] ? wm : m[gi];
                const int32_t old = prob(sm.e14, m[gi] - mn);
                const int32_t pr = valid ? prob(sm.e14, s - mn) : 0;
                put_prob<D>(sm, g, lane, pr);
                const int32_t ts = wave_sum(pr);  // <= 64 * 16384
                sum[gi] = fx_sat32(fx_rnd((int64_t)sum[gi] * ((int64_t)old << 2) +
                                          ((int64_t)ts << 18), 16));
                m[gi] = mn;
                if (old != 16384) {
#pragma unroll
                    for (int ei = 0; ei < EW; ei++)
                        acc[gi][ei] = fx_sat32(fx_rnd((int64_t)acc[gi][ei] *
                                                      ((int64_t)old << 2), 16));
                }
            }
        }
        __syncthreads();  // probabilities staged
#pragma unroll
        for (int ei = 0; ei < EW; ei++) {
            const uint32_t e = lane + 64 * ei;
            if (e >= D) break;
            v4u vr[TILE / 8];
            load_v_row<D>(sm, e, vr);
#pragma unroll
            for (int gi = 0; gi < GW; gi++) {
                const uint32_t g = wave + NW * gi;
                if (g >= G) break;
                const int32_t tv = row_pv(sm.p + g * TILE, sm.cp + g * TILE, vr, vcorr);
                acc[gi][ei] = fx_sat32((int64_t)acc[gi][ei] + ((int64_t)tv << 8));
            }
        }
        __syncthreads();  // tile consumed
    }
    int16_t* dst = a.out + (size_t)t * a.ldo + (size_t)h * G * D;
#pragma unroll
    for (int gi = 0; gi < GW; gi++) {
        const uint32_t g = wave + NW * gi;
        if (g >= G) break;
        const int64_t inv = fx_inv_sum(sum[gi]);
#pragma unroll
        for (int ei = 0; ei < EW; ei++) {
            const uint32_t e = lane + 64 * ei;
            if (e >= D) break;
            dst[g * D + e] = fx_sat16(fx_rnd((int64_t)acc[gi][ei] * inv, 16));
        }
    }
    store_appended<D>(a, sm, h, own, true, true);
}

// ---------------------------------------------------------------------
// Head path: one wavefront per (row, query head) walks every tile, for the
// contexts of the fused path.  Every load of the first tile is issued at
// once: the cache rows go to registers (lane p holds the K row of position
// p, lanes e and e + 64 the V^T rows of those elements), the current
// block's rows are rotated into LDS, the exp table is staged, and the
// wavefront then computes without a workgroup barrier.  The serial chain
// of one head is short, and the grid covers every (row, head), so this is
// the latency path for decode and for 8-row blocks at short contexts.
// ---------------------------------------------------------------------
template <int D>
struct __attribute__((aligned(16))) HeadSmem {
    int16_t q[D], cq[D];        // rotated query, c(q), bank-paired
    int16_t kc[8][D];           // the block's K rows after RoPE, bank-paired
    int16_t vc[8][D];           // the block's V rows
    int16_t p[TILE], cp[TILE];  // a tile's probabilities and c(p), paired
    int16_t e14[2056];          // Q2.14 exp table
};

template <int D>
struct HeadRows {
    static constexpr int EW = (D + 63) / 64;  // elements per lane in PV
    v4u k[D / 8];
    v4u v[EW][TILE / 8];
};

// This lane's cache rows of `tile`: the K row of its position (cached
// positions only) and the V^T chunks that hold cached positions.
template <int D>
__device__ __forceinline__ void head_load(const AttnArgs& a, uint32_t h, uint32_t tile,
                                          HeadRows<D>& R) {
    const uint32_t lane = threadIdx.x, p = tile * TILE + lane;
    const int16_t* kp = a.kcache + page_off<D>(a, h, tile);
    const int16_t* vp = a.vcache + page_off<D>(a, h, tile);
#pragma unroll
    for (int c = 0; c < D / 8; c++)
        R.k[c] = p < a.pos0 ? *(const v4u*)(kp + (size_t)lane * D + 8 * c) : v4u{0, 0, 0, 0};
#pragma unroll
    for (int ei = 0; ei < HeadRows<D>::EW; ei++) {
        const uint32_t e = lane + 64 * ei;
#pragma unroll
        for (int c = 0; c < TILE / 8; c++)
            R.v[ei][c] = e < D && tile * TILE + 8 * c < a.pos0
                             ? *(const v4u*)(vp + (size_t)e * TILE + 8 * c)
                             : v4u{0, 0, 0, 0};
    }
}


template <int D>
__global__ __launch_bounds__(64) void attention_head_kernel(AttnArgs a) {
    __shared__ HeadSmem<D> sm;
    constexpr int EW = HeadRows<D>::EW;
    const uint32_t t = blockIdx.x, g = blockIdx.y, lane = threadIdx.x;
    const uint32_t h = g / a.group;
    const uint32_t n = a.pos0 + t + 1, own = n - 1;
    const uint32_t ntiles = (n + TILE - 1) / TILE;
    const int64_t scale = (int64_t)a.qk_scale << 8;

    // ---- every load of the first tile ----
    HeadRows<D> rows;
    head_load<D>(a, h, 0, rows);
    v4u ex[5];
#pragma unroll
    for (int u = 0; u < 5; u++) {
        const uint32_t c = lane + 64 * u < 257 ? lane + 64 * u : 256;
        ex[u] = *(const v4u*)(a.exp14 + 8 * c);
    }
    const uint32_t c = lane < D / 2 ? lane : 0;  // RoPE pair (c, c + D/2)
    const int16_t* qrow = a.qkv + (size_t)t * a.ldqkv + (size_t)g * D;
    const int16_t* qrope = a.rope + (size_t)own * D;
    const int32_t qx0 = qrow[c], qx1 = qrow[D / 2 + c], qc = qrope[c], qs = qrope[D / 2 + c];
    int32_t kx0[8], kx1[8], kc[8], ks[8], vv[8][EW];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        if (r <= (int)t) {
            const int16_t* row = a.qkv + (size_t)r * a.ldqkv;
            const int16_t* krow = row + (size_t)a.num_heads * D + (size_t)h * D;
            const int16_t* vrow = row + (size_t)(a.num_heads + a.num_kv_heads) * D + (size_t)h * D;
            const int16_t* kr = a.rope + (size_t)(a.pos0 + r) * D;
            kx0[r] = krow[c];
            kx1[r] = krow[D / 2 + c];
            kc[r] = kr[c];
            ks[r] = kr[D / 2 + c];
#pragma unroll
            for (int ei = 0; ei < EW; ei++) {
                const uint32_t e = lane + 64 * ei;
                vv[r][ei] = e < D ? vrow[e] : 0;
            }
        }
    }
    // ---- staging (one wavefront: LDS operations stay in order) ----
#pragma unroll
    for (int u = 0; u < 5; u++) {
        const uint32_t cc = lane + 64 * u < 257 ? lane + 64 * u : 256;
        *(v4u*)(sm.e14 + 8 * cc) = ex[u];
    }
    if (lane < D / 2) {
        int32_t y0, y1;
        rope_pair(qx0, qx1, qc, qs, y0, y1);
        sm.q[paired(c)] = (int16_t)y0;
        sm.q[paired(D / 2 + c)] = (int16_t)y1;
        sm.cq[paired(c)] = (int16_t)sat_corr(y0);
        sm.cq[paired(D / 2 + c)] = (int16_t)sat_corr(y1);
    }
#pragma unroll
    for (int r = 0; r < 8; r++) {
        if (r <= (int)t) {
            if (lane < D / 2) {
                int32_t y0, y1;
                rope_pair(kx0[r], kx1[r], kc[r], ks[r], y0, y1);
                sm.kc[r][paired(c)] = (int16_t)y0;
                sm.kc[r][paired(D / 2 + c)] = (int16_t)y1;
            }
#pragma unroll
            for (int ei = 0; ei < EW; ei++) {
                const uint32_t e = lane + 64 * ei;
                if (e < D) sm.vc[r][e] = (int16_t)vv[r][ei];
            }
        }
    }

    int32_t m = INT16_MIN, sum = 0, acc[EW];
#pragma unroll
    for (int ei = 0; ei < EW; ei++) acc[ei] = 0;
    for (uint32_t tile = 0; tile < ntiles; tile++) {
        if (tile > 0) head_load<D>(a, h, tile, rows);
        const uint32_t p = tile * TILE + lane;
        const bool valid = p < n;
        // K row of this lane's position: cached, or a row of this block
        const bool blk = p >= a.pos0 && p <= own;
        const int16_t* kb = sm.kc[blk ? p - a.pos0 : 0];
        v4u kr[D / 8];
        uint32_t mk = 0;
#pragma unroll
        for (int cc = 0; cc < D / 8; cc++)
            kr[cc] = clamp4(blk ? *(const v4u*)(kb + 8 * cc) : rows.k[cc], mk);
        const bool kcorr = __any(mk != 0);
        // q and c(q) are read inside the loop (hoisted, they would hold
        // 2 D/8 vector registers across it)
        uint32_t qoff = 0;
        asm volatile("" : "+v"(qoff));
        const int32_t s = valid ? row_score<D>(sm.q + qoff, sm.cq + qoff, kr, kcorr, scale)
                                : INT16_MIN;
        const int32_t wm = wave_max(s);
        const int32_t mn = wm > m ? wm : m;
        const int32_t old = prob(sm.e14, m - mn);
        const int32_t pr = valid ? prob(sm.e14, s - mn) : 0;
        sm.p[paired(lane)] = (int16_t)pr;
        sm.cp[paired(lane)] = (int16_t)sat_corr(pr);
        const int32_t ts = wave_sum(pr);  // <= 64 * 16384
        sum = fx_sat32(fx_rnd((int64_t)sum * ((int64_t)old << 2) + ((int64_t)ts << 18), 16));
        m = mn;
        if (old != 16384) {
#pragma unroll
            for (int ei = 0; ei < EW; ei++)
                acc[ei] = fx_sat32(fx_rnd((int64_t)acc[ei] * ((int64_t)old << 2), 16));
        }
        // V^T rows: the block's rows in this tile go to their own slots
        // (slots beyond the context meet probability 0)
        for (uint32_t r = 0; r <= t; r++) {
            const uint32_t pp = a.pos0 + r;
            if (pp / TILE != tile) continue;
            const uint32_t slot = paired(pp % TILE);
#pragma unroll
            for (int ei = 0; ei < EW; ei++) {
                const uint32_t e = lane + 64 * ei < D ? lane + 64 * ei : 0;
#pragma unroll
                for (int cc = 0; cc < TILE / 8; cc++)
                    if (slot / 8 == (uint32_t)cc)
                        rows.v[ei][cc] = put_half(rows.v[ei][cc], slot % 8, sm.vc[r][e]);
            }
        }
        v4u vr[EW][TILE / 8];
        uint32_t mv = 0;
#pragma unroll
        for (int ei = 0; ei < EW; ei++)
#pragma unroll
            for (int cc = 0; cc < TILE / 8; cc++) vr[ei][cc] = clamp4(rows.v[ei][cc], mv);
        const bool vcorr = __any(mv != 0);
#pragma unroll
        for (int ei = 0; ei < EW; ei++) {
            if (lane + 64 * ei >= D) break;
            const int32_t tv = row_pv(sm.p, sm.cp, vr[ei], vcorr);
            acc[ei] = fx_sat32((int64_t)acc[ei] + ((int64_t)tv << 8));
        }
    }
    const int64_t inv = fx_inv_sum(sum);
#pragma unroll
    for (int ei = 0; ei < EW; ei++) {
        const uint32_t e = lane + 64 * ei;
        if (e < D)
            a.out[(size_t)t * a.ldo + (size_t)g * D + e] =
                fx_sat16(fx_rnd((int64_t)acc[ei] * inv, 16));
    }
    if (g % a.group == 0) {  // this row's K (rotated, paired) and V into the cache
        const uint32_t tile = own / TILE, slot = own % TILE;
        if (lane < D / 8)
            *(v4u*)(a.kcache + page_off<D>(a, h, tile) + slot * D + 8 * lane) =
                *(const v4u*)(sm.kc[t] + 8 * lane);
#pragma unroll
        for (int ei = 0; ei < EW; ei++) {
            const uint32_t e = lane + 64 * ei;
            if (e < D) a.vcache[page_off<D>(a, h, tile) + e * TILE + paired(slot)] = sm.vc[t][e];
        }
    }
}


template <int D>
__global__ __launch_bounds__(D * 2) void attention_split_head_kernel(AttnArgs a) {
    __shared__ SplitSmem<D> sm;
    split_head_body<D, false>(a, blockIdx.x, blockIdx.y, sm, [] { return true; });
}

// ---------------------------------------------------------------------
// Fused attention sublayer (decode rows, split-head attention): QKV
// blocks, then attention workgroups, then O blocks, in one launch (see
// SublayerArgs).  Hand-offs: the QKV and attention outputs are written
// with device-coherent stores, each producing workgroup then arrives on a
// counter, and the consumers poll (bounded) after issuing every load that
// does not depend on them.  Arrivals are spread over counter lines so
// that no line takes more than a few tens of atomics per launch (one
// line for all 640 QKV blocks measured several microseconds of
// serialised atomics).
// ---------------------------------------------------------------------
#ifndef LLM_SUB_P12
#define LLM_SUB_P12 1  // fused sublayer: 12-bit copies where both matrices have one
#endif
#ifndef LLM_SUB_QKV_NB
#define LLM_SUB_QKV_NB 1
#endif
// QKV blocks per workgroup of the fused attention sublayer
constexpr uint32_t kSubQkvBlocks = LLM_SUB_QKV_NB;

// O blocks per workgroup of the fused attention sublayer (half the waiting
// workgroups of one block each, at the same measured time)
constexpr uint32_t kSubOBlocks = 2;

// P12: both projections read their 12-bit copies (qkv.p0, o.p0); CORR:
// with their corrections.
template <int D, int RT, int QEPI, int LW, bool P12 = false, bool CORR = false>
__global__ __launch_bounds__(D * 2) void attention_sublayer_kernel(SublayerArgs s) {
    constexpr int WPB = D / 32, SPW = 4;
    constexpr uint32_t NBR = kSubQkvBlocks > kSubOBlocks ? kSubQkvBlocks : kSubOBlocks;
    __shared__ SplitSmem<D> sm;
    __shared__ int64_t red[NBR * WPB * 4 * RT];
    __shared__ uint32_t flag;
    uint32_t* const sync = s.sync;
    const uint32_t idx = blockIdx.x;
    if (idx < s.nq) {
        proj_block<RT, QEPI, WPB, SPW, false, true, LW, kSubQkvBlocks, P12, CORR>(
            s.qkv, idx, red, [] { return true; });
        arrive(sync + kSyncStride * (idx % kSyncQkvLines));
        return;
    }
    if (idx < s.nq + s.na) {
        const uint32_t k = idx - s.nq;
        const uint32_t t = k / s.at.num_heads, g = k % s.at.num_heads;
        if (!split_head_body<D, true>(s.at, t, g, sm, [&] {
                const uint32_t per = s.nq / kSyncQkvLines, extra = s.nq % kSyncQkvLines;
                return wait_counts(
                    sync, kSyncStride, kSyncQkvLines,
                    [&](uint32_t l) { return s.qkv_base[l] + per + (l < extra ? 1u : 0u); },
                    s.wait_limit, sync + kSyncAbort, s.host_abort, &flag);
            }))
            return;
        arrive(sync + kSyncAttn, kSyncAttnLines, kSyncStride);
        return;
    }
    const uint32_t b = idx - s.nq - s.na;
    proj_block<RT, EPI_RESID, WPB, SPW, true, false, LW, kSubOBlocks, P12, CORR>(s.o, b, red, [&] {
        return wait_counts(
            sync + kSyncAttn + kSyncStride * (b % kSyncAttnLines), 0, 1,
            [&](uint32_t) { return s.attn_base + s.na; }, s.wait_limit, sync + kSyncAbort, s.host_abort, &flag);
    });
}

// ---------------------------------------------------------------------
// Split path, phase A: scores and tile maxima for a chunk of tiles; the
// row's own K is appended by the chunk that holds its position.
// grid (rows, kv_heads, chunks).
// ---------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(NT) void attention_scores_kernel(AttnArgs a) {
    __shared__ Smem<D> sm;
    const uint32_t t = blockIdx.x, h = blockIdx.y, c = blockIdx.z;
    const uint32_t G = a.group;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = a.pos0 + t + 1, own = n - 1;
    const uint32_t ntiles = (n + TILE - 1) / TILE;
    const uint32_t t0 = c * a.chunk_tiles;
    if (t0 >= ntiles) return;
    const uint32_t t1 = t0 + a.chunk_tiles < ntiles ? t0 + a.chunk_tiles : ntiles;
    const int64_t scale = (int64_t)a.qk_scale << 8;
    const size_t rh = (size_t)t * a.num_kv_heads + h;

    ProLoad pl{};
    TileLoad<D> ld;
    issue_prologue<D>(a, t, h, true, false, pl);
    TileGeo tg = tile_geo(a, n, t0);
    issue_k<D>(a, h, tg, ld);
    commit_prologue<D>(a, sm, true, false, pl);
    for (uint32_t tile = t0; tile < t1; tile++) {
        publish_flags<D>(sm, commit_k<D>(sm, tg, ld, own), 0);
        const uint32_t tl = tg.tl;
        __syncthreads();  // tile staged
        const bool kcorr = (read_flags<D>(sm) & 1) != 0;
        if (tile + 1 < t1) {
            tg = tile_geo(a, n, tile + 1);
            issue_k<D>(a, h, tg, ld);
        }
        v4u kr[D / 8];
        load_k_row<D>(sm, lane, kr);
        for (uint32_t g = wave; g < G; g += NW) {
            const bool valid = lane < tl;
            const int32_t s = valid ? row_score<D>(sm.q + g * D, sm.cq + g * D, kr, kcorr, scale)
                                    : INT16_MIN;
            const size_t base = (rh * a.max_tiles + tile) * G + g;
            a.s_scores[base * TILE + lane] = (int16_t)s;
            const int32_t mx = wave_max(s);
            if (lane == 0) a.s_tmax[base] = (int16_t)mx;
        }
        __syncthreads();  // tile consumed
    }
    if (own / TILE >= t0 && own / TILE < t1) store_appended<D>(a, sm, h, own, true, false);
}

// ---------------------------------------------------------------------
// Split path, phase B: probabilities, tile sums and PV values for a chunk
// given the prefix max; the last chunk of a (row, KV head) to finish runs
// the sequential rounding scan and writes the output.
// ---------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(NT) void attention_pv_kernel(AttnArgs a) {
    __shared__ Smem<D> sm;
    __shared__ int32_t mrun[MAXG];
    __shared__ int32_t cflag[MAXG], ctsum[MAXG];
    const uint32_t t = blockIdx.x, h = blockIdx.y, c = blockIdx.z;
    const uint32_t G = a.group;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = a.pos0 + t + 1, own = n - 1;
    const uint32_t ntiles = (n + TILE - 1) / TILE;
    const uint32_t nchunks = (ntiles + a.chunk_tiles - 1) / a.chunk_tiles;
    const uint32_t t0 = c * a.chunk_tiles;
    if (t0 >= ntiles) return;
    const uint32_t t1 = t0 + a.chunk_tiles < ntiles ? t0 + a.chunk_tiles : ntiles;
    const size_t rh = (size_t)t * a.num_kv_heads + h;

    ProLoad pl{};
    TileLoad<D> ld;
    issue_prologue<D>(a, t, h, false, true, pl);
    TileGeo tg = tile_geo(a, n, t0);
    issue_v<D>(a, h, tg, ld);
    commit_prologue<D>(a, sm, false, true, pl);
    if (threadIdx.x < G) {
        mrun[threadIdx.x] = INT16_MIN;
        cflag[threadIdx.x] = 0;
        ctsum[threadIdx.x] = 0;
    }
    constexpr int IT = MAXG * D / NT > 0 ? MAXG * D / NT : 1;  // (g, e) items per thread
    int32_t csum[IT];
#pragma unroll
    for (int u = 0; u < IT; u++) csum[u] = 0;
    __syncthreads();
    // running max before this chunk: parallel over (tile, head)
    for (uint32_t idx = threadIdx.x; idx < t0 * G; idx += blockDim.x)
        __hip_atomic_fetch_max(&mrun[idx % G],
                               (int32_t)a.s_tmax[(rh * a.max_tiles + idx / G) * G + idx % G],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    for (uint32_t tile = t0; tile < t1; tile++) {
        const uint32_t tl = tg.tl;
        int32_t sc[MAXG / NW], tm[MAXG / NW];
#pragma unroll
        for (int gi = 0; gi < MAXG / NW; gi++) {
            const uint32_t g = wave + NW * gi;
            sc[gi] = tm[gi] = 0;
            if (g < G) {
                const size_t base = (rh * a.max_tiles + tile) * G + g;
                sc[gi] = a.s_scores[base * TILE + lane];
                tm[gi] = a.s_tmax[base];
            }
        }
        publish_flags<D>(sm, 0, commit_v<D>(sm, tg, ld, own));
        __syncthreads();  // mrun complete; V staged
        const bool vcorr = (read_flags<D>(sm) & 2) != 0;
        if (tile + 1 < t1) {
            tg = tile_geo(a, n, tile + 1);
            issue_v<D>(a, h, tg, ld);
        }
#pragma unroll
        for (int gi = 0; gi < MAXG / NW; gi++) {
            const uint32_t g = wave + NW * gi;
            if (g < G) {
                const int32_t mn = tm[gi] > mrun[g] ? tm[gi] : mrun[g];
                const int32_t pr = lane < tl ? prob(sm.e14, sc[gi] - mn) : 0;
                put_prob<D>(sm, g, lane, pr);
                const int32_t ts = wave_sum(pr);
                if (lane == 0) {
                    st_coherent(&a.s_tsum[(rh * a.max_tiles + tile) * G + g], ts);
                    ctsum[g] += ts << 2;               // this wave owns head g
                    if (tm[gi] > mrun[g]) cflag[g] = 1;  // the running max rises
                }
            }
        }
        __syncthreads();  // probabilities staged
#pragma unroll
        for (int u = 0; u < IT; u++) {
            const uint32_t idx = threadIdx.x + NT * u;
            if (idx >= G * D) break;
            const uint32_t g = idx / D, e = idx % D;
            v4u vr[TILE / 8];
            load_v_row<D>(sm, e, vr);
            const size_t base = (rh * a.max_tiles + tile) * G + g;
            const int32_t tv = row_pv(sm.p + g * TILE, sm.cp + g * TILE, vr, vcorr);
            st_coherent(&a.s_tval[base * D + e], (int16_t)tv);
            csum[u] += tv << 8;
        }
        __syncthreads();  // tile consumed
        if (threadIdx.x < G) {
            const int32_t v = a.s_tmax[(rh * a.max_tiles + tile) * G + threadIdx.x];
            mrun[threadIdx.x] = v > mrun[threadIdx.x] ? v : mrun[threadIdx.x];
        }
    }
    if (own / TILE >= t0 && own / TILE < t1) store_appended<D>(a, sm, h, own, false, true);
    // The chunk's summary per query head (and element).
    const size_t rc = rh * a.max_chunks + c;
#pragma unroll
    for (int u = 0; u < IT; u++) {
        const uint32_t idx = threadIdx.x + NT * u;
        if (idx < G * D) st_coherent(&a.c_sum[rc * G * D + idx], csum[u]);
    }
    if (threadIdx.x < G) {
        st_coherent(&a.c_flag[rc * G + threadIdx.x], cflag[threadIdx.x]);
        st_coherent(&a.c_tsum[rc * G + threadIdx.x], ctsum[threadIdx.x]);
    }
    // Publish, then let the last chunk of this (row, head) finish.
    if (!arrive_last(&a.counters[rh], nchunks, &sm.last)) return;
    // The per-tile recurrence (sum, acc rounded at every tile).  A chunk in
    // which the running max does not rise only adds: its factors are
    // exp(0) = 1.0, so rnd(v * 2^16, 16) = v, and while |acc| and sum stay
    // clear of the int32 bounds by the chunk's largest possible movement
    // (tile values << 8 < 2^23, tile sums << 2 <= 2^22) no saturation can
    // occur inside it; such a chunk is applied as one addition.  Other
    // chunks run tile by tile.
    constexpr int SB = 16;  // chunks whose summaries are in flight together
    const uint32_t CT = a.chunk_tiles;
    for (uint32_t idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
        const uint32_t g = idx / D, e = idx % D;
        ScanState st{INT16_MIN, 0, 0};
        for (uint32_t c0 = 0; c0 < nchunks; c0 += SB) {
            int32_t fl[SB], cs[SB], ct[SB];
#pragma unroll
            for (int u = 0; u < SB; u++) {
                fl[u] = 1, cs[u] = 0, ct[u] = 0;
                if (c0 + u < nchunks) {
                    const size_t q = rh * a.max_chunks + c0 + u;
                    fl[u] = ld_coherent(&a.c_flag[q * G + g]);
                    cs[u] = ld_coherent(&a.c_sum[q * G * D + idx]);
                    ct[u] = ld_coherent(&a.c_tsum[q * G + g]);
                }
            }
#pragma unroll
            for (int u = 0; u < SB; u++) {
                const uint32_t cc = c0 + u;
                if (cc < nchunks) {
                    const uint32_t j0 = cc * CT, j1 = j0 + CT < ntiles ? j0 + CT : ntiles;
                    const int64_t nt = j1 - j0;
                    const int64_t aa = st.acc < 0 ? -(int64_t)st.acc : st.acc;
                    if (!fl[u] && aa <= INT32_MAX - (nt << 23) &&
                        st.sum <= INT32_MAX - (nt << 22)) {
                        st.acc += cs[u];
                        st.sum += ct[u];
                    } else {
                        st = scan_tiles<D>(a.s_tval, a.s_tmax, a.s_tsum, sm.e14,
                                           rh * a.max_tiles, G, g, e, j0, j1, st);
                    }
                }
            }
        }
        const int32_t sum = st.sum, acc = st.acc;
        const int64_t inv = fx_inv_sum(sum);
        a.out[(size_t)t * a.ldo + (size_t)h * G * D + idx] =
            fx_sat16(fx_rnd((int64_t)acc * inv, 16));
    }
}

// ---------------------------------------------------------------------
// Tile path (long contexts, head_dim a multiple of 32): one workgroup of
// D / 32 wavefronts per (row, query head, tile), in two launches.
//   (1) attention_tile_scores_kernel: the tile's scores (split-head QK)
//       and their maximum; the K row of each row's own position is
//       appended by the workgroup that holds it.
//   (2) attention_tile_pv_kernel: the running max before and after the
//       tile (a prefix max of the tile maxima), the tile's probabilities,
//       their sum and the rounded PV value of every element (split-head
//       PV); the V append; the last workgroup of a (row, query head) to
//       arrive runs the per-tile rounding recurrence over all tiles, 64
//       tiles of operands staged in LDS at a time.
// Scratch indices as in the chunked path: (row, KV head, tile, head in
// group).
// ---------------------------------------------------------------------
template <int D>
struct __attribute__((aligned(16))) TileScoresSmem {
    static constexpr int NWH = D / 32;
    int16_t q[D], cq[D];                  // rotated query, c(q)
    int16_t kv[8][D];                     // the block's K rows after RoPE
    v4u part[NWH][TILE];                  // QK bank partials (int32)
    int16_t scr[NWH][SLICE_SCRATCH];      // per wavefront: slice transposes
};
template <int D>
struct __attribute__((aligned(16))) TilePvSmem {
    static constexpr int NWH = D / 32;
    static constexpr int NTH = 2 * D;
    int16_t kv[8][D];                     // the block's V rows
    int16_t p[NWH][TILE], cp[NWH][TILE];  // per wavefront: probabilities, c(p)
    int16_t e14[2056];                    // Q2.14 exp table
    uint32_t last;
    int32_t m0;                           // one-launch path: running max before the tile
    int32_t rinv;                         // 1 / the recurrence's final sum
    int32_t fac[NTH / 64][64];            // per wavefront: a piece's rescale factors
    union __attribute__((aligned(16))) {
        int16_t scr[NWH][SLICE_SCRATCH];  // per wavefront: slice transposes
        struct {                          // then the recurrence operands of up
            int16_t tv[64][D];            // to 64 tiles: PV values
            int32_t tmax[64], tsum[64];   // [tile][element], maxima, sums
        };
    };
};

// Block rows [r0, r1] of a row's block that fall in `tile` (nrow = 0 when
// none does); r0 is a row of the block in any case.
struct TileRows {
    uint32_t r0, nrow;
};
__device__ __forceinline__ TileRows tile_rows(const AttnArgs& a, uint32_t tile, uint32_t own) {
    TileRows r;
    const uint32_t lo = tile * TILE, hi = tile * TILE + TILE - 1;
    r.r0 = lo > a.pos0 ? lo - a.pos0 : 0;
    r.nrow = hi >= a.pos0 ? (own < hi ? own : hi) - a.pos0 + 1 - r.r0 : 0;
    return r;
}

// Workgroup -> (row, query head, tile) of the tile path.  Workgroups go to
// the 8 XCDs round robin by linear index; the query heads of one (row, KV
// head, tile), which read the same K / V page, are placed on one XCD one
// after another, so that all but the first find the page in that XCD's L2
// (heads placed on 8 XCDs read each page 8 times from memory).  The grid
// is padded to whole groups of 8 (row, KV head, tile) triples.
struct TileWg {
    uint32_t t, g, tile;
    bool valid;
};
__device__ __forceinline__ TileWg tile_wg(const AttnArgs& a) {
    const uint32_t L = blockIdx.x, x = L % 8, seq = L / 8, G = a.group;
    const uint32_t triple = (seq / G) * 8 + x;  // ((row, tile), KV head)
    const uint32_t h = triple % a.num_kv_heads, rt = triple / a.num_kv_heads;
    TileWg w;
    w.t = rt / a.grid_tiles;
    w.tile = rt % a.grid_tiles;
    w.g = h * G + seq % G;
    w.valid = w.t < a.grid_rows;
    return w;
}
__host__ __device__ inline uint32_t tile_grid(uint32_t rows, uint32_t tiles, uint32_t kv_heads,
                                              uint32_t group) {
    return 8 * group * ((rows * tiles * kv_heads + 7) / 8);
}

// One-launch tile path: a (row, query head) has at most 64 tiles (one
// polling lane per tile).  Its tile maxima and tile sums carry a flag bit
// in the same word (zero between launches: the workgroup that combines the
// tiles clears them).
constexpr uint32_t kTileFusedMaxTiles = 64;
constexpr uint32_t kMaxValid = 0x10000u;     // s_tmax32: flag | (uint16) maximum
constexpr uint32_t kSumValid = 0x80000000u;  // s_tsum: flag | tile sum (< 2^21)

// Phase 1 of the tile path for a workgroup inside the row's context: the
// tile's scores and their maximum; FUSED keeps the scores in LDS (lsc, lmt)
// and publishes the flagged maximum with a device-coherent store.
template <int D, bool FUSED>
__device__ __forceinline__ void tile_scores_phase(const AttnArgs& a, const TileWg& wg,
                                                  TileScoresSmem<D>& sm, int16_t* lsc,
                                                  int32_t* lmt) {
    static_assert(D % 32 == 0, "tile path: head_dim a multiple of 32");
    constexpr uint32_t NTH = D * 2;
    constexpr int NK = (8 * (D / 2) + NTH - 1) / NTH;  // block K items per thread
    const uint32_t t = wg.t, g = wg.g, tile = wg.tile, tid = threadIdx.x;
    const uint32_t n = a.pos0 + t + 1, own = n - 1;
    const uint32_t lane = tid & 63, w = tid >> 6;
    const uint32_t G = a.group, h = g / G, gi = g % G;
    const int64_t scale = (int64_t)a.qk_scale << 8;

    // ---- staging loads (indices clamped: every load is issued), this
    // tile's slices, then the staging writes ----
    const uint32_t qc = tid < D / 2 ? tid : 0;
    const int16_t* qrow = a.qkv + (size_t)t * a.ldqkv + (size_t)g * D;
    const int16_t* qrope = a.rope + (size_t)own * D;
    const int32_t qx0 = qrow[qc], qx1 = qrow[D / 2 + qc], qcs = qrope[qc], qsn = qrope[D / 2 + qc];
    const TileRows tr = tile_rows(a, tile, own);
    const uint32_t nk = tr.nrow * (D / 2);
    int32_t kx[NK][4];
#pragma unroll
    for (int u = 0; u < NK; u++) {
        const uint32_t i = tid + NTH * u < nk ? tid + NTH * u : 0;
        const uint32_t r = tr.r0 + i / (D / 2), c = i % (D / 2);
        const int16_t* krow = a.qkv + (size_t)r * a.ldqkv + (size_t)a.num_heads * D +
                              (size_t)h * D;
        const int16_t* kr = a.rope + (size_t)(a.pos0 + r) * D;
        kx[u][0] = krow[c];
        kx[u][1] = krow[D / 2 + c];
        kx[u][2] = kr[c];
        kx[u][3] = kr[D / 2 + c];
    }
    SplitRegs regs;
    slice_load<D>(a, h, tile, w, lane, regs);
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
            const uint32_t r = tr.r0 + i / (D / 2), c = i % (D / 2);
            int32_t y0, y1;
            rope_pair(kx[u][0], kx[u][1], kx[u][2], kx[u][3], y0, y1);
            sm.kv[r][paired(c)] = (int16_t)y0;
            sm.kv[r][paired(D / 2 + c)] = (int16_t)y1;
        }
    }
    lds_barrier();
    const uint32_t p = tile * TILE + lane;
    const bool valid = p < n;
    const bool blk = p >= a.pos0 && p <= own;
    const bool cached = p < a.pos0;
    const int16_t* kb = sm.kv[blk ? p - a.pos0 : 0] + 32 * w;
    v4u kr[4];
    slice_k_rows(sm.scr[w], regs, lane, kr);
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
    sm.part[w][lane] = v4u{(uint32_t)b0, (uint32_t)b1, (uint32_t)b2, (uint32_t)b3};
    lds_barrier();
    if (w == 0) {
        uint32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;  // bank sums mod 2^32
#pragma unroll
        for (int ww = 0; ww < TileScoresSmem<D>::NWH; ww++) {
            const v4u pv = sm.part[ww][lane];
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
        int32_t ts = fx_sat32(t64);
        ts = rnd16_mul(ts, (int32_t)scale);  // scale = qk_scale << 8 <= 2^16
        const int32_t s = valid ? sat16_32(rnd32(ts, 8)) : INT16_MIN;
        const size_t base = (((size_t)t * a.num_kv_heads + h) * a.max_tiles + tile) * G + gi;
        const int32_t mx = wave_max(s);
        if (FUSED) {
            lsc[lane] = (int16_t)s;
            if (lane == 0) {
                *lmt = mx;
                st_coherent(&a.s_tmax32[base], (int32_t)(kMaxValid | (uint16_t)mx));
            }
        } else {
            a.s_scores[base * TILE + lane] = (int16_t)s;
            if (lane == 0) a.s_tmax[base] = (int16_t)mx;
        }
    }
    if (gi == 0 && own / TILE == tile && tid < D / 8)  // this row's K into the cache
        *(v4u*)(a.kcache + page_off<D>(a, h, tile) + (own % TILE) * D + 8 * tid) =
            *(const v4u*)(sm.kv[t] + 8 * tid);
}

template <int D>
__global__ __launch_bounds__(D * 2) void attention_tile_scores_kernel(AttnArgs a) {
    __shared__ TileScoresSmem<D> sm;
    const TileWg wg = tile_wg(a);
    if (!wg.valid) return;                             // padding
    if (wg.tile * TILE >= a.pos0 + wg.t + 1) return;   // beyond this row's context
    tile_scores_phase<D, false>(a, wg, sm, nullptr, nullptr);
}

// The wavefront's V^T slice of `tile` alone (see slice_load).
template <int D>
__device__ __forceinline__ void slice_load_v(const AttnArgs& a, uint32_t h, uint32_t tile,
                                             uint32_t w, uint32_t lane, SplitRegs& R) {
    const uint32_t tp = tile < a.tiles ? tile : a.tiles - 1;
    const int16_t* vp = a.vcache + page_off<D>(a, h, tp) + (size_t)32 * w * TILE + 8 * lane;
#pragma unroll
    for (int c = 0; c < 4; c++) R.v[c] = *(const v4u*)(vp + 512 * c);
}

// Phase 2 of the tile path for a workgroup inside the row's context: the
// tile's probabilities under the running max, their sum, its PV values,
// and the recurrence over the tiles of the (row, query head).  Non-FUSED:
// the scores and maxima come from the scores launch, the last tile to
// arrive runs the recurrence.  FUSED: this workgroup's scores are lsc /
// lmt; after its own loads are issued it polls the flagged maxima of the
// earlier tiles, publishes its PV values and then its flagged tile sum,
// and the workgroup of the last tile polls the other tiles' sums and runs
// the recurrence.
// OARR (FUSED only): the output row slice is stored device-coherently and
// the combining workgroup then arrives on a.attn_arrive (kSyncAttnLines
// counters), for O blocks of the same launch.
template <int D, bool FUSED, bool OARR = false>
__device__ __forceinline__ void tile_pv_phase(const AttnArgs& a, const TileWg& wg,
                                              TilePvSmem<D>& sm, const int16_t* lsc,
                                              const int32_t* lmt) {
    static_assert(!OARR || FUSED, "the O hand-off follows the one-launch combine");
    static_assert(D % 32 == 0, "tile path: head_dim a multiple of 32");
    constexpr uint32_t NTH = D * 2;
    constexpr int NM = 4;                        // tile maxima per lane (tiles < 256)
    const uint32_t t = wg.t, g = wg.g, tile = wg.tile, tid = threadIdx.x;
    const uint32_t n = a.pos0 + t + 1, own = n - 1;
    const uint32_t ntiles = (n + TILE - 1) / TILE;
    const uint32_t lane = tid & 63, w = tid >> 6;
    const uint32_t G = a.group, h = g / G, gi = g % G;
    const size_t rh = (size_t)t * a.num_kv_heads + h;
    const size_t base = (rh * a.max_tiles + tile) * G + gi;

    // ---- staging loads (indices clamped: every load is issued), this
    // tile's V slice, then the staging writes.  One launch with more than
    // one wavefront: the wavefronts past the first load and stage the exp
    // table and the block's V rows while the first polls the maxima ----
    constexpr bool SPLIT = FUSED && NTH > 64;
    constexpr uint32_t SW = SPLIT ? NTH - 64 : NTH;  // staging threads
    constexpr int NE2 = (257 + SW - 1) / SW, NV2 = (8 * D + SW - 1) / SW;
    const uint32_t sid = SPLIT ? tid - 64 : tid;     // index among them
    const bool stager = !SPLIT || tid >= 64;
    const TileRows tr = tile_rows(a, tile, own);
    const uint32_t nv = tr.nrow * D;
    v4u ex[NE2];
    int16_t vx[NV2];
    auto stage_load = [&] {
#pragma unroll
        for (int u = 0; u < NE2; u++) {
            const uint32_t c = sid + SW * u;
            ex[u] = *(const v4u*)(a.exp14 + 8 * (c < 257 ? c : 256));
        }
#pragma unroll
        for (int u = 0; u < NV2; u++) {
            const uint32_t i = sid + SW * u < nv ? sid + SW * u : 0;
            vx[u] = a.qkv[(size_t)(tr.r0 + i / D) * a.ldqkv +
                          (size_t)(a.num_heads + a.num_kv_heads) * D + (size_t)h * D + i % D];
        }
    };
    auto stage_write = [&] {
#pragma unroll
        for (int u = 0; u < NE2; u++) {
            const uint32_t c = sid + SW * u;
            if (c < 257) *(v4u*)(sm.e14 + 8 * c) = ex[u];
        }
#pragma unroll
        for (int u = 0; u < NV2; u++) {
            const uint32_t i = sid + SW * u;
            if (i < nv) sm.kv[tr.r0 + i / D][i % D] = vx[u];
        }
    };
    if (stager) stage_load();
    int32_t sc = 0, mt = 0, mprev = INT16_MIN;  // mprev: maxima of the earlier tiles
    if (!FUSED) {
        sc = a.s_scores[base * TILE + lane];
        mt = a.s_tmax[base];
#pragma unroll
        for (int u = 0; u < NM; u++) {  // this lane's share
            const uint32_t j = lane + 64 * u;
            const int32_t v = a.s_tmax[(rh * a.max_tiles + (j < tile ? j : 0)) * G + gi];
            mprev = j < tile && v > mprev ? v : mprev;
        }
        for (uint32_t j = lane + 64 * NM; j < tile; j += 64) {  // contexts beyond 256 tiles
            const int32_t v = a.s_tmax[(rh * a.max_tiles + j) * G + gi];
            mprev = v > mprev ? v : mprev;
        }
    }
    SplitRegs regs;
    slice_load_v<D>(a, h, tile, w, lane, regs);
    if (SPLIT && stager) stage_write();  // before the poll's barrier
    if (FUSED) {
        // lane j < tile of wavefront 0 polls tile j's maximum
        // (tile < kTileFusedMaxTiles); their maximum goes through LDS
        // before the poll's barrier
        uint32_t v = 0;
        if (!poll_flags((const uint32_t*)&a.s_tmax32[rh * a.max_tiles * G + gi], G, tile,
                        kMaxValid, &v, a.wait_limit, a.abort, a.host_abort, &sm.last,
                        [&](uint32_t vl) {
                            const int32_t mx = wave_max(
                                lane < tile ? (int32_t)(int16_t)(vl & 0xffffu) : INT16_MIN);
                            if (lane == 0) sm.m0 = mx;
                        }))
            return;
        sc = lsc[lane];
        mt = *lmt;
    }
    if (!SPLIT) {
        stage_write();
        lds_barrier();
    }
    // ---- probabilities under the running max after this tile ----
    const int32_t m0 = FUSED ? sm.m0 : wave_max(mprev);  // running max before the tile
    const int32_t mn = mt > m0 ? mt : m0;      // and after it
    const bool valid = tile * TILE + lane < n;
    const int32_t pr = valid ? prob(sm.e14, sc - mn) : 0;
    sm.p[w][paired(lane)] = (int16_t)pr;
    sm.cp[w][paired(lane)] = (int16_t)sat_corr(pr);
    const int32_t tsum = wave_sum(pr);  // <= 64 * 16384
    // ---- PV over half hh of the tile for element e ----
    const uint32_t el = lane & 31, hh = lane >> 5, e = 32 * w + el;
    v4u vr[4];
    slice_v_rows(sm.scr[w], regs, lane, vr);
#pragma unroll
    for (int c = 0; c < 4; c++)  // chunks holding no cached position: zero
        vr[c] = tile * TILE + 32 * hh + 8 * c < a.pos0 ? vr[c] : v4u{0, 0, 0, 0};
    for (uint32_t r = tr.r0; r < tr.r0 + tr.nrow; r++) {
        const uint32_t slot = paired((a.pos0 + r) % TILE);
        if (slot / 32 != hh) continue;
#pragma unroll
        for (int c = 0; c < 4; c++)
            if ((slot % 32) / 8 == (uint32_t)c) vr[c] = put_half(vr[c], slot % 8, sm.kv[r][e]);
    }
    uint32_t mv = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) vr[c] = clamp4(vr[c], mv);
    const bool vcorr = __any(mv != 0);
    int32_t b0 = 0, b1 = 0, b2 = 0, b3 = 0;
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
    b0 += __shfl_xor(b0, 32, 64);
    b1 += __shfl_xor(b1, 32, 64);
    b2 += __shfl_xor(b2, 32, 64);
    b3 += __shfl_xor(b3, 32, 64);
    int32_t tv = fx_sat32((int64_t)b0 + b1 + b2 + b3);
    tv = sat16_32(rnd32(rnd32(tv, 6), 8));  // rnd(tv 2^10, 16) = rnd(tv, 6)
    {  // elements e..e+3 in one 8-byte store (lane % 4 == 0 of each half-wave)
        const uint32_t t1 = (uint16_t)__shfl_down(tv, 1, 64), t2 = (uint16_t)__shfl_down(tv, 2, 64),
                       t3 = (uint16_t)__shfl_down(tv, 3, 64);
        const uint64_t q4 = (uint64_t)((uint16_t)tv | (t1 << 16)) | ((uint64_t)(t2 | (t3 << 16)) << 32);
        if (hh == 0 && (lane & 3) == 0) st_coherent((uint64_t*)&a.s_tval[base * D + e], q4);
    }
    if (gi == 0 && own / TILE == tile && tid < D)  // this row's V into the cache
        a.vcache[page_off<D>(a, h, tile) + tid * TILE + paired(own % TILE)] = sm.kv[t][tid];
    if (FUSED) {
        // the PV values are performed, then the flagged sum is published
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            st_coherent(&a.s_tsum[base], (int32_t)(kSumValid | (uint32_t)tsum));
            __builtin_amdgcn_s_waitcnt(0);  // before this workgroup reads it back
        }
        if (tile + 1 != ntiles) return;
        // the last tile's workgroup: every earlier tile's sum is published
        uint32_t v = 0;
        if (!poll_flags((const uint32_t*)&a.s_tsum[rh * a.max_tiles * G + gi], G, tile,
                        kSumValid, &v, a.wait_limit, a.abort, a.host_abort, &sm.last))
            return;
    } else {
        // ---- the last tile of this (row, query head) to arrive runs the
        // recurrence ----
        if (tid == 0) st_coherent(&a.s_tsum[base], tsum);
        const uint32_t ng = tile_groups(a.max_tiles), grp = tile / kArriveGroup;
        uint32_t* top = a.counters + ((size_t)t * a.num_heads + g) * (1 + ng) * kCounterStride;
        const uint32_t in_grp = ntiles - grp * kArriveGroup < kArriveGroup
                                    ? ntiles - grp * kArriveGroup : kArriveGroup;
        if (!arrive_last(top + (1 + grp) * kCounterStride, in_grp, &sm.last)) return;
        if (!arrive_last(top, tile_groups(ntiles), &sm.last)) return;
    }
    // Steps padded with (maximum INT16_MIN, sum 0, value 0) change
    // nothing.
    int32_t m = INT16_MIN, sum = 0, acc = 0;
    constexpr uint32_t kElemWaves = (D + 63) / 64;         // wavefronts holding elements
    constexpr bool kSumWave = NTH / 64 > kElemWaves;       // one more for the sum
    constexpr int PL = 64 * D / 4 / NTH;  // 4-value groups per thread per piece
    // A piece's operands are loaded while the previous piece is computed.
    struct Piece {
        uint64_t vals[PL];
        int32_t tm, tsv;
    };
    auto load_piece = [&](uint32_t j0, Piece& pc) {
        const uint32_t nj = j0 < ntiles ? (ntiles - j0 < 64 ? ntiles - j0 : 64) : 0;
#pragma unroll
        for (int u = 0; u < PL; u++) {  // all in flight
            const uint32_t i = 4 * (tid + NTH * u), j = i / D, ee = i % D;
            pc.vals[u] = j < nj ? ld_coherent((const uint64_t*)&a.s_tval[
                                      ((rh * a.max_tiles + j0 + j) * G + gi) * D + ee])
                                : 0ull;
        }
        pc.tm = INT16_MIN;
        pc.tsv = 0;
        if (tid < nj) {
            const size_t b = (rh * a.max_tiles + j0 + tid) * G + gi;
            if (FUSED) {
                pc.tm = (int16_t)(ld_coherent(&a.s_tmax32[b]) & 0xffff);
                pc.tsv = (int32_t)((uint32_t)ld_coherent(&a.s_tsum[b]) & ~kSumValid);
            } else {
                pc.tm = a.s_tmax[b];
                pc.tsv = ld_coherent(&a.s_tsum[b]);
            }
        }
    };
    Piece cur;
    load_piece(0, cur);
    for (uint32_t j0 = 0; j0 < ntiles; j0 += 64) {
        const uint32_t nj = ntiles - j0 < 64 ? ntiles - j0 : 64;
        lds_barrier();  // the previous piece consumed
#pragma unroll
        for (int u = 0; u < PL; u++) {
            const uint32_t i = 4 * (tid + NTH * u);
            *(uint64_t*)&sm.tv[i / D][i % D] = cur.vals[u];
        }
        if (tid < 64) {
            sm.tmax[tid] = cur.tm;
            sm.tsum[tid] = cur.tsv;
        }
        if (j0 + 64 < ntiles) load_piece(j0 + 64, cur);
        lds_barrier();
        // The same for every element, formed by every wavefront with all
        // its lanes: lane j holds tile j0 + j's maximum, the running
        // max before it (the max of m and the earlier maxima) and the
        // tile's rescale factor: exp(before - after) << 2 where the tile
        // raises the max, else 65536 (1.0), under which rnd(v * 2^16, 16) =
        // v leaves sum and acc as they are.
        const int32_t tmj = sm.tmax[lane];
        const int32_t before = wave_prefix_max_excl(tmj, m);
        const bool rise = tmj > before;
        // (lanes that do not rise look up exp(0): the table holds x <= 0)
        const int32_t pj = (int32_t)prob(sm.e14, rise ? before - tmj : 0) << 2;
        const int32_t fj = rise ? pj : 65536;
        m = max(m, wave_max(tmj));
        // Every tile the same straight-line step, the reference's per-tile
        // order and rounding, in full-rate 24-bit products: with v = 2^16 h
        // + l (l the low 16 bits) and f <= 2^16, rnd(v f, 16) = h f +
        // ((l f + 2^15) >> 16) exactly, |h f| <= 2^31 and l f < 2^32 - 2^15;
        // the rescaled acc stays within int32 (|v f / 2^16| <= |v|), and
        // every term of sum is non-negative, so its saturation is that of
        // nested saturating additions.  The factors go through LDS (a
        // wavefront's own copy: its LDS operations complete in order).  The
        // sum, the same for every element, is carried by the first
        // wavefront past the element lanes where the workgroup has one.
        sm.fac[w][lane] = fj;
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        auto sum_step = [&](int32_t sv, int32_t f, int32_t tk) -> int32_t {
            const uint32_t lo = (__umul24((uint32_t)sv & 0xffffu, (uint32_t)f) + 32768u) >> 16;
            return __builtin_elementwise_add_sat(
                __builtin_elementwise_add_sat(__mul24(sv >> 16, f), tk << 2), (int32_t)lo);
        };
        if (tid < D) {
            for (uint32_t j = 0; j < nj; j += 8) {
                int32_t tvv[8], fv[8], tk[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    tvv[u] = sm.tv[j + u][tid];
                    fv[u] = sm.fac[w][j + u];
                    if (!kSumWave) tk[u] = sm.tsum[j + u];
                }
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    if (!kSumWave) sum = sum_step(sum, fv[u], tk[u]);
                    acc = __builtin_elementwise_add_sat(rnd16_mul(acc, fv[u]), tvv[u] * 256);
                }
            }
        } else if (kSumWave && w == kElemWaves) {
            for (uint32_t j = 0; j < nj; j += 8) {
                int32_t fv[8], tk[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    fv[u] = sm.fac[w][j + u];
                    tk[u] = sm.tsum[j + u];
                }
#pragma unroll
                for (int u = 0; u < 8; u++) sum = sum_step(sum, fv[u], tk[u]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // fac read before the next piece
    }
    // 1 / sum (a division) on the sum's wavefront, beside the elements'
    // chains
    int32_t inv;
    if (kSumWave) {
        if (w == kElemWaves && lane == 0) sm.rinv = fx_inv_sum(sum);
        lds_barrier();
        inv = sm.rinv;
    } else {
        inv = fx_inv_sum(sum);
    }
    if (tid < D) {
        const int16_t o = sat16_32(rnd16_mul(acc, inv));  // 0 <= inv < 2^15
        int16_t* op = &a.out[(size_t)t * a.ldo + (size_t)g * D + tid];
        if (OARR)
            st_coherent(op, o);
        else
            *op = o;
    }
    if (FUSED) {
        // every tile of this (row, query head) has read the maxima and
        // published its sum: clear the flags for the next launch
        for (uint32_t j = tid; j < ntiles; j += NTH) {
            const size_t b = (rh * a.max_tiles + j) * G + gi;
            st_coherent(&a.s_tmax32[b], 0);
            st_coherent(&a.s_tsum[b], 0);
        }
    }
    if (OARR) arrive(a.attn_arrive, kSyncAttnLines, kSyncStride);
}

template <int D>
__global__ __launch_bounds__(D * 2) void attention_tile_pv_kernel(AttnArgs a) {
    __shared__ TilePvSmem<D> sm;
    const TileWg wg = tile_wg(a);
    if (!wg.valid) return;                             // padding
    if (wg.tile * TILE >= a.pos0 + wg.t + 1) return;   // beyond this row's context
    tile_pv_phase<D, false>(a, wg, sm, nullptr, nullptr);
}

// The tile path in one launch (contexts of at most kTileFusedMaxTiles
// tiles; launched only when every workgroup of the grid fits on the device
// at once, so that the workgroups a tile waits for are all running): the
// scores phase, which publishes the tile's flagged maximum, and the PV
// phase, which waits for the earlier tiles' maxima after issuing its own
// loads; the last tile's workgroup combines the tiles.
template <int D>
__global__ __launch_bounds__(D * 2) void attention_tile_fused_kernel(AttnArgs a) {
    __shared__ union {
        TileScoresSmem<D> s;
        TilePvSmem<D> p;
    } sm;
    __shared__ int16_t lsc[TILE];
    __shared__ int32_t lmt;
    const TileWg wg = tile_wg(a);
    if (!wg.valid) return;                        // padding
    const uint32_t n = a.pos0 + wg.t + 1;
    if (wg.tile * TILE >= n) return;              // beyond this row's context
    tile_scores_phase<D, true>(a, wg, sm.s, lsc, &lmt);
    __syncthreads();  // phase 1's LDS use ends
    tile_pv_phase<D, true>(a, wg, sm.p, lsc, &lmt);
}

// The one-launch tile path and the O projection in one launch (decode
// rows): tile workgroups as in attention_tile_fused_kernel, the combining
// workgroup of each (row, query head) storing its slice coherently and
// arriving on the attention counters; then O blocks (proj_block, two per
// workgroup) that issue their weight loads, wait for every (row, query
// head) and finish with the residual and FFN-norm epilogue.  Launched only
// when the whole grid is resident at once.
template <int D, int RT, int LW, bool P12, bool CORR = false>
__global__ __launch_bounds__(D * 2) void attention_tile_o_kernel(TileOArgs s) {
    constexpr int WPB = D / 32, SPW = 4;
    __shared__ union {
        TileScoresSmem<D> s;
        TilePvSmem<D> p;
    } sm;
    __shared__ int16_t lsc[TILE];
    __shared__ int32_t lmt;
    __shared__ int64_t red[kSubOBlocks * WPB * 4 * RT];
    __shared__ uint32_t flag;
    if (blockIdx.x < s.ntile) {
        const TileWg wg = tile_wg(s.at);
        if (!wg.valid) return;                    // padding
        if (wg.tile * TILE >= s.at.pos0 + wg.t + 1) return;  // beyond this row's context
        tile_scores_phase<D, true>(s.at, wg, sm.s, lsc, &lmt);
        __syncthreads();  // phase 1's LDS use ends
        tile_pv_phase<D, true, true>(s.at, wg, sm.p, lsc, &lmt);
        return;
    }
    const uint32_t b = blockIdx.x - s.ntile;
    proj_block<RT, EPI_RESID, WPB, SPW, true, false, LW, kSubOBlocks, P12, CORR>(s.o, b, red, [&] {
        return wait_counts(
            s.sync + kSyncAttn + kSyncStride * (b % kSyncAttnLines), 0, 1,
            [&](uint32_t) { return s.attn_base + s.arrivals; }, s.wait_limit, s.sync + kSyncAbort,
            s.host_abort, &flag);
    });
}

// Workgroups of the one-launch tile path the device holds at once.  The
// per-CU occupancy is a property of the kernel's gfx950 code object (the
// only target this library builds), the same on every device; it is
// queried once, under C++'s thread-safe initialisation of a local static.
template <int D>
uint32_t tile_fused_capacity(uint32_t cus) {
    static const int per_cu = [] {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nb, reinterpret_cast<const void*>(&attention_tile_fused_kernel<D>), 2 * D, 0) !=
            hipSuccess)
            nb = 0;
        return nb;
    }();
    return (uint32_t)per_cu * cus;
}
template <int D>
static hipError_t launch_d(const AttnArgs& a, uint32_t rows, uint32_t kv_heads,
                           uint32_t chunks, hipStream_t st) {
    const uint32_t tiles = (a.pos0 + rows + TILE - 1) / TILE;
    if (tiles > kSplitHeadMaxTiles && a.use_gqa && attention_gqa_ok(a, rows))
        return launch_attention_gqa(a, rows, st);
    if (D % 32 == 0 && tiles > kSplitHeadMaxTiles) {
        constexpr int DT = D % 32 == 0 ? D : 32;
        AttnArgs g = a;
        g.grid_rows = rows;
        g.grid_tiles = tiles;
        const uint32_t grid = tile_grid(rows, tiles, a.num_kv_heads, a.group);
        if (a.tile_fused && a.s_tmax32 && tiles <= kTileFusedMaxTiles &&
            grid <= tile_fused_capacity<DT>(a.cus)) {
            if (!a.coop) {
                attention_tile_fused_kernel<DT><<<grid, 2 * D, 0, st>>>(g);
                return hipGetLastError();
            }
            void* args[] = {&g};
            const hipError_t e = hipLaunchCooperativeKernel(
                reinterpret_cast<const void*>(&attention_tile_fused_kernel<DT>), dim3(grid),
                dim3(2 * D), args, 0, st);
            if (e != hipErrorCooperativeLaunchTooLarge) return e;
            (void)hipGetLastError();  // refused: the two launches below
        }
        attention_tile_scores_kernel<DT><<<grid, 2 * D, 0, st>>>(g);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        attention_tile_pv_kernel<DT><<<grid, 2 * D, 0, st>>>(g);
        return hipGetLastError();
    }
    if (D % 32 == 0 || chunks <= 1) {
        // a wavefront per (row, query head) for single rows and pairs; a
        // workgroup per (row, KV head) beyond (measured at configs[1])
        if (D % 32 == 0 && rows <= kSplitHeadRows)
            attention_split_head_kernel<D % 32 == 0 ? D : 32>
                <<<dim3(rows, a.num_heads), 2 * D, 0, st>>>(a);
        else if (rows <= kHeadPathRows)
            attention_head_kernel<D><<<dim3(rows, a.num_heads), 64, 0, st>>>(a);
        else
            attention_fused_kernel<D><<<dim3(rows, kv_heads), NT, 0, st>>>(a);
        return hipGetLastError();
    }
    attention_scores_kernel<D><<<dim3(rows, kv_heads, chunks), NT, 0, st>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    attention_pv_kernel<D><<<dim3(rows, kv_heads, chunks), NT, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, uint32_t rows, uint32_t kv_heads,
                            uint32_t chunks, hipStream_t st) {
    switch (a.head_dim) {
    case 16: return launch_d<16>(a, rows, kv_heads, chunks, st);
    case 32: return launch_d<32>(a, rows, kv_heads, chunks, st);
    case 48: return launch_d<48>(a, rows, kv_heads, chunks, st);
    case 64: return launch_d<64>(a, rows, kv_heads, chunks, st);
    case 80: return launch_d<80>(a, rows, kv_heads, chunks, st);
    case 96: return launch_d<96>(a, rows, kv_heads, chunks, st);
    case 112: return launch_d<112>(a, rows, kv_heads, chunks, st);
    case 128: return launch_d<128>(a, rows, kv_heads, chunks, st);
    default: return hipErrorInvalidValue;
    }
}


// The smallest residency over the widening and 12-bit variants of the
// launch.
template <int D, int RT, int QEPI>
static int sublayer_capacity_of(int cus) {
    int per_cu[5] = {0, 0, 0, 0, 0};
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu[0], attention_sublayer_kernel<D, RT, QEPI, 4>, 2 * D, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu[1], attention_sublayer_kernel<D, RT, QEPI, 1>, 2 * D, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu[2], attention_sublayer_kernel<D, RT, QEPI, 0>, 2 * D, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu[3], attention_sublayer_kernel<D, RT, QEPI, 4, true>, 2 * D, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu[4], attention_sublayer_kernel<D, RT, QEPI, 4, true, true>, 2 * D, 0) !=
            hipSuccess)
        return 0;
    return std::min({per_cu[0], per_cu[1], per_cu[2], per_cu[3], per_cu[4]}) * cus;
}

template <int D, int RT>
static int sublayer_capacity_q(int qkv_epi, int cus) {
    return qkv_epi == EPI_STORE_NORM_IN ? sublayer_capacity_of<D, RT, EPI_STORE_NORM_IN>(cus)
                                        : sublayer_capacity_of<D, RT, EPI_STORE>(cus);
}

int sublayer_capacity(uint32_t head_dim, uint32_t rows, int qkv_epi, int cus) {
    if (head_dim == 64)
        return rows == 1 ? sublayer_capacity_q<64, 1>(qkv_epi, cus)
                         : sublayer_capacity_q<64, 2>(qkv_epi, cus);
    if (head_dim == 128)
        return rows == 1 ? sublayer_capacity_q<128, 1>(qkv_epi, cus)
                         : sublayer_capacity_q<128, 2>(qkv_epi, cus);
    return 0;
}

uint32_t sublayer_qkv_workgroups(uint32_t blocks) {
    return (blocks + kSubQkvBlocks - 1) / kSubQkvBlocks;
}
uint32_t sublayer_o_workgroups(uint32_t blocks) {
    return (blocks + kSubOBlocks - 1) / kSubOBlocks;
}

bool sublayer_fused_ok(const SublayerArgs& s, uint32_t rows, int qkv_epi, int L_qkv, int L_o,
                       int capacity) {
    const uint32_t D = s.at.head_dim;
    if ((D != 64 && D != 128) || rows == 0 || rows > 2) return false;
    if (qkv_epi != EPI_STORE && qkv_epi != EPI_STORE_NORM_IN) return false;
    const uint32_t tiles = (s.at.pos0 + rows + TILE - 1) / TILE;
    if (tiles > kSplitHeadMaxTiles || rows > kSplitHeadRows) return false;
    // up to 4 k-steps per wavefront (any widening interval: see launch_sub)
    const uint32_t wpb = D / 32;
    (void)L_qkv;
    (void)L_o;
    if (s.qkv.steps > 4 * wpb || s.o.steps > 4 * wpb) return false;
    // both projections from their 12-bit copies, or both from the 16-bit
    if (!(sublayer_reads_p12(s) || (s.qkv.w0 && s.o.w0))) return false;
    if (!s.sync || !s.host_abort) return false;
    return (int64_t)s.na + s.no < capacity;
}

template <int D, int RT, int LW, bool P12 = false, bool CORR = false>
static void launch_sub_l(const SublayerArgs& s, int qkv_epi, hipStream_t st) {
    const uint32_t grid = s.nq + s.na + s.no;
    if (qkv_epi == EPI_STORE_NORM_IN)
        attention_sublayer_kernel<D, RT, EPI_STORE_NORM_IN, LW, P12, CORR><<<grid, 2 * D, 0, st>>>(s);
    else
        attention_sublayer_kernel<D, RT, EPI_STORE, LW, P12, CORR><<<grid, 2 * D, 0, st>>>(s);
}

bool sublayer_reads_p12(const SublayerArgs& s) {
#if LLM_SUB_P12
    return s.qkv.p0 && s.o.p0;
#else
    return !(s.qkv.w0 && s.o.w0) && s.qkv.p0 && s.o.p0;
#endif
}

// The int32 sums of the QKV and O roles (up to 4 k-steps per wavefront)
// widen once when both matrices' widening intervals reach 4, after every
// step when they are at least 1, and every product otherwise; from the
// 12-bit copies they never need to.
template <int D, int RT>
static void launch_sub(const SublayerArgs& s, int qkv_epi, int L, hipStream_t st) {
    if (sublayer_reads_p12(s) && (s.qkv.corr0 || s.o.corr0))
        launch_sub_l<D, RT, 4, true, true>(s, qkv_epi, st);
    else if (sublayer_reads_p12(s))
        launch_sub_l<D, RT, 4, true>(s, qkv_epi, st);
    else if (L >= 4) launch_sub_l<D, RT, 4>(s, qkv_epi, st);
    else if (L >= 1) launch_sub_l<D, RT, 1>(s, qkv_epi, st);
    else launch_sub_l<D, RT, 0>(s, qkv_epi, st);
}

hipError_t launch_attention_sublayer(const SublayerArgs& s, uint32_t rows, int qkv_epi,
                                     int L, hipStream_t st) {
    if (s.at.head_dim == 64)
        rows == 1 ? launch_sub<64, 1>(s, qkv_epi, L, st) : launch_sub<64, 2>(s, qkv_epi, L, st);
    else
        rows == 1 ? launch_sub<128, 1>(s, qkv_epi, L, st) : launch_sub<128, 2>(s, qkv_epi, L, st);
    return hipGetLastError();
}

// The variant of the tile + O launch for an O projection: 12-bit with
// corrections, 12-bit, or 16-bit at widening interval 4 / 1 / every
// product.
int tile_o_variant(const ProjArgs& o, int L) {
    if (o.p0 && o.corr0) return 4;
    if (o.p0) return 3;
    return L >= 4 ? 0 : (L >= 1 ? 1 : 2);
}

// Workgroups of one variant of the tile + O launch the device holds at
// once.
template <int D, int RT>
static int tile_o_capacity_of(int variant, int cus) {
    int pc = 0;
    hipError_t e;
    switch (variant) {
    case 0: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc, attention_tile_o_kernel<D, RT, 4, false>, 2 * D, 0); break;
    case 1: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc, attention_tile_o_kernel<D, RT, 1, false>, 2 * D, 0); break;
    case 2: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc, attention_tile_o_kernel<D, RT, 0, false>, 2 * D, 0); break;
    case 3: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc, attention_tile_o_kernel<D, RT, 4, true>, 2 * D, 0); break;
    default: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc, attention_tile_o_kernel<D, RT, 4, true, true>, 2 * D, 0); break;
    }
    return e == hipSuccess ? pc * cus : 0;
}

int tile_o_capacity(uint32_t head_dim, uint32_t rows, int variant, int cus) {
    if (head_dim == 64)
        return rows == 1 ? tile_o_capacity_of<64, 1>(variant, cus) : tile_o_capacity_of<64, 2>(variant, cus);
    if (head_dim == 128)
        return rows == 1 ? tile_o_capacity_of<128, 1>(variant, cus) : tile_o_capacity_of<128, 2>(variant, cus);
    return 0;
}

bool tile_o_prepare(TileOArgs& s, uint32_t rows, int capacity) {
    const AttnArgs& a = s.at;
    const uint32_t D = a.head_dim;
    if ((D != 64 && D != 128) || rows == 0 || rows > 2) return false;
    const uint32_t tiles = (a.pos0 + rows + TILE - 1) / TILE;
    // the attention launch would take the one-launch tile path
    if (tiles <= kSplitHeadMaxTiles || tiles > kTileFusedMaxTiles) return false;
    if (a.use_gqa && attention_gqa_ok(a, rows)) return false;
    if (!a.tile_fused || !a.s_tmax32 || a.coop) return false;
    // O: up to 4 k-steps per wavefront, from the 12-bit or the 16-bit copy
    if (s.o.steps > 4 * (D / 32) || !(s.o.p0 || s.o.w0)) return false;
    if (!s.sync || !s.host_abort) return false;
    s.at.grid_rows = rows;
    s.at.grid_tiles = tiles;
    s.at.attn_arrive = s.sync + kSyncAttn;
    s.ntile = tile_grid(rows, tiles, a.num_kv_heads, a.group);
    s.no = (((s.o.n + 3) / 4) + kSubOBlocks - 1) / kSubOBlocks;
    s.arrivals = rows * a.num_heads;
    return (int64_t)s.ntile + s.no <= capacity;
}

template <int D, int RT>
static void launch_tile_o_d(const TileOArgs& s, int L, hipStream_t st) {
    const uint32_t grid = s.ntile + s.no;
    switch (tile_o_variant(s.o, L)) {
    case 4: attention_tile_o_kernel<D, RT, 4, true, true><<<grid, 2 * D, 0, st>>>(s); break;
    case 3: attention_tile_o_kernel<D, RT, 4, true><<<grid, 2 * D, 0, st>>>(s); break;
    case 0: attention_tile_o_kernel<D, RT, 4, false><<<grid, 2 * D, 0, st>>>(s); break;
    case 1: attention_tile_o_kernel<D, RT, 1, false><<<grid, 2 * D, 0, st>>>(s); break;
    default: attention_tile_o_kernel<D, RT, 0, false><<<grid, 2 * D, 0, st>>>(s); break;
    }
}

hipError_t launch_attention_tile_o(const TileOArgs& s, uint32_t rows, int L, hipStream_t st) {
    if (s.at.head_dim == 64)
        rows == 1 ? launch_tile_o_d<64, 1>(s, L, st) : launch_tile_o_d<64, 2>(s, L, st);
    else
        rows == 1 ? launch_tile_o_d<128, 1>(s, L, st) : launch_tile_o_d<128, 2>(s, L, st);
    return hipGetLastError();
}

}  // namespace llm
