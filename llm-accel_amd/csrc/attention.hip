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
// So product = q * clamp(k, -2048, 2048) + [k >= 2048] * c(q), and a bank
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
// Cache pages (64 positions of one layer and KV head): K rows [64][d] with
// each row's elements in the bank-paired order, V transposed [d][64] with
// positions in the bank-paired order, so staging a tile is a straight
// 16-byte copy.
//
// Long contexts: the running max over tiles is a prefix max (exact), so
// tiles are split over workgroups: (A) scores and per-tile maxima, (B)
// probabilities, tile sums and per-tile PV values given the prefix max,
// and a sequential scan of the per-tile rounding recurrence performed by
// the last workgroup of each (row, KV head) to finish (atomic counter, no
// waiting).
#include "attention.h"

#include "fixed_point.h"

namespace llm {

namespace {

constexpr int TILE = 64;
constexpr int MAXG = 16;
constexpr int MAXD = 128;
constexpr int KROW = MAXD + 8;   // padded LDS row of the K tile (int16)
constexpr int VROW = TILE + 8;   // padded LDS row of the V^T tile (int16)

typedef short s16x2 __attribute__((ext_vector_type(2)));

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

// Clamp both int16 halves of a dword to [-2048, 2048]; mask halves that
// were >= 2048.
__device__ __forceinline__ void clamp_word(uint32_t w, uint32_t& cl, uint32_t& mk) {
    const int32_t lo = (int16_t)(w & 0xffff), hi = (int16_t)(w >> 16);
    cl = (uint32_t)(uint16_t)clamp_k(lo) | ((uint32_t)(uint16_t)clamp_k(hi) << 16);
    mk = (uint32_t)(lo >= 2048) | ((uint32_t)(hi >= 2048) << 16);
}

__device__ __forceinline__ int16_t prob(const int16_t* exp14, int32_t x) {
    x = fx_sat16(x);
    x = x < -2048 ? -2048 : x;
    return exp14[x + 2048];
}

__device__ __forceinline__ int32_t wave_max(int32_t v) {
    for (int off = 32; off > 0; off >>= 1) {
        int32_t o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}
__device__ __forceinline__ int32_t wave_sum(int32_t v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

struct __attribute__((aligned(16))) Smem {
    int16_t q[MAXG * MAXD];     // rotated queries, bank-paired
    int16_t cq[MAXG * MAXD];    // c(q) of every query element
    int16_t p[MAXG * TILE];     // Q2.14 probabilities, positions paired
    int16_t cp[MAXG * TILE];    // c(p)
    int16_t e14[2056];          // Q2.14 exp table, x = -2048..0
    union {
        struct {
            int16_t k[TILE * KROW];   // clamped K tile, rows bank-paired
            int16_t km[TILE * KROW];  // [K >= 2048]
        };
        struct {
            int16_t vt[MAXD * VROW];  // clamped V tile transposed
            int16_t vm[MAXD * VROW];  // [V >= 2048]
        };
    };
    int32_t pages[64];  // page index of every tile this workgroup visits
    int32_t flags[4];  // [0] K tile has a value >= 2048, [1] V tile does,
                       // [3] this workgroup finishes the scan
};

constexpr int MAXT = 64;  // tiles one workgroup may visit (page indices)

// Rotate (x0, x1) by the Q8.8 table entry (c, s): host:4765-4788.
__device__ __forceinline__ void rope_pair(int32_t x0, int32_t x1, int32_t c,
                                          int32_t s, int16_t& y0, int16_t& y1) {
    y0 = fx_sat16(fx_rnd((int64_t)x0 * c - (int64_t)x1 * s, 8));
    y1 = fx_sat16(fx_rnd((int64_t)x1 * c + (int64_t)x0 * s, 8));
}

__device__ __forceinline__ int16_t lane16(const uint4& v, uint32_t j) {
    const uint32_t w = j < 2 ? v.x : (j < 4 ? v.y : (j < 6 ? v.z : v.w));
    return (int16_t)((j & 1) ? (w >> 16) : (w & 0xffff));
}

// Tile range [t0, t1) of one workgroup and where the row sits.
struct Span {
    uint32_t t0, t1, n;  // tiles, context length of the row
};

// Prologue, one memory round trip: page indices of the span, the rotated
// query group with c(q), and (optionally) the exp table.
__device__ void prologue(const AttnArgs& a, Smem& sm, uint32_t t, uint32_t h,
                         const Span& sp, bool queries, bool exp_table) {
    const uint32_t d = a.head_dim, half = d / 2, G = a.group, hc = half / 8;
    const uint32_t pos = a.pos0 + t;
    const int16_t* rope = a.rope + (size_t)pos * d;
    const int16_t* q = a.qkv + (size_t)t * a.ldqkv + (size_t)h * G * d;
    const uint32_t tid = threadIdx.x;
    // issue
    int32_t page = 0;
    if (tid < sp.t1 - sp.t0) page = a.page_table[h * a.tiles + sp.t0 + tid];
    uint4 e = make_uint4(0, 0, 0, 0), e2 = e;
    if (exp_table) {
        e = *(const uint4*)(a.exp14 + 8 * tid);
        if (tid == 0) e2 = *(const uint4*)(a.exp14 + 8 * 256);
    }
    const bool qi = queries && tid < G * hc;
    const uint32_t g = qi ? tid / hc : 0, c = qi ? 8 * (tid % hc) : 0;
    uint4 x0 = e, x1 = e, cs = e, sn = e;
    if (qi) {
        x0 = *(const uint4*)(q + g * d + c);
        x1 = *(const uint4*)(q + g * d + half + c);
        cs = *(const uint4*)(rope + c);
        sn = *(const uint4*)(rope + half + c);
    }
    // commit
    if (tid < sp.t1 - sp.t0) sm.pages[tid] = page;
    if (exp_table) {
        *(uint4*)(sm.e14 + 8 * tid) = e;
        if (tid == 0) *(uint4*)(sm.e14 + 8 * 256) = e2;
    }
    if (qi) {
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) {
            int16_t y0, y1;
            rope_pair(lane16(x0, j), lane16(x1, j), lane16(cs, j), lane16(sn, j), y0, y1);
            sm.q[g * d + paired(c + j)] = y0;
            sm.q[g * d + paired(half + c + j)] = y1;
            sm.cq[g * d + paired(c + j)] = (int16_t)sat_corr(y0);
            sm.cq[g * d + paired(half + c + j)] = (int16_t)sat_corr(y1);
        }
    }
}

__device__ __forceinline__ uint32_t cached_in_tile(const AttnArgs& a, uint32_t tile,
                                                   uint32_t tl) {
    const uint32_t base = tile * TILE;
    return a.pos0 > base ? (a.pos0 - base < tl ? a.pos0 - base : tl) : 0;
}

// K tile in registers: cached rows from the page (16-byte chunks) and one
// current-block item (8 RoPE pairs of a row of the projection buffer).
struct KLoad {
    static constexpr int PER = TILE * (MAXD / 8) / 256;
    uint4 pg[PER];
    uint4 x0, x1, cs, sn;
};

__device__ void issue_k(const AttnArgs& a, const Smem& sm, uint32_t h,
                        uint32_t tile, uint32_t tl, const Span& sp, KLoad& L) {
    const uint32_t d = a.head_dim, half = d / 2, chunks = d / 8, hc = half / 8;
    const uint32_t ncache = cached_in_tile(a, tile, tl);
    const int16_t* page = a.kcache + (size_t)sm.pages[tile - sp.t0] * TILE * d;
#pragma unroll
    for (int u = 0; u < KLoad::PER; u++) {
        const uint32_t idx = threadIdx.x + 256 * u;
        if (idx < ncache * chunks)
            L.pg[u] = *(const uint4*)(page + (idx / chunks) * d + 8 * (idx % chunks));
    }
    const uint32_t idx = threadIdx.x;
    if (idx < (tl - ncache) * hc) {
        const uint32_t p = ncache + idx / hc, c = 8 * (idx % hc);
        const uint32_t pos = tile * TILE + p, r = pos - a.pos0;
        const int16_t* k = a.qkv + (size_t)r * a.ldqkv + a.num_heads * d + h * d;
        const int16_t* rope = a.rope + (size_t)pos * d;
        L.x0 = *(const uint4*)(k + c);
        L.x1 = *(const uint4*)(k + half + c);
        L.cs = *(const uint4*)(rope + c);
        L.sn = *(const uint4*)(rope + half + c);
    }
}

// Clamped K and its >= 2048 mask into LDS; the row `append_row` of the
// current block also goes to its page (after RoPE).
__device__ void commit_k(const AttnArgs& a, Smem& sm, uint32_t h, uint32_t tile,
                         uint32_t tl, const Span& sp, const KLoad& L,
                         int append_row) {
    const uint32_t d = a.head_dim, half = d / 2, chunks = d / 8, hc = half / 8;
    const uint32_t ncache = cached_in_tile(a, tile, tl);
    uint32_t any = 0;
#pragma unroll
    for (int u = 0; u < KLoad::PER; u++) {
        const uint32_t idx = threadIdx.x + 256 * u;
        if (idx >= ncache * chunks) break;
        const uint32_t p = idx / chunks, c = idx % chunks;
        uint4 cl, mk;
        clamp_word(L.pg[u].x, cl.x, mk.x);
        clamp_word(L.pg[u].y, cl.y, mk.y);
        clamp_word(L.pg[u].z, cl.z, mk.z);
        clamp_word(L.pg[u].w, cl.w, mk.w);
        *(uint4*)(sm.k + p * KROW + 8 * c) = cl;
        *(uint4*)(sm.km + p * KROW + 8 * c) = mk;
        any |= mk.x | mk.y | mk.z | mk.w;
    }
    const uint32_t idx = threadIdx.x;
    if (idx < (tl - ncache) * hc) {
        const uint32_t p = ncache + idx / hc, c = 8 * (idx % hc);
        const uint32_t r = tile * TILE + p - a.pos0;
        int16_t* page = a.kcache + (size_t)sm.pages[tile - sp.t0] * TILE * d;
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) {
            int16_t y0, y1;
            rope_pair(lane16(L.x0, j), lane16(L.x1, j), lane16(L.cs, j),
                      lane16(L.sn, j), y0, y1);
            const uint32_t e0 = paired(c + j), e1 = paired(half + c + j);
            sm.k[p * KROW + e0] = (int16_t)clamp_k(y0);
            sm.k[p * KROW + e1] = (int16_t)clamp_k(y1);
            sm.km[p * KROW + e0] = y0 >= 2048;
            sm.km[p * KROW + e1] = y1 >= 2048;
            any |= (y0 >= 2048) | (y1 >= 2048);
            if ((int)r == append_row) {
                page[p * d + e0] = y0;
                page[p * d + e1] = y1;
            }
        }
    }
    if (any) atomicOr(&sm.flags[0], 1);
}

// V tile in registers: page chunks of 8 paired positions of one element
// (cached positions) and one current-block item (8 elements of a row).
struct VLoad {
    static constexpr int PER = MAXD * (TILE / 8) / 256;
    uint4 pg[PER];
    uint4 cur;
};

__device__ void issue_v(const AttnArgs& a, const Smem& sm, uint32_t h,
                        uint32_t tile, uint32_t tl, const Span& sp,
                        uint32_t ncache, VLoad& L) {
    const uint32_t d = a.head_dim;
    const int16_t* page = a.vcache + (size_t)sm.pages[tile - sp.t0] * TILE * d;
#pragma unroll
    for (int u = 0; u < VLoad::PER; u++) {
        const uint32_t idx = threadIdx.x + 256 * u;
        const uint32_t e = idx / (TILE / 8), c = idx % (TILE / 8);
        L.pg[u] = make_uint4(0, 0, 0, 0);
        if (e < d && 8 * c < ncache) L.pg[u] = *(const uint4*)(page + e * TILE + 8 * c);
    }
    const uint32_t idx = threadIdx.x;
    if (idx < (tl - ncache) * (d / 8)) {
        const uint32_t r = tile * TILE + ncache + idx / (d / 8) - a.pos0;
        L.cur = *(const uint4*)(a.qkv + (size_t)r * a.ldqkv +
                                (a.num_heads + a.num_kv_heads) * d + h * d +
                                8 * (idx % (d / 8)));
    }
}

// Phase 1: page chunks (non-cached slots zero) into LDS.
__device__ void commit_v_pages(const AttnArgs& a, Smem& sm, uint32_t ncache,
                               const VLoad& L) {
    const uint32_t d = a.head_dim;
    uint32_t any = 0;
#pragma unroll
    for (int u = 0; u < VLoad::PER; u++) {
        const uint32_t idx = threadIdx.x + 256 * u;
        const uint32_t e = idx / (TILE / 8), c = idx % (TILE / 8);
        if (e >= d) break;
        uint32_t w[4] = {L.pg[u].x, L.pg[u].y, L.pg[u].z, L.pg[u].w};
        if (8 * c + 8 > ncache) {
#pragma unroll
            for (uint32_t j = 0; j < 8; j++)
                if (8 * c + slot_pos(j) >= ncache)
                    w[j >> 1] &= ~(0xffffu << (16 * (j & 1)));
        }
        uint4 cl, mk;
        clamp_word(w[0], cl.x, mk.x);
        clamp_word(w[1], cl.y, mk.y);
        clamp_word(w[2], cl.z, mk.z);
        clamp_word(w[3], cl.w, mk.w);
        *(uint4*)(sm.vt + e * VROW + 8 * c) = cl;
        *(uint4*)(sm.vm + e * VROW + 8 * c) = mk;
        any |= mk.x | mk.y | mk.z | mk.w;
    }
    if (any) atomicOr(&sm.flags[1], 1);
}

// Phase 2 (after a barrier): current-block rows scattered into their
// slots; the row `append_row` also goes to its page.
__device__ void commit_v_rows(const AttnArgs& a, Smem& sm, uint32_t tile,
                              uint32_t tl, const Span& sp, uint32_t ncache,
                              const VLoad& L, int append_row) {
    const uint32_t d = a.head_dim;
    const uint32_t idx = threadIdx.x;
    if (idx >= (tl - ncache) * (d / 8)) return;
    const uint32_t p = ncache + idx / (d / 8), c = 8 * (idx % (d / 8));
    const uint32_t r = tile * TILE + p - a.pos0;
    int16_t* page = a.vcache + (size_t)sm.pages[tile - sp.t0] * TILE * d;
    uint32_t any = 0;
#pragma unroll
    for (uint32_t j = 0; j < 8; j++) {
        const int32_t v = lane16(L.cur, j);
        sm.vt[(c + j) * VROW + paired(p)] = (int16_t)clamp_k(v);
        sm.vm[(c + j) * VROW + paired(p)] = v >= 2048;
        any |= v >= 2048;
        if ((int)r == append_row) page[(c + j) * TILE + paired(p)] = (int16_t)v;
    }
    if (any) atomicOr(&sm.flags[1], 1);
}

// Score of query head g at tile position p.
__device__ __forceinline__ int16_t tile_score(const AttnArgs& a, const Smem& sm,
                                              uint32_t g, uint32_t p, bool corr,
                                              int64_t scale) {
    const uint32_t d = a.head_dim;
    const int16_t* qg = sm.q + g * d;
    const int16_t* kp = sm.k + p * KROW;
    int32_t b0 = 0, b1 = 0, b2 = 0, b3 = 0;
    for (uint32_t c = 0; c < d; c += 8) {
        const uint4 kv = *(const uint4*)(kp + c);
        const uint4 qv = *(const uint4*)(qg + c);
        b0 = dot2(kv.x, qv.x, b0);
        b1 = dot2(kv.y, qv.y, b1);
        b2 = dot2(kv.z, qv.z, b2);
        b3 = dot2(kv.w, qv.w, b3);
    }
    if (corr) {
        const int16_t* cg = sm.cq + g * d;
        const int16_t* mp = sm.km + p * KROW;
        for (uint32_t c = 0; c < d; c += 8) {
            const uint4 mv = *(const uint4*)(mp + c);
            const uint4 cv = *(const uint4*)(cg + c);
            b0 = dot2(mv.x, cv.x, b0);
            b1 = dot2(mv.y, cv.y, b1);
            b2 = dot2(mv.z, cv.z, b2);
            b3 = dot2(mv.w, cv.w, b3);
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

// Q8.8 PV tile value of (query head g, element e): banks, x fm(1/64).
__device__ __forceinline__ int32_t tile_pv(const Smem& sm, uint32_t g,
                                           uint32_t e, bool corr) {
    const int16_t* pg = sm.p + g * TILE;
    const int16_t* ve = sm.vt + e * VROW;
    int32_t b0 = 0, b1 = 0, b2 = 0, b3 = 0;
#pragma unroll
    for (uint32_t c = 0; c < TILE; c += 8) {
        const uint4 vv = *(const uint4*)(ve + c);
        const uint4 pv = *(const uint4*)(pg + c);
        b0 = dot2(vv.x, pv.x, b0);
        b1 = dot2(vv.y, pv.y, b1);
        b2 = dot2(vv.z, pv.z, b2);
        b3 = dot2(vv.w, pv.w, b3);
    }
    if (corr) {
        const int16_t* cg = sm.cp + g * TILE;
        const int16_t* me = sm.vm + e * VROW;
#pragma unroll
        for (uint32_t c = 0; c < TILE; c += 8) {
            const uint4 mv = *(const uint4*)(me + c);
            const uint4 cv = *(const uint4*)(cg + c);
            b0 = dot2(mv.x, cv.x, b0);
            b1 = dot2(mv.y, cv.y, b1);
            b2 = dot2(mv.z, cv.z, b2);
            b3 = dot2(mv.w, cv.w, b3);
        }
    }
    int32_t t = fx_sat32((int64_t)b0 + b1 + b2 + b3);
    t = fx_sat32(fx_rnd((int64_t)t * 1024, 16));
    return fx_sat16(fx_rnd(t, 8));
}

__device__ __forceinline__ void put_prob(Smem& sm, uint32_t g, uint32_t lane,
                                         int32_t pr) {
    sm.p[g * TILE + paired(lane)] = (int16_t)pr;
    sm.cp[g * TILE + paired(lane)] = (int16_t)sat_corr(pr);
}

__device__ __forceinline__ uint32_t row_tiles(const AttnArgs& a, uint32_t t) {
    return (a.pos0 + t + 1 + TILE - 1) / TILE;
}

}  // namespace

// ---------------------------------------------------------------------
// Fused path: one workgroup per (row, KV head) walks every tile.
// 256 threads; wave w owns query heads w, w+4, ...; in QK and softmax
// lanes are tile positions, in PV lanes are head elements.  Each tile costs
// one memory round trip: its K and V loads are issued together and V stays
// in registers while QK runs.
// ---------------------------------------------------------------------
__global__ __launch_bounds__(256) void attention_fused_kernel(AttnArgs a) {
    __shared__ Smem sm;
    const uint32_t t = blockIdx.x, h = blockIdx.y;
    const uint32_t G = a.group, d = a.head_dim;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = a.pos0 + t + 1;
    const Span sp{0, (n + TILE - 1) / TILE, n};
    const int64_t scale = (int64_t)a.qk_scale << 8;
    prologue(a, sm, t, h, sp, true, true);

    constexpr int GW = MAXG / 4;  // query heads per wave (max)
    constexpr int EW = MAXD / 64; // element chunks per lane (max)
    int32_t m[GW], sum[GW], acc[GW][EW];
#pragma unroll
    for (int i = 0; i < GW; i++) {
        m[i] = INT16_MIN;  // fm(-128)
        sum[i] = 0;
#pragma unroll
        for (int j = 0; j < EW; j++) acc[i][j] = 0;
    }

    for (uint32_t tile = 0; tile < sp.t1; tile++) {
        const uint32_t tl = n - tile * TILE < TILE ? n - tile * TILE : TILE;
        const uint32_t ncache = cached_in_tile(a, tile, tl);
        if (threadIdx.x == 0) sm.flags[0] = sm.flags[1] = 0;
        __syncthreads();  // pages/queries staged; previous PV finished
        KLoad kl;
        VLoad vl;
        issue_k(a, sm, h, tile, tl, sp, kl);
        issue_v(a, sm, h, tile, tl, sp, ncache, vl);
        commit_k(a, sm, h, tile, tl, sp, kl, (int)t);
        __syncthreads();
        const bool kcorr = sm.flags[0] != 0;
#pragma unroll
        for (int gi = 0; gi < GW; gi++) {
            const uint32_t g = wave + 4 * gi;
            if (g >= G) break;
            const bool valid = lane < tl;
            const int32_t s = valid ? tile_score(a, sm, g, lane, kcorr, scale)
                                    : INT16_MIN;
            const int32_t wm = wave_max(s);
            const int32_t mn = wm > m[gi] ? wm : m[gi];
            const int32_t old = prob(sm.e14, m[gi] - mn);
            const int32_t pr = valid ? prob(sm.e14, s - mn) : 0;
            put_prob(sm, g, lane, pr);
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
        __syncthreads();  // K tile consumed: V reuses its storage
        commit_v_pages(a, sm, ncache, vl);
        __syncthreads();
        commit_v_rows(a, sm, tile, tl, sp, ncache, vl, (int)t);
        __syncthreads();
        const bool vcorr = sm.flags[1] != 0;
#pragma unroll
        for (int gi = 0; gi < GW; gi++) {
            const uint32_t g = wave + 4 * gi;
            if (g >= G) break;
#pragma unroll
            for (int ei = 0; ei < EW; ei++) {
                const uint32_t e = lane + 64 * ei;
                if (e >= d) break;
                const int32_t tv = tile_pv(sm, g, e, vcorr);
                acc[gi][ei] = fx_sat32((int64_t)acc[gi][ei] + ((int64_t)tv << 8));
            }
        }
    }
    int16_t* dst = a.out + (size_t)t * a.ldo + (size_t)h * G * d;
#pragma unroll
    for (int gi = 0; gi < GW; gi++) {
        const uint32_t g = wave + 4 * gi;
        if (g >= G) break;
        const int64_t inv = fx_inv_sum(sum[gi]);
#pragma unroll
        for (int ei = 0; ei < EW; ei++) {
            const uint32_t e = lane + 64 * ei;
            if (e >= d) break;
            dst[g * d + e] = fx_sat16(fx_rnd((int64_t)acc[gi][ei] * inv, 16));
        }
    }
}

// ---------------------------------------------------------------------
// Split path, phase A: scores and tile maxima for a chunk of tiles; the
// row's own K and V are appended by the chunk that holds its position.
// grid (rows, kv_heads, chunks).
// ---------------------------------------------------------------------
__global__ __launch_bounds__(256) void attention_scores_kernel(AttnArgs a) {
    __shared__ Smem sm;
    const uint32_t t = blockIdx.x, h = blockIdx.y, c = blockIdx.z;
    const uint32_t G = a.group, d = a.head_dim;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = a.pos0 + t + 1, ntiles = row_tiles(a, t);
    const uint32_t t0 = c * a.chunk_tiles;
    if (t0 >= ntiles) return;
    const Span sp{t0, t0 + a.chunk_tiles < ntiles ? t0 + a.chunk_tiles : ntiles, n};
    const int64_t scale = (int64_t)a.qk_scale << 8;
    prologue(a, sm, t, h, sp, true, false);
    const size_t rh = (size_t)t * a.num_kv_heads + h;
    for (uint32_t tile = sp.t0; tile < sp.t1; tile++) {
        const uint32_t tl = n - tile * TILE < TILE ? n - tile * TILE : TILE;
        if (threadIdx.x == 0) sm.flags[0] = 0;
        __syncthreads();
        KLoad kl;
        issue_k(a, sm, h, tile, tl, sp, kl);
        commit_k(a, sm, h, tile, tl, sp, kl, (int)t);
        __syncthreads();
        const bool kcorr = sm.flags[0] != 0;
        for (uint32_t g = wave; g < G; g += 4) {
            const bool valid = lane < tl;
            const int32_t s = valid ? tile_score(a, sm, g, lane, kcorr, scale)
                                    : INT16_MIN;
            const size_t base = (rh * a.max_tiles + tile) * G + g;
            a.s_scores[base * TILE + lane] = (int16_t)s;
            const int32_t mx = wave_max(s);
            if (lane == 0) a.s_tmax[base] = (int16_t)mx;
        }
        __syncthreads();
    }
    const uint32_t own = (a.pos0 + t) / TILE;
    if (own >= sp.t0 && own < sp.t1) {
        const uint32_t slot = (a.pos0 + t) % TILE;
        const int16_t* v = a.qkv + (size_t)t * a.ldqkv +
                           (a.num_heads + a.num_kv_heads) * d + h * d;
        int16_t* page = a.vcache + (size_t)sm.pages[own - sp.t0] * TILE * d;
        for (uint32_t e = threadIdx.x; e < d; e += blockDim.x)
            page[e * TILE + paired(slot)] = v[e];
    }
}

// ---------------------------------------------------------------------
// Split path, phase B: probabilities, tile sums and PV values for a chunk
// given the prefix max; the last chunk of a (row, KV head) to finish runs
// the sequential rounding scan and writes the output.
// ---------------------------------------------------------------------
__global__ __launch_bounds__(256) void attention_pv_kernel(AttnArgs a) {
    __shared__ Smem sm;
    __shared__ int32_t mrun[MAXG];
    const uint32_t t = blockIdx.x, h = blockIdx.y, c = blockIdx.z;
    const uint32_t G = a.group, d = a.head_dim;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = a.pos0 + t + 1, ntiles = row_tiles(a, t);
    const uint32_t nchunks = (ntiles + a.chunk_tiles - 1) / a.chunk_tiles;
    const uint32_t t0 = c * a.chunk_tiles;
    if (t0 >= ntiles) return;
    const Span sp{t0, t0 + a.chunk_tiles < ntiles ? t0 + a.chunk_tiles : ntiles, n};
    const size_t rh = (size_t)t * a.num_kv_heads + h;
    if (threadIdx.x < G) mrun[threadIdx.x] = INT16_MIN;
    prologue(a, sm, t, h, sp, false, true);
    __syncthreads();
    // running max before this chunk: parallel over (tile, head)
    for (uint32_t idx = threadIdx.x; idx < t0 * G; idx += blockDim.x)
        atomicMax(&mrun[idx % G], (int32_t)a.s_tmax[(rh * a.max_tiles + idx / G) * G + idx % G]);
    for (uint32_t tile = sp.t0; tile < sp.t1; tile++) {
        const uint32_t tl = n - tile * TILE < TILE ? n - tile * TILE : TILE;
        if (threadIdx.x == 0) sm.flags[1] = 0;
        __syncthreads();
        VLoad vl;
        issue_v(a, sm, h, tile, tl, sp, tl, vl);
        int32_t sc[MAXG / 4], tm[MAXG / 4];
#pragma unroll
        for (int gi = 0; gi < MAXG / 4; gi++) {
            const uint32_t g = wave + 4 * gi;
            if (g >= G) break;
            const size_t base = (rh * a.max_tiles + tile) * G + g;
            sc[gi] = a.s_scores[base * TILE + lane];
            tm[gi] = a.s_tmax[base];
        }
        commit_v_pages(a, sm, tl, vl);
#pragma unroll
        for (int gi = 0; gi < MAXG / 4; gi++) {
            const uint32_t g = wave + 4 * gi;
            if (g >= G) break;
            const int32_t mn = tm[gi] > mrun[g] ? tm[gi] : mrun[g];
            const int32_t pr = lane < tl ? prob(sm.e14, sc[gi] - mn) : 0;
            put_prob(sm, g, lane, pr);
            const int32_t ts = wave_sum(pr);
            if (lane == 0) a.s_tsum[(rh * a.max_tiles + tile) * G + g] = ts;
        }
        __syncthreads();
        const bool vcorr = sm.flags[1] != 0;
        for (uint32_t idx = threadIdx.x; idx < G * d; idx += blockDim.x) {
            const uint32_t g = idx / d, e = idx % d;
            const size_t base = (rh * a.max_tiles + tile) * G + g;
            a.s_tval[base * d + e] = (int16_t)tile_pv(sm, g, e, vcorr);
        }
        __syncthreads();
        if (threadIdx.x < G) {
            const int32_t v = a.s_tmax[(rh * a.max_tiles + tile) * G + threadIdx.x];
            mrun[threadIdx.x] = v > mrun[threadIdx.x] ? v : mrun[threadIdx.x];
        }
    }
    // Publish, then let the last chunk of this (row, head) finish.
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = atomicAdd(&a.counters[rh], 1u);
        sm.flags[3] = prev == nchunks - 1;
    }
    __syncthreads();
    if (!sm.flags[3]) return;
    __threadfence();
    // Rescale factor and tile sum of every (tile, head), staged in LDS
    // (the p / cp arrays are free now): old in p, sum recurrence per head.
    constexpr int SB = 16;  // tiles whose values are in flight together
    for (uint32_t idx = threadIdx.x; idx < G * d; idx += blockDim.x) {
        const uint32_t g = idx / d, e = idx % d;
        int32_t m = INT16_MIN, sum = 0, acc = 0;
        for (uint32_t j0 = 0; j0 < ntiles; j0 += SB) {
            int32_t tv[SB], tmx[SB], tsm[SB];
#pragma unroll
            for (int u = 0; u < SB; u++) {
                const uint32_t j = j0 + u;
                if (j < ntiles) {
                    const size_t base = (rh * a.max_tiles + j) * G + g;
                    tv[u] = a.s_tval[base * d + e];
                    tmx[u] = a.s_tmax[base];
                    tsm[u] = a.s_tsum[base];
                }
            }
#pragma unroll
            for (int u = 0; u < SB; u++) {
                if (j0 + u >= ntiles) break;
                const int32_t mn = tmx[u] > m ? tmx[u] : m;
                const int64_t old = (int64_t)prob(sm.e14, m - mn) << 2;
                sum = fx_sat32(fx_rnd((int64_t)sum * old + ((int64_t)tsm[u] << 18), 16));
                acc = fx_sat32(fx_rnd((int64_t)acc * old, 16));
                acc = fx_sat32((int64_t)acc + ((int64_t)tv[u] << 8));
                m = mn;
            }
        }
        const int64_t inv = fx_inv_sum(sum);
        a.out[(size_t)t * a.ldo + (size_t)h * G * d + idx] =
            fx_sat16(fx_rnd((int64_t)acc * inv, 16));
    }
    if (threadIdx.x == 0) a.counters[rh] = 0;  // ready for the next launch
}

hipError_t launch_attention(const AttnArgs& a, uint32_t rows, uint32_t kv_heads,
                            uint32_t chunks, hipStream_t st) {
    if (chunks <= 1) {
        attention_fused_kernel<<<dim3(rows, kv_heads), 256, 0, st>>>(a);
        return hipGetLastError();
    }
    attention_scores_kernel<<<dim3(rows, kv_heads, chunks), 256, 0, st>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    attention_pv_kernel<<<dim3(rows, kv_heads, chunks), 256, 0, st>>>(a);
    return hipGetLastError();
}

}  // namespace llm
