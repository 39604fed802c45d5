// ops.hip -- kernels of the operator-level commands: QK / PV / softmax over
// one 64-position tile, flash attention over the paged cache, the KV
// append of DECODE_SMOKE, SiLU*up and residual add.
//
// These are the reference's diagnostic granularity (one operator per
// controller command), not the resident path: each kernel is a plain,
// exact restatement sized for a few rows, with one workgroup per query
// row.  Arithmetic follows the reference's golden definitions of the same
// operators (host/host_qwen_8x64.cpp:3144-3278, :3419-3575, :3609-3738;
// kernel/compute_stream.cpp:123-147, :205-225, :388-478).
#include "ops.h"

#include "attn_common.h"
#include "fixed_point.h"

namespace llm {
namespace {

// One attention product term: a Q8.8 value times golden_weight_t of a Q8.8
// value (saturated to Q4.12), AP_RND-narrowed to Q16.16
// (host/host_qwen_8x64.cpp:3243-3256).  |a * w| <= 2^30, so the product
// and its rounding fit int32.
__device__ __forceinline__ int32_t wt_term(int32_t a, int32_t b) {
    return (a * fx_fm_to_wt(b) + 8) >> 4;
}

// Bank sums.  Every term has |t| <= 2^26 and a bank of the reference adds
// at most 32 of them (head_dim <= 128, tiles of 64 positions): a running
// sum can leave the int32 range only at its last term, so the exact sum
// clamped once equals the reference's saturating running sum.
struct Banks {
    int64_t b[4] = {0, 0, 0, 0};
    __device__ __forceinline__ void add(uint32_t idx, int32_t t) {
        const uint32_t j = idx & 3u;
        b[0] += j == 0 ? t : 0;
        b[1] += j == 1 ? t : 0;
        b[2] += j == 2 ? t : 0;
        b[3] += j == 3 ? t : 0;
    }
    // golden_accum_t(banks[0] + banks[1] + banks[2] + banks[3])
    __device__ __forceinline__ int32_t total() const {
        return fx_sat32((int64_t)fx_sat32(b[0]) + fx_sat32(b[1]) + fx_sat32(b[2]) +
                        fx_sat32(b[3]));
    }
};

// QK narrowing: total *= accum(fm(1/sqrt(d))), then fm().
__device__ __forceinline__ int32_t qk_score(int32_t total, int32_t qk_scale) {
    const int32_t scaled = fx_sat32(fx_rnd((int64_t)total * ((int64_t)qk_scale << 8), 16));
    return fx_sat16(fx_rnd(scaled, 8));
}

// Element index of slot s of a bank-paired row (groups of 8 stored as
// elements [0 4 1 5 2 6 3 7]).
__device__ __forceinline__ uint32_t slot_elem(uint32_t s) {
    return (s & ~7u) | slot_pos(s & 7u);
}

// exp of a score difference (<= 0), clamped to [-8, 0] in Q8.8: the Q8.8
// table (legacy) or the Q2.14 table, both indexed x + 2048.
__device__ __forceinline__ int32_t exp_diff(int32_t dlt, const int16_t* table) {
    dlt = fx_sat16(dlt);
    dlt = dlt < -2048 ? -2048 : (dlt > 0 ? 0 : dlt);
    return table[dlt + 2048];
}

// ---------------------------------------------------------------------
// ATTN_QK (golden_attention_mm(q, k, 64, true), host:3219-3278): one
// workgroup per query row, one lane per tile position.
// ---------------------------------------------------------------------
__global__ __launch_bounds__(64) void op_qk_kernel(const int16_t* __restrict__ q,
                                                   const int16_t* __restrict__ k,
                                                   uint32_t group, uint32_t d,
                                                   uint32_t tile_len, int32_t qk_scale,
                                                   int16_t* __restrict__ out) {
    const uint32_t row = blockIdx.x, h = row / group, p = threadIdx.x;
    int32_t y = 0;
    if (p < tile_len) {
        const int16_t* qr = q + (size_t)row * d;
        const int16_t* kr = k + ((size_t)h * tile_len + p) * d;
        Banks bk;
        for (uint32_t e = 0; e < d; e++) bk.add(e, wt_term(qr[e], kr[e]));
        y = qk_score(bk.total(), qk_scale);
    }
    out[(size_t)row * 64 + p] = (int16_t)y;
}

// ---------------------------------------------------------------------
// ATTN_PV (golden_attention_mm(p, v, d, false), host:3219-3278): one
// workgroup per query row, one lane per output element.
// ---------------------------------------------------------------------
__global__ __launch_bounds__(128) void op_pv_kernel(const int16_t* __restrict__ p,
                                                    const int16_t* __restrict__ v,
                                                    uint32_t group, uint32_t d,
                                                    uint32_t tile_len,
                                                    int16_t* __restrict__ out) {
    const uint32_t row = blockIdx.x, h = row / group, e = threadIdx.x;
    if (e >= d) return;
    const int16_t* pr = p + (size_t)row * 64;
    const int16_t* vh = v + (size_t)h * tile_len * d;
    Banks bk;
    for (uint32_t j = 0; j < tile_len; j++) bk.add(j, wt_term(pr[j], vh[(size_t)j * d + e]));
    out[(size_t)row * d + e] = fx_sat16(fx_rnd(bk.total(), 8));
}

// ---------------------------------------------------------------------
// SOFTMAX (stream_softmax_rows, kernel/compute_stream.cpp:388-478): row
// maximum from fm(-128), e = exp(x - max) in Q8.8, inverse of the Q8.8
// sum by cu_recip_approx, out = fm(e * inv).  One wavefront per row.
// ---------------------------------------------------------------------
__global__ __launch_bounds__(64) void op_softmax_kernel(const int16_t* __restrict__ x,
                                                        uint32_t n,
                                                        const int16_t* __restrict__ exp8,
                                                        int16_t* __restrict__ out) {
    const uint32_t row = blockIdx.x, c = threadIdx.x;
    const bool valid = c < n;
    const int32_t v = valid ? x[(size_t)row * 64 + c] : INT16_MIN;
    int32_t m = v;
    for (int off = 32; off > 0; off >>= 1) m = max(m, __shfl_xor(m, off, 64));
    const int32_t e = valid ? exp_diff(v - m, exp8) : 0;
    // the Q16.16 sum of the Q8.8 values (<= 64 * 256: no saturation)
    // narrowed back to Q8.8 is their exact sum
    int32_t s = e;
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    const int32_t inv = fx_recip(s);
    if (valid) out[(size_t)row * n + c] = fx_sat16(fx_rnd((int64_t)e * inv, 8));
}

// ---------------------------------------------------------------------
// Flash attention over the cache pages, one workgroup per (KV head,
// token, query head), tiles of 64 positions anchored at position 0 in
// order (the online recurrence of compute_cc8_flash_probabilities_one_core
// / compute_cc8_prefill_flash_probabilities_one_core, ctrl:4743-4896,
// :4998-5150).  Per tile: the four wavefronts each sum a quarter of the
// head dimension for every position; wavefront 0 finishes the scores, the
// maximum, the probabilities and the running sum; lanes < head_dim
// rescale their accumulator and add the tile's PV value.
// ---------------------------------------------------------------------
__global__ __launch_bounds__(256) void op_flash_kernel(OpFlashArgs a) {
    const uint32_t G = a.group, D = a.head_dim, T = a.tokens;
    const uint32_t wg = blockIdx.x;  // (h * T + t) * G + g
    const uint32_t t = (wg / G) % T, h = wg / (G * T);
    const uint32_t n = a.pos0 + t + 1;
    const size_t head_off = (size_t)h * a.tiles * 64 * D;
    const int16_t* kh = a.kcache + head_off;
    const int16_t* vh = a.vcache + head_off;
    const int16_t* table = a.legacy ? a.exp8 : a.exp14;
    const int sh = a.legacy ? 8 : 2;  // probability -> Q16.16

    __shared__ int16_t qs[128];
    __shared__ int32_t red[4][64][4];
    __shared__ int32_t prob[64];
    __shared__ int32_t old_s, sum_s;
    const uint32_t tid = threadIdx.x;
    if (tid < D) qs[tid] = a.q[(size_t)wg * D + tid];
    __syncthreads();

    const uint32_t p = tid & 63, part = tid >> 6, per = D / 4;
    int32_t acc = 0;                  // lanes < D: element tid
    int32_t m = INT16_MIN, sum = 0;   // wavefront 0
    for (uint32_t tb = 0; tb < n; tb += 64) {
        const uint32_t tl = n - tb < 64 ? n - tb : 64;
        const size_t page = (size_t)(tb / 64) * 64 * D;
        // partial bank sums of position p over slots [part * per, +per):
        // at most 8 terms of a bank, |sum| <= 2^29
        int32_t b[4] = {0, 0, 0, 0};
        if (p < tl) {
            const int16_t* kr = kh + page + (size_t)p * D;
            for (uint32_t s = part * per; s < (part + 1) * per; s += 4) {
                const uint2 w = *(const uint2*)(kr + s);
                const int32_t kv[4] = {(int16_t)(w.x & 0xffff), (int16_t)(w.x >> 16),
                                       (int16_t)(w.y & 0xffff), (int16_t)(w.y >> 16)};
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const uint32_t e = slot_elem(s + u);
                    const int32_t term = wt_term(qs[e], kv[u]);
                    const uint32_t j = e & 3u;
                    b[0] += j == 0 ? term : 0;
                    b[1] += j == 1 ? term : 0;
                    b[2] += j == 2 ? term : 0;
                    b[3] += j == 3 ? term : 0;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) red[part][p][j] = b[j];
        __syncthreads();
        if (tid < 64) {
            int32_t sc = INT32_MIN;
            if (p < tl) {
                Banks bk;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    bk.b[j] = (int64_t)red[0][p][j] + red[1][p][j] + red[2][p][j] + red[3][p][j];
                sc = qk_score(bk.total(), a.qk_scale);
            }
            int32_t mx = sc;
            for (int off = 32; off > 0; off >>= 1) mx = max(mx, __shfl_xor(mx, off, 64));
            const int32_t m_new = max(m, mx);
            const int32_t old = exp_diff(m - m_new, table);
            const int32_t pr = p < tl ? exp_diff(sc - m_new, table) : 0;
            prob[p] = pr;
            int32_t ts = pr;  // <= 64 * 16384
            for (int off = 32; off > 0; off >>= 1) ts += __shfl_xor(ts, off, 64);
            const int64_t old_acc = (int64_t)old << sh;
            sum = fx_sat32(fx_rnd((int64_t)sum * old_acc + (((int64_t)ts << sh) << 16), 16));
            m = m_new;
            if (tid == 0) {
                old_s = (int32_t)old_acc;
                sum_s = sum;
            }
        }
        __syncthreads();
        if (tid < D) {
            acc = fx_sat32(fx_rnd((int64_t)acc * old_s, 16));
            // V page row tid: positions in the bank-paired order; slots past
            // the tile hold probability 0 and add nothing
            const int16_t* vr = vh + page + (size_t)tid * 64;
            int32_t c[4] = {0, 0, 0, 0};  // at most 16 terms each, |sum| <= 2^30
            for (uint32_t s = 0; s < 64; s += 4) {
                const uint2 w = *(const uint2*)(vr + s);
                const int32_t vv[4] = {(int16_t)(w.x & 0xffff), (int16_t)(w.x >> 16),
                                       (int16_t)(w.y & 0xffff), (int16_t)(w.y >> 16)};
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const uint32_t pos = slot_elem(s + u);
                    const int32_t term = wt_term(prob[pos], vv[u]);
                    const uint32_t j = pos & 3u;
                    c[0] += j == 0 ? term : 0;
                    c[1] += j == 1 ? term : 0;
                    c[2] += j == 2 ? term : 0;
                    c[3] += j == 3 ? term : 0;
                }
            }
            Banks bk;
#pragma unroll
            for (int j = 0; j < 4; j++) bk.b[j] = c[j];
            int32_t total = bk.total();
            if (!a.legacy) total = fx_sat32(fx_rnd((int64_t)total * 1024, 16));  // x fm(1/64)
            const int32_t tv = fx_sat16(fx_rnd(total, 8));
            acc = fx_sat32((int64_t)acc + (int64_t)tv * 256);
        }
    }
    if (tid < D)
        a.out[(size_t)wg * D + tid] =
            fx_sat16(fx_rnd((int64_t)acc * fx_inv_sum(sum_s), 16));
}

__global__ __launch_bounds__(128) void op_kv_append_kernel(int16_t* __restrict__ kc,
                                                           int16_t* __restrict__ vc,
                                                           uint32_t tiles, uint32_t d,
                                                           uint32_t pos,
                                                           const int16_t* __restrict__ k,
                                                           const int16_t* __restrict__ v) {
    const uint32_t h = blockIdx.x, e = threadIdx.x;
    if (e >= d) return;
    const uint32_t slot = pos % 64;
    const size_t page = ((size_t)h * tiles + pos / 64) * 64 * d;
    kc[page + (size_t)slot * d + paired(e)] = k[(size_t)h * d + e];
    vc[page + (size_t)e * 64 + paired(slot)] = v[(size_t)h * d + e];
}

// SILU_MUL (stream_silu_mul, compute_stream.cpp:123-147 / golden_silu_mul
// host:3199-3217) and RESIDUAL_ADD (stream_add_residual :205-225).
__global__ __launch_bounds__(256) void op_silu_mul_kernel(const int16_t* __restrict__ g,
                                                          const int16_t* __restrict__ u,
                                                          uint32_t n,
                                                          const int16_t* __restrict__ exp8,
                                                          int16_t* __restrict__ out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = fx_sat16(fx_rnd((int64_t)fx_silu(g[i], exp8) * u[i], 8));
}

__global__ __launch_bounds__(256) void op_residual_kernel(const int16_t* __restrict__ x,
                                                          const int16_t* __restrict__ y,
                                                          uint32_t n, int16_t* __restrict__ out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = fx_sat16((int32_t)x[i] + y[i]);
}

}  // namespace

hipError_t launch_op_qk(const int16_t* q, const int16_t* k, uint32_t kv_heads,
                        uint32_t group, uint32_t head_dim, uint32_t tile_len,
                        int32_t qk_scale, int16_t* out, hipStream_t st) {
    if (kv_heads * group == 0 || tile_len == 0 || tile_len > 64) return hipErrorInvalidValue;
    op_qk_kernel<<<kv_heads * group, 64, 0, st>>>(q, k, group, head_dim, tile_len, qk_scale,
                                                 out);
    return hipGetLastError();
}

hipError_t launch_op_pv(const int16_t* p, const int16_t* v, uint32_t kv_heads,
                        uint32_t group, uint32_t head_dim, uint32_t tile_len,
                        int16_t* out, hipStream_t st) {
    if (kv_heads * group == 0 || head_dim > 128 || tile_len == 0 || tile_len > 64)
        return hipErrorInvalidValue;
    op_pv_kernel<<<kv_heads * group, 128, 0, st>>>(p, v, group, head_dim, tile_len, out);
    return hipGetLastError();
}

hipError_t launch_op_softmax(const int16_t* x, uint32_t rows, uint32_t tile_len,
                             const int16_t* exp8, int16_t* out, hipStream_t st) {
    if (rows == 0 || tile_len == 0 || tile_len > 64) return hipErrorInvalidValue;
    op_softmax_kernel<<<rows, 64, 0, st>>>(x, tile_len, exp8, out);
    return hipGetLastError();
}

hipError_t launch_op_silu_mul(const int16_t* gate, const int16_t* up, uint32_t n,
                              const int16_t* exp8, int16_t* out, hipStream_t st) {
    if (n == 0) return hipSuccess;
    op_silu_mul_kernel<<<(n + 255) / 256, 256, 0, st>>>(gate, up, n, exp8, out);
    return hipGetLastError();
}

hipError_t launch_op_residual(const int16_t* a, const int16_t* b, uint32_t n,
                              int16_t* out, hipStream_t st) {
    if (n == 0) return hipSuccess;
    op_residual_kernel<<<(n + 255) / 256, 256, 0, st>>>(a, b, n, out);
    return hipGetLastError();
}

hipError_t launch_op_flash(const OpFlashArgs& a, hipStream_t st) {
    // qs holds one query row; the slot loops read whole 4-slot words
    if (a.kv_heads * a.tokens * a.group == 0 || a.head_dim == 0 || a.head_dim > 128 ||
        a.head_dim % 16 != 0 || a.pos0 + a.tokens > a.tiles * 64)
        return hipErrorInvalidValue;
    op_flash_kernel<<<a.kv_heads * a.tokens * a.group, 256, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_op_kv_append(int16_t* kcache, int16_t* vcache, uint32_t tiles,
                               uint32_t kv_heads, uint32_t head_dim, uint32_t pos,
                               const int16_t* k, const int16_t* v, hipStream_t st) {
    if (kv_heads == 0 || head_dim > 128 || pos >= tiles * 64) return hipErrorInvalidValue;
    op_kv_append_kernel<<<kv_heads, 128, 0, st>>>(kcache, vcache, tiles, head_dim, pos, k, v);
    return hipGetLastError();
}

}  // namespace llm
