// kernels.hip -- CDNA4 (gfx950) kernels of the resident decoder-layer path.
//
// Every kernel is exact integer arithmetic; rounding and saturation follow
// the reference's ap_fixed chain (see fixed_point.h).  Layouts in HBM:
//
//   weights  "tile4x128": matrix [N][K] is stored as row blocks of 4 output
//            rows; within a block, k-steps of 128 columns; within a step,
//            [4 rows][16 lanes][8 columns].  One wavefront load of 16 B per
//            lane reads one contiguous 1 KiB step of a block.  N is padded
//            to a multiple of 4 and K to a multiple of 128 with zeros.
//   KV cache pages of 64 positions (one attention tile) x head_dim int16,
//            addressed through a page table [layer][kv_head][tile].
#include "kernels.h"

#include "fixed_point.h"

namespace llm {

typedef short s16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int32_t dot2(uint32_t a, uint32_t b, int32_t c) {
    // v_dot2_i32_i16, no clamp: exact while |c + a.lo*b.lo + a.hi*b.hi| <
    // 2^31, which the host guarantees through the widening interval L.
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s16x2, a),
                                  __builtin_bit_cast(s16x2, b), c, false);
}

__device__ __forceinline__ int64_t dot2_wide(uint32_t a, uint32_t b) {
    int32_t a0 = (int16_t)(a & 0xffff), a1 = (int16_t)(a >> 16);
    int32_t b0 = (int16_t)(b & 0xffff), b1 = (int16_t)(b >> 16);
    return (int64_t)(a0 * b0) + (int64_t)(a1 * b1);
}

// ---------------------------------------------------------------------
// RMSNorm: one workgroup per row.
// ---------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_kernel(
    const int16_t* __restrict__ x, uint32_t ldx,
    const int16_t* __restrict__ gamma, uint32_t cols,
    int16_t* __restrict__ y, uint32_t ldy) {
    const int16_t* xr = x + (size_t)blockIdx.x * ldx;
    int64_t s = 0;
    for (uint32_t c = threadIdx.x; c < cols; c += 256)
        s += (int32_t)xr[c] * xr[c];
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    __shared__ int64_t part[4];
    __shared__ int32_t gain;
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0)
        gain = fx_rmsnorm_gain(part[0] + part[1] + part[2] + part[3], cols);
    __syncthreads();
    const int64_t g = gain;
    int16_t* yr = y + (size_t)blockIdx.x * ldy;
    for (uint32_t c = threadIdx.x; c < cols; c += 256)
        yr[c] = fx_sat16(fx_rnd((int64_t)xr[c] * g * gamma[c], 16));
}

// ---------------------------------------------------------------------
// Projection: Y[r][n] = narrow(sum_k X[r][k] * W[n][k]) for r < rows.
// Workgroup = 4 wavefronts on one 4-row block; the wavefronts split the
// k-steps, lane (i, j) = (lane / 16, lane % 16) owns row i and columns
// 8j..8j+7 of each step.  Partial sums stay in int32 for L steps (8L
// products, bounded by the host), then widen to int64; the 16 lanes of a
// row and the 4 wavefronts reduce in int64.
// ---------------------------------------------------------------------
template <int RT, int L, int EPI>
__global__ __launch_bounds__(256) void proj_kernel(ProjArgs a) {
    constexpr int NM = EPI == EPI_SILU ? 2 : 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane >> 4, j = lane & 15;
    const uint32_t b = blockIdx.x;
    const uint32_t S = a.steps;
    const uint32_t s0 = wave * S / 4, s1 = (wave + 1) * S / 4;

    int64_t acc[NM][RT];
    int32_t part[NM][RT];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < RT; r++) acc[m][r] = 0, part[m][r] = 0;

    const int16_t* wp0 = a.w0 + ((size_t)(b * S + s0) * 4 + i) * 128 + j * 8;
    const int16_t* wp1 = NM == 2
        ? a.w1 + ((size_t)(b * S + s0) * 4 + i) * 128 + j * 8 : nullptr;
    const int16_t* xp = a.x + (size_t)s0 * 128 + j * 8;

    for (uint32_t s = s0; s < s1;) {
        const uint32_t lim = (L == 0) ? s1 : (s + L < s1 ? s + L : s1);
#pragma unroll 2
        for (; s < lim; s++) {
            uint4 wv[NM];
            wv[0] = *(const uint4*)(wp0);
            wp0 += 512;
            if (NM == 2) {
                wv[NM - 1] = *(const uint4*)(wp1);
                wp1 += 512;
            }
            uint4 xv[RT];
#pragma unroll
            for (int r = 0; r < RT; r++)
                xv[r] = *(const uint4*)(xp + (size_t)r * a.ldx);
            xp += 128;
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    if (L == 0) {
                        acc[m][r] += dot2_wide(wv[m].x, xv[r].x) +
                                     dot2_wide(wv[m].y, xv[r].y) +
                                     dot2_wide(wv[m].z, xv[r].z) +
                                     dot2_wide(wv[m].w, xv[r].w);
                    } else {
                        int32_t p = part[m][r];
                        p = dot2(wv[m].x, xv[r].x, p);
                        p = dot2(wv[m].y, xv[r].y, p);
                        p = dot2(wv[m].z, xv[r].z, p);
                        p = dot2(wv[m].w, xv[r].w, p);
                        part[m][r] = p;
                    }
                }
        }
        if (L != 0) {
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    acc[m][r] += part[m][r];
                    part[m][r] = 0;
                }
        }
    }

#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int off = 8; off > 0; off >>= 1)
                acc[m][r] += __shfl_xor(acc[m][r], off, 64);

    __shared__ int64_t red[4][NM][4][RT];
    if (j == 0) {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < RT; r++) red[wave][m][i][r] = acc[m][r];
    }
    __syncthreads();
    const int t = threadIdx.x;
    if (t < 4 * RT) {
        const int ii = t / RT, r = t % RT;
        const uint32_t n = b * 4 + ii;
        if ((uint32_t)r < a.rows && n < a.n) {
            int64_t tot[NM];
#pragma unroll
            for (int m = 0; m < NM; m++)
                tot[m] = red[0][m][ii][r] + red[1][m][ii][r] +
                         red[2][m][ii][r] + red[3][m][ii][r];
            int16_t y = fx_narrow_projection(tot[0]);
            if (EPI == EPI_RESID) {
                y = fx_sat16((int32_t)y + a.res[(size_t)r * a.ldr + n]);
            } else if (EPI == EPI_SILU) {
                int16_t up = fx_narrow_projection(tot[NM - 1]);
                int16_t sg = fx_silu(y, a.exp8);
                y = fx_sat16(fx_rnd((int64_t)sg * up, 8));
            }
            a.out[(size_t)r * a.ldo + n] = y;
        }
    }
}

// ---------------------------------------------------------------------
// RoPE on Q and K, append K (rotated) and V to the paged cache.  One
// workgroup per active row t at absolute position pos0 + t.
// ---------------------------------------------------------------------
__global__ __launch_bounds__(256) void rope_append_kernel(RopeArgs a) {
    const uint32_t t = blockIdx.x, pos = a.pos0 + t;
    const uint32_t d = a.head_dim, half = d / 2;
    const int16_t* rope = a.rope + (size_t)pos * d;
    const int16_t* row = a.qkv + (size_t)t * a.ldqkv;
    const uint32_t tile = pos / 64, slot = pos % 64;
    for (uint32_t idx = threadIdx.x; idx < a.num_heads * half; idx += 256) {
        const uint32_t h = idx / half, e = idx % half;
        const int32_t x0 = row[h * d + e], x1 = row[h * d + half + e];
        const int32_t c = rope[e], s = rope[half + e];
        int16_t* qo = a.q + (size_t)t * a.ldq + h * d;
        qo[e] = fx_sat16(fx_rnd((int64_t)x0 * c - (int64_t)x1 * s, 8));
        qo[half + e] = fx_sat16(fx_rnd((int64_t)x1 * c + (int64_t)x0 * s, 8));
    }
    const int16_t* krow = row + a.num_heads * d;
    const int16_t* vrow = krow + a.num_kv_heads * d;
    for (uint32_t idx = threadIdx.x; idx < a.num_kv_heads * half; idx += 256) {
        const uint32_t h = idx / half, e = idx % half;
        const int32_t x0 = krow[h * d + e], x1 = krow[h * d + half + e];
        const int32_t c = rope[e], s = rope[half + e];
        const int32_t page = a.page_table[h * a.tiles + tile];
        int16_t* ko = a.kcache + ((size_t)page * 64 + slot) * d;
        ko[e] = fx_sat16(fx_rnd((int64_t)x0 * c - (int64_t)x1 * s, 8));
        ko[half + e] = fx_sat16(fx_rnd((int64_t)x1 * c + (int64_t)x0 * s, 8));
    }
    for (uint32_t idx = threadIdx.x; idx < a.num_kv_heads * d; idx += 256) {
        const uint32_t h = idx / d, e = idx % d;
        const int32_t page = a.page_table[h * a.tiles + tile];
        a.vcache[((size_t)page * 64 + slot) * d + e] = vrow[h * d + e];
    }
}

// ---------------------------------------------------------------------
// Tiled online-softmax attention, one workgroup per (active row, KV head):
// the GQA group's G query heads share every K/V tile staged in LDS.
// Arithmetic: golden_tiled_flash_attention_q2_14 (raw payload), host
// :3609-3738 == controller :5491-5765.
// ---------------------------------------------------------------------
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a) {
    constexpr int MAXG = 16, MAXD = 128, TILE = 64;
    const uint32_t t = blockIdx.x, h = blockIdx.y;
    const uint32_t G = a.group, d = a.head_dim, Gd = G * d;
    const uint32_t n = a.pos0 + t + 1;
    __shared__ int16_t qs[MAXG * MAXD];
    __shared__ int16_t ks[TILE * MAXD];
    __shared__ int16_t vs[TILE * MAXD];
    __shared__ int16_t sc[MAXG * TILE];
    __shared__ int16_t pr[MAXG * TILE];
    __shared__ int16_t mx[MAXG];
    __shared__ int32_t sm[MAXG];
    __shared__ int32_t old[MAXG];

    const int16_t* qsrc = a.q + (size_t)t * a.ldq + (size_t)h * Gd;
    for (uint32_t idx = threadIdx.x; idx < Gd; idx += 256) qs[idx] = qsrc[idx];
    if (threadIdx.x < G) {
        mx[threadIdx.x] = INT16_MIN;  // fm(-128)
        sm[threadIdx.x] = 0;
    }
    int32_t acc[MAXG * MAXD / 256];
#pragma unroll
    for (int k = 0; k < MAXG * MAXD / 256; k++) acc[k] = 0;
    const int64_t scale = (int64_t)a.qk_scale << 8;  // accum(fm(1/sqrt d))

    for (uint32_t tb = 0, tile = 0; tb < n; tb += TILE, tile++) {
        const uint32_t tl = n - tb < TILE ? n - tb : TILE;
        const int32_t page = a.page_table[h * a.tiles + tile];
        const int16_t* kp = a.kcache + (size_t)page * TILE * d;
        const int16_t* vp = a.vcache + (size_t)page * TILE * d;
        __syncthreads();
        for (uint32_t idx = threadIdx.x; idx < tl * d; idx += 256) {
            ks[idx] = kp[idx];
            vs[idx] = vp[idx];
        }
        __syncthreads();
        // QK scores: four k-mod-4 banks of AP_RND(Q8.8 x Q4.12) products.
        // d <= 128 gives <= 32 terms per bank, so only a bank's final sum
        // can leave the Q16.16 range; clamping the exact sum is therefore
        // the same as saturating every accumulation.
        for (uint32_t idx = threadIdx.x; idx < G * TILE; idx += 256) {
            const uint32_t g = idx / TILE, p = idx % TILE;
            if (p >= tl) continue;
            int64_t bank[4] = {0, 0, 0, 0};
            for (uint32_t e = 0; e < d; e++) {
                int32_t w = fx_fm_to_wt(ks[p * d + e]);
                bank[e & 3] += fx_rnd((int64_t)qs[g * d + e] * w, 4);
            }
            int64_t total = (int64_t)fx_sat32(bank[0]) + fx_sat32(bank[1]) +
                            fx_sat32(bank[2]) + fx_sat32(bank[3]);
            int32_t tq = fx_sat32(total);
            tq = fx_sat32(fx_rnd((int64_t)tq * scale, 16));
            sc[g * TILE + p] = fx_sat16(fx_rnd(tq, 8));
        }
        __syncthreads();
        // Online softmax state per query head (Q2.14 probabilities).
        if (threadIdx.x < G) {
            const uint32_t g = threadIdx.x;
            int32_t m = mx[g];
            for (uint32_t p = 0; p < tl; p++)
                m = sc[g * TILE + p] > m ? sc[g * TILE + p] : m;
            int32_t diff = fx_sat16((int32_t)mx[g] - m);
            diff = diff < -2048 ? -2048 : diff;
            const int64_t o = (int64_t)a.exp14[diff + 2048] << 2;
            int64_t tsum = 0;
            for (uint32_t p = 0; p < tl; p++) {
                int32_t x = fx_sat16((int32_t)sc[g * TILE + p] - m);
                x = x < -2048 ? -2048 : x;
                int16_t pv = a.exp14[x + 2048];
                pr[g * TILE + p] = pv;
                tsum += (int64_t)pv << 2;
            }
            sm[g] = fx_sat32(fx_rnd((int64_t)sm[g] * o + (tsum << 16), 16));
            mx[g] = (int16_t)m;
            old[g] = (int32_t)o;
        }
        __syncthreads();
        // Rescale accumulators, then add this tile's PV (payload = Q2.14
        // bits read as Q8.8, x fm(1/64), narrowed to Q8.8 per tile).
#pragma unroll
        for (int k = 0; k < MAXG * MAXD / 256; k++) {
            const uint32_t idx = threadIdx.x + 256 * k;
            if (idx >= Gd) break;
            const uint32_t g = idx / d, e = idx % d;
            int32_t av = fx_sat32(fx_rnd((int64_t)acc[k] * old[g], 16));
            int64_t bank[4] = {0, 0, 0, 0};
            for (uint32_t p = 0; p < tl; p++) {
                int32_t w = fx_fm_to_wt(vs[p * d + e]);
                bank[p & 3] += fx_rnd((int64_t)pr[g * TILE + p] * w, 4);
            }
            int32_t tot = fx_sat32((int64_t)fx_sat32(bank[0]) + fx_sat32(bank[1]) +
                                   fx_sat32(bank[2]) + fx_sat32(bank[3]));
            tot = fx_sat32(fx_rnd((int64_t)tot * 1024, 16));
            const int32_t tv = fx_sat16(fx_rnd(tot, 8));
            acc[k] = fx_sat32((int64_t)av + ((int64_t)tv << 8));
        }
    }
    __syncthreads();
    int16_t* dst = a.out + (size_t)t * a.ldo + (size_t)h * Gd;
#pragma unroll
    for (int k = 0; k < MAXG * MAXD / 256; k++) {
        const uint32_t idx = threadIdx.x + 256 * k;
        if (idx >= Gd) break;
        const uint32_t g = idx / d;
        const int64_t inv = fx_inv_sum(sm[g]);
        dst[idx] = fx_sat16(fx_rnd((int64_t)acc[k] * inv, 16));
    }
}

// ---------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------
template <int RT, int EPI>
static hipError_t launch_proj_rt(const ProjArgs& a, int L, uint32_t blocks,
                                 hipStream_t st) {
    switch (L) {
    case 0: proj_kernel<RT, 0, EPI><<<blocks, 256, 0, st>>>(a); break;
    case 1: proj_kernel<RT, 1, EPI><<<blocks, 256, 0, st>>>(a); break;
    case 4: proj_kernel<RT, 4, EPI><<<blocks, 256, 0, st>>>(a); break;
    case 8: proj_kernel<RT, 8, EPI><<<blocks, 256, 0, st>>>(a); break;
    default: proj_kernel<RT, 16, EPI><<<blocks, 256, 0, st>>>(a); break;
    }
    return hipGetLastError();
}

template <int EPI>
static hipError_t launch_proj_epi(const ProjArgs& a, int L, uint32_t blocks,
                                  hipStream_t st) {
    if (a.rows <= 1) return launch_proj_rt<1, EPI>(a, L, blocks, st);
    if (a.rows <= 2) return launch_proj_rt<2, EPI>(a, L, blocks, st);
    if (a.rows <= 4) return launch_proj_rt<4, EPI>(a, L, blocks, st);
    return launch_proj_rt<8, EPI>(a, L, blocks, st);
}

hipError_t launch_proj(const ProjArgs& a, int epi, int L, uint32_t blocks,
                       hipStream_t st) {
    switch (epi) {
    case EPI_STORE: return launch_proj_epi<EPI_STORE>(a, L, blocks, st);
    case EPI_RESID: return launch_proj_epi<EPI_RESID>(a, L, blocks, st);
    default: return launch_proj_epi<EPI_SILU>(a, L, blocks, st);
    }
}

hipError_t launch_rmsnorm(const int16_t* x, uint32_t ldx, const int16_t* gamma,
                          uint32_t cols, int16_t* y, uint32_t ldy, uint32_t rows,
                          hipStream_t st) {
    rmsnorm_kernel<<<rows, 256, 0, st>>>(x, ldx, gamma, cols, y, ldy);
    return hipGetLastError();
}

hipError_t launch_rope_append(const RopeArgs& a, uint32_t rows, hipStream_t st) {
    rope_append_kernel<<<rows, 256, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, uint32_t rows, uint32_t kv_heads,
                            hipStream_t st) {
    attention_kernel<<<dim3(rows, kv_heads), 256, 0, st>>>(a);
    return hipGetLastError();
}

}  // namespace llm
