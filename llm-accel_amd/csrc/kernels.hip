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

// Constant-gain RMSNorm: one thread per element.
__global__ __launch_bounds__(256) void rmsnorm_const_kernel(
    const int16_t* __restrict__ x, uint32_t ldx,
    const int16_t* __restrict__ gamma, uint32_t cols, int16_t* __restrict__ y,
    uint32_t ldy, uint32_t total, int32_t gain) {
    const uint32_t idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const uint32_t r = idx / cols, c = idx % cols;
    y[(size_t)r * ldy + c] =
        fx_sat16(fx_rnd((int64_t)x[(size_t)r * ldx + c] * gain * gamma[c], 16));
}

// ---------------------------------------------------------------------
// Projection: Y[r][n] = narrow(sum_k X[r][k] * W[n][k]) for r < rows.
// Workgroup = 4 wavefronts on one 4-row block; the wavefronts split the
// k-steps, lane (i, j) = (lane / 16, lane % 16) owns row i and columns
// 8j..8j+7 of each step.  Partial sums stay in int32 for L steps (8L
// products, bounded by the host), then widen to int64; the 16 lanes of a
// row and the 4 wavefronts reduce in int64.
// ---------------------------------------------------------------------
// Eight inputs normalised with a constant gain: rnd(x * gain * gamma, 16),
// zero at columns >= cols.
// |x * gain * gamma| < 2^15 * 2^13 * 2^15, so the product shifted right by 16
// fits 32 bits before the saturation.
__device__ __forceinline__ int32_t norm1(int32_t x, int32_t gg) {
    const int32_t y = (int32_t)(((int64_t)x * gg + 32768) >> 16);
    return y < -32768 ? -32768 : (y > 32767 ? 32767 : y);
}
// Eight inputs normalised with a constant gain: rnd(x * gain * gamma, 16);
// columns >= cols have gamma 0 (the caller zeroes g there).
__device__ __forceinline__ uint4 norm8(uint4 x, uint4 g, int32_t gain) {
    uint32_t w[4] = {x.x, x.y, x.z, x.w};
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int32_t lo = norm1((int16_t)(w[i] & 0xffff), gain * (int16_t)(gw[i] & 0xffff));
        const int32_t hi = norm1((int16_t)(w[i] >> 16), gain * (int16_t)(gw[i] >> 16));
        w[i] = (uint32_t)(uint16_t)lo | ((uint32_t)hi << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

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
            if (EPI == EPI_STORE_NORM_IN) {
                const uint32_t k0 = s * 128 + j * 8;
                const uint4 gv = k0 < a.in_cols ? *(const uint4*)(a.in_gamma + k0)
                                                : make_uint4(0, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < RT; r++)
                    xv[r] = norm8(xv[r], gv, a.in_gain);
            }
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
                if (a.norm_out)
                    a.norm_out[(size_t)r * a.ldn + n] = fx_sat16(fx_rnd(
                        (int64_t)y * a.norm_gain * a.norm_gamma[n], 16));
                if (a.final_out)
                    a.final_out[(size_t)r * a.ldn + n] = fx_sat16(fx_rnd(
                        (int64_t)y * a.norm_gain * a.final_gamma[n], 16));
            } else if (EPI == EPI_SILU) {
                int16_t up = fx_narrow_projection(tot[NM - 1]);
                int16_t sg = fx_silu(y, a.exp8);
                y = fx_sat16(fx_rnd((int64_t)sg * up, 8));
            }
            a.out[(size_t)r * a.ldo + n] = y;
        }
    }
    if (EPI == EPI_RESID && a.final_out && t < 32) {
        const int ii = t >> 3, r = t & 7;
        const uint32_t n = b * 4 + ii;
        if ((uint32_t)r >= a.rows && n < a.n)
            a.final_out[(size_t)r * a.ldn + n] = a.res[(size_t)r * a.ldr + n];
    }
}

// ---------------------------------------------------------------------
// Plain copy (calibration reference for HBM counters).
// ---------------------------------------------------------------------
__global__ __launch_bounds__(256) void copy_kernel(const uint4* __restrict__ src,
                                                   uint4* __restrict__ dst,
                                                   size_t n16) {
    for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n16;
         i += (size_t)gridDim.x * 256)
        dst[i] = src[i];
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
    case EPI_STORE_NORM_IN: return launch_proj_epi<EPI_STORE_NORM_IN>(a, L, blocks, st);
    default: return launch_proj_epi<EPI_SILU>(a, L, blocks, st);
    }
}

hipError_t launch_copy(const uint4* src, uint4* dst, size_t n16,
                       hipStream_t st) {
    copy_kernel<<<2048, 256, 0, st>>>(src, dst, n16);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const int16_t* x, uint32_t ldx, const int16_t* gamma,
                          uint32_t cols, int16_t* y, uint32_t ldy, uint32_t rows,
                          int32_t const_gain, hipStream_t st) {
    if (const_gain > 0) {
        const uint32_t total = rows * cols;
        rmsnorm_const_kernel<<<(total + 255) / 256, 256, 0, st>>>(
            x, ldx, gamma, cols, y, ldy, total, const_gain);
    } else {
        rmsnorm_kernel<<<rows, 256, 0, st>>>(x, ldx, gamma, cols, y, ldy);
    }
    return hipGetLastError();
}

}  // namespace llm
