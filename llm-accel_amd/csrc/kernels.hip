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

#include "coherent.h"
#include "fixed_point.h"
#include "proj_common.h"

// Launch shapes (measured choices; overridable at build time for sweeps).
#ifndef LLM_PROJ_WPB
#define LLM_PROJ_WPB 4      // wavefronts per 4-row block (VALU kernel)
#endif
#ifndef LLM_P12_WPB
#define LLM_P12_WPB 8       // the same, 12-bit kernel, one matrix (decode QKV: 748 vs 746 tok/s at 4)
#endif
#ifndef LLM_PROJ_WPB_SILU
#define LLM_PROJ_WPB_SILU 8 // the same for gate|up (twice the loads per step)
#endif
#ifndef LLM_PROJ_UNROLL
#define LLM_PROJ_UNROLL 2   // k-steps whose loads are issued together
#endif
#ifndef LLM_PROJ_UNROLL_LONG
#define LLM_PROJ_UNROLL_LONG 2  // the same for 16-wavefront blocks
#endif
#ifndef LLM_PROJ_LONG_STEPS
#define LLM_PROJ_LONG_STEPS 48  // k-steps from which 1-2 row blocks use 16 waves
#endif
#ifndef LLM_MF_KS
#define LLM_MF_KS 8         // matrix-core kernel: wavefronts per workgroup
#endif
#ifndef LLM_MF_WG_TARGET
#define LLM_MF_WG_TARGET 128  // matrix-core kernel: split K below this many workgroups
#endif
#ifndef LLM_MF_QMAX
#define LLM_MF_QMAX 12      // matrix-core kernel: K chunks per wavefront (<= 12)
#endif
#ifndef LLM_MF_PD1
#define LLM_MF_PD1 4        // K chunks of loads in flight per wavefront, one matrix
#endif
#ifndef LLM_MF_PD2
#define LLM_MF_PD2 2        // the same for gate|up (two matrices)
#endif
#ifndef LLM_P12_MAX_ROWS
#define LLM_P12_MAX_ROWS 2  // 12-bit VALU kernel: blocks of at most this many rows (1 or 2)
#endif
#ifndef LLM_MF12_KS
#define LLM_MF12_KS 8       // 12-bit matrix-core kernel: wavefronts per workgroup
#endif
#ifndef LLM_MF12_MIN_STEPS
#define LLM_MF12_MIN_STEPS 4  // 12-bit matrix-core kernel: fewer wavefronts below this many steps each
#endif
#ifndef LLM_MF12_WG_TARGET
#define LLM_MF12_WG_TARGET 128  // 12-bit matrix-core kernel: split K below this many workgroups
#endif
#ifndef LLM_MF12_LONG_STEPS
#define LLM_MF12_LONG_STEPS 64  // 12-bit matrix-core kernel: one matrix with at least this many
#endif                          // k-steps (down) takes 16 wavefronts and >= 256 workgroups
#ifndef LLM_MF12_PD1
#define LLM_MF12_PD1 2      // 12-bit matrix-core kernel: k-steps of loads in flight, one matrix
#endif
#ifndef LLM_MF12_PD2
#define LLM_MF12_PD2 1      // the same for gate|up
#endif

namespace llm {

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
// SPW > 0: every wavefront has at most SPW k-steps and issues all of their
// loads (weights, activations, gammas) before the first product; loads past
// its last step repeat that step (in bounds, products of zero).  SPW = 0:
// a loop over the steps, LLM_PROJ_UNROLL steps of loads at a time.
template <int RT, int L, int EPI, int WPB, int SPW>
__global__ __launch_bounds__(64 * WPB) void proj_kernel(ProjArgs a) {
    constexpr int NM = EPI == EPI_SILU ? 2 : 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane >> 4, j = lane & 15;
    const uint32_t b = blockIdx.x;
    // epilogue thread t < 4 RT: output row et % RT of block row et / RT
    const int et = threadIdx.x;
    const uint32_t en = b * 4 + et / RT, er = et % RT;
    const bool eout = et < 4 * RT && er < a.rows && en < a.n;
    EpiIn ei{0, 0, 0};
    if (eout) ei = epi_fetch<EPI>(a, er, en);
    // rows >= rows of the final-norm pair copy the residual rows
    const uint32_t fn = b * 4 + (et >> 3), fr = et & 7;
    const bool efill = EPI == EPI_RESID && a.final_out && et < 32 && fr >= a.rows && fn < a.n;
    int16_t fill = 0;
    if (efill) fill = a.res[(size_t)fr * a.ldr + fn];
    const uint32_t S = a.steps;
    const uint32_t s0 = wave * S / WPB, s1 = (wave + 1) * S / WPB;

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

    if constexpr (SPW > 0) {
        const uint32_t cnt = s1 - s0;  // <= SPW (the launcher's choice)
        uint4 wv[SPW][NM], xv[SPW][RT];
        // EPI_STORE_NORM_IN: lane l loads and normalises columns 2l, 2l + 1
        // of each step and row (once per wavefront, not once per row of the
        // block), shared through LDS
        constexpr bool NIN = EPI == EPI_STORE_NORM_IN;
        uint32_t x2[SPW][RT], g2[SPW];
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const uint32_t du = cnt == 0 ? 0 : ((uint32_t)u < cnt ? u : cnt - 1);
            wv[u][0] = *(const uint4*)(wp0 + (size_t)du * 512);
            if (NM == 2) wv[u][NM - 1] = *(const uint4*)(wp1 + (size_t)du * 512);
            if constexpr (NIN) {
#pragma unroll
                for (int r = 0; r < RT; r++)
                    x2[u][r] = *(const uint32_t*)(a.x + (size_t)r * a.ldx +
                                                  (size_t)(s0 + du) * 128 + 2 * lane);
                g2[u] = *(const uint32_t*)(a.in_gamma + (s0 + du) * 128 + 2 * lane);
            } else {
#pragma unroll
                for (int r = 0; r < RT; r++)
                    xv[u][r] = *(const uint4*)(xp + (size_t)r * a.ldx + du * 128);
            }
        }
        if constexpr (NIN) {
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
        }
        // every step is computed: no branch may separate a load from its
        // use, or the compiler sinks the load into the branch; steps past
        // the wavefront's last contribute zero weights
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const uint32_t keep = lane_mask((uint32_t)u < cnt);
#pragma unroll
            for (int m = 0; m < NM; m++) wv[u][m] = and4(wv[u][m], keep);
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    if (L == 0) {  // any weight: every product widened
                        acc[m][r] += dot2_wide(wv[u][m].x, xv[u][r].x) +
                                     dot2_wide(wv[u][m].y, xv[u][r].y) +
                                     dot2_wide(wv[u][m].z, xv[u][r].z) +
                                     dot2_wide(wv[u][m].w, xv[u][r].w);
                    } else {
                        int32_t p = part[m][r];
                        p = dot2(wv[u][m].x, xv[u][r].x, p);
                        p = dot2(wv[u][m].y, xv[u][r].y, p);
                        p = dot2(wv[u][m].z, xv[u][r].z, p);
                        p = dot2(wv[u][m].w, xv[u][r].w, p);
                        part[m][r] = p;
                    }
                }
            if (L != 0 && L < SPW && (u + 1) % L == 0) {
#pragma unroll
                for (int m = 0; m < NM; m++)
#pragma unroll
                    for (int r = 0; r < RT; r++) acc[m][r] += part[m][r], part[m][r] = 0;
            }
        }
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < RT; r++) acc[m][r] += part[m][r];
    }
    constexpr int UNR = WPB >= 16 ? LLM_PROJ_UNROLL_LONG : LLM_PROJ_UNROLL;
    for (uint32_t s = s0; SPW == 0 && s < s1;) {
        const uint32_t lim = (L == 0) ? s1 : (s + L < s1 ? s + L : s1);
#pragma unroll UNR
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
                // unconditional (the norm table is padded to whole k-steps):
                // past in_cols the activations are 0 and so is the product
                const uint4 gv = *(const uint4*)(a.in_gamma + s * 128 + j * 8);
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
        for (int r = 0; r < RT; r++) acc[m][r] = row16_sum(acc[m][r]);

    __shared__ int64_t red[WPB][NM][4][RT];
    if (j == 15) {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < RT; r++) red[wave][m][i][r] = acc[m][r];
    }
    __syncthreads();
    if (eout) {
        const int ii = et / RT;
        int64_t tot[NM];
#pragma unroll
        for (int m = 0; m < NM; m++) {
            tot[m] = tree_sum64<WPB>([&](int w) { return red[w][m][ii][er]; });
        }
        if constexpr (EPI == EPI_SILU && RT <= 2)
            silu_out_scalar<4 * RT>(a, er, en, tot[0], tot[NM - 1], et);
        else
            proj_out<EPI>(a, er, en, tot[0], tot[NM - 1], ei);
    }
    if (efill) a.final_out[(size_t)fr * a.ldn + fn] = fill;
}

// ---------------------------------------------------------------------
// Projection over 12-bit weights ("p12"), for matrices whose weights all
// lie in [-2048, 2047]: w + 2048 = 256 h + l with l a byte and h a nibble,
// so that sum_k w x = 256 sum h x + sum l x - 2048 sum x, every term an
// exact integer (the same sums as the 16-bit kernel, 3/4 of its bytes).
// Per 4-row block and k-step 768 bytes: the l bytes of lane (i, j) (row i,
// columns 8j..8j+7) at 8 (16 i + j), then its h nibbles as one word at
// 512 + 4 (16 i + j), column 2m in bits 4m..4m+3 and column 2m + 1 in bits
// 16 + 4m..16 + 4m + 3, so that (word >> 4m) & 0x000F000F is the int16
// pair of columns (2m, 2m + 1).  A wavefront holds at most SPW k-steps,
// all loaded before the first product; partial sums stay in int32
// (SPW <= 32: |sum l x| <= 8 SPW 255 2^15 < 2^31).
// ---------------------------------------------------------------------
// CORR: the copies carry corrections (ProjArgs::corr0 / corr1; a separate
// variant, so that the common one holds no registers for them): the slot
// words are loaded when the kernel starts, a row's activations at its
// correction columns in the epilogue, for rows that have any.
template <int RT, int EPI, int WPB, int SPW, bool CORR = false>
__global__ __launch_bounds__(64 * WPB) void proj_p12_kernel(ProjArgs a) {
    static_assert(SPW <= 32, "int32 partial sums");
    constexpr int NM = EPI == EPI_SILU ? 2 : 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane >> 4, j = lane & 15;
    const uint32_t b = blockIdx.x;
    const int et = threadIdx.x;
    const uint32_t en = b * 4 + et / RT, er = et % RT;
    const bool eout = et < 4 * RT && er < a.rows && en < a.n;
    EpiIn ei{0, 0, 0};
    if (eout) ei = epi_fetch<EPI>(a, er, en);
    CorrIn cr[NM] = {};
    if (CORR && eout) {
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const uint32_t* corr = m == 0 ? a.corr0 : a.corr1;
            if (corr) corr_slots(corr, en, cr[m]);
        }
    }
    const uint32_t fn = b * 4 + (et >> 3), fr = et & 7;
    const bool efill = EPI == EPI_RESID && a.final_out && et < 32 && fr >= a.rows && fn < a.n;
    int16_t fill = 0;
    if (efill) fill = a.res[(size_t)fr * a.ldr + fn];
    const uint32_t S = a.steps;
    const uint32_t s0 = wave * S / WPB, s1 = (wave + 1) * S / WPB;
    const uint32_t cnt = s1 - s0;  // <= SPW (the launcher's choice)

    const uint8_t* wp[NM];
    wp[0] = a.p0 + (size_t)(b * S + s0) * 768;
    if (NM == 2) wp[NM - 1] = a.p1 + (size_t)(b * S + s0) * 768;
    const int16_t* xp = a.x + (size_t)s0 * 128 + j * 8;
    uint2 lo[SPW][NM];
    uint32_t hi[SPW][NM];
    uint4 xv[SPW][RT], gv[SPW];
    uint32_t x2[SPW], g2[SPW];
    uint32_t xw[SPW][RT];  // columns 2 lane, 2 lane + 1 of each step (spread8)
    // EPI_STORE_NORM_IN (one row: the kernel's only use): lane l loads and
    // normalises columns 2l, 2l + 1 of each step once per wavefront
    constexpr bool NIN = EPI == EPI_STORE_NORM_IN && RT == 1;
    // every other epilogue: each step's activations loaded once per
    // wavefront and spread to the lanes' column groups
    constexpr bool SPREAD = EPI != EPI_STORE_NORM_IN;
#pragma unroll
    for (int u = 0; u < SPW; u++) {
        const uint32_t du = cnt == 0 ? 0 : ((uint32_t)u < cnt ? u : cnt - 1);
#pragma unroll
        for (int m = 0; m < NM; m++) {
            lo[u][m] = *(const uint2*)(wp[m] + (size_t)du * 768 + 8 * lane);
            hi[u][m] = *(const uint32_t*)(wp[m] + (size_t)du * 768 + 512 + 4 * lane);
        }
        if constexpr (NIN) {
            // columns 2 lane, 2 lane + 1 of the step (normalised once per wave)
            x2[u] = *(const uint32_t*)(a.x + (size_t)(s0 + du) * 128 + 2 * lane);
            g2[u] = *(const uint32_t*)(a.in_gamma + (s0 + du) * 128 + 2 * lane);
        } else if constexpr (SPREAD) {
#pragma unroll
            for (int r = 0; r < RT; r++)
                xw[u][r] = *(const uint32_t*)(a.x + (size_t)r * a.ldx + (size_t)(s0 + du) * 128 + 2 * lane);
        } else {
#pragma unroll
            for (int r = 0; r < RT; r++) xv[u][r] = *(const uint4*)(xp + (size_t)r * a.ldx + du * 128);
            // the norm table is padded to whole k-steps
            gv[u] = *(const uint4*)(a.in_gamma + (s0 + du) * 128 + j * 8);
        }
    }
    if constexpr (NIN) {
        // the wave's steps normalised, 2 columns per lane, shared through
        // LDS (a wavefront's LDS operations complete in order)
        __shared__ uint32_t xs[WPB][SPW][64];
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const int32_t lo16 = norm1((int16_t)(x2[u] & 0xffff), __mul24(a.in_gain, (int16_t)(g2[u] & 0xffff)));
            const int32_t hi16 = norm1((int16_t)(x2[u] >> 16), __mul24(a.in_gain, (int16_t)(g2[u] >> 16)));
            xs[wave][u][lane] = (uint32_t)(uint16_t)lo16 | ((uint32_t)hi16 << 16);
        }
#pragma unroll
        for (int u = 0; u < SPW; u++) xv[u][0] = *(const uint4*)&xs[wave][u][4 * j];
    }
    int32_t pl[NM][RT], ph[NM][RT], sx[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        sx[r] = 0;
#pragma unroll
        for (int m = 0; m < NM; m++) pl[m][r] = 0, ph[m][r] = 0;
    }
    // steps past the wavefront's last carry zero activations (no branch
    // between a load and its use)
#pragma unroll
    for (int u = 0; u < SPW; u++) {
        const uint32_t keep = lane_mask((uint32_t)u < cnt);
#pragma unroll
        for (int r = 0; r < RT; r++) {
            uint4 xr;
            if constexpr (SPREAD)
                xr = spread8(xw[u][r], j);
            else if constexpr (NIN)
                xr = xv[u][r];
            else
                xr = norm8(xv[u][r], gv[u], a.in_gain);
            const uint4 x = and4(xr, keep);
            sx[r] = dot2(0x00010001u, x.x, sx[r]);
            sx[r] = dot2(0x00010001u, x.y, sx[r]);
            sx[r] = dot2(0x00010001u, x.z, sx[r]);
            sx[r] = dot2(0x00010001u, x.w, sx[r]);
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const uint2 l8 = lo[u][m];
                const uint32_t h4 = hi[u][m];
                int32_t p = pl[m][r], q = ph[m][r];
                p = dot2(__builtin_amdgcn_perm(0u, l8.x, 0x0c010c00u), x.x, p);
                p = dot2(__builtin_amdgcn_perm(0u, l8.x, 0x0c030c02u), x.y, p);
                p = dot2(__builtin_amdgcn_perm(0u, l8.y, 0x0c010c00u), x.z, p);
                p = dot2(__builtin_amdgcn_perm(0u, l8.y, 0x0c030c02u), x.w, p);
                q = dot2(h4 & 0x000f000fu, x.x, q);
                q = dot2((h4 >> 4) & 0x000f000fu, x.y, q);
                q = dot2((h4 >> 8) & 0x000f000fu, x.z, q);
                q = dot2((h4 >> 12) & 0x000f000fu, x.w, q);
                pl[m][r] = p;
                ph[m][r] = q;
            }
        }
    }
    int64_t acc[NM][RT];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < RT; r++) {
            acc[m][r] = 256 * (int64_t)ph[m][r] + pl[m][r] - 2048 * (int64_t)sx[r];
            acc[m][r] = row16_sum(acc[m][r]);
        }
    __shared__ int64_t red[WPB][NM][4][RT];
    if (j == 15) {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < RT; r++) red[wave][m][i][r] = acc[m][r];
    }
    __syncthreads();
    if (eout) {
        const int ii = et / RT;
        int64_t tot[NM];
#pragma unroll
        for (int m = 0; m < NM; m++) {
            tot[m] = tree_sum64<WPB>([&](int w) { return red[w][m][ii][er]; });
            if (CORR && (cr[m].e[0] | cr[m].e[1] | cr[m].e[2] | cr[m].e[3]) != 0) {
                corr_inputs<EPI, false>(a, er, cr[m]);
                tot[m] += corr_sum(cr[m]);
            }
        }
        if constexpr (EPI == EPI_SILU)
            silu_out_scalar<4 * RT>(a, er, en, tot[0], tot[NM - 1], et);
        else
            proj_out<EPI>(a, er, en, tot[0], tot[NM - 1], ei);
    }
    if (efill) a.final_out[(size_t)fr * a.ldn + fn] = fill;
}

// ---------------------------------------------------------------------
// Projection on the matrix cores, for blocks of several rows.
//
// int16 operands are split into bytes, w = 256 a + b + 128 and
// x = 256 c + d + 128 with a = w >> 8 and b = (w & 255) - 128 in [-128, 127]
// (likewise c, d), so that
//   sum w x = 65536 sum ac + 256 (sum ad + sum bc) + sum bd
//           + 32768 sum a + 128 sum b + 32768 sum c + 128 sum d + 16384 K
// over the padded K (zero weights pad; whatever the activations hold there
// enters both sides alike).  The 16 rows of the A operand of
// v_mfma_i32_16x16x64_i8 hold both byte planes of the (at most 8)
// activation rows: row r < 8 the high bytes c of activation row r, row
// 8 + r its low bytes d.  One product with the weights' high plane then
// gives sum ac (rows 0-7) and sum ad (rows 8-15), one with the low plane
// sum bc and sum bd: two matrix products per matrix and K chunk.  Each sum
// is bounded by 2^14 K < 2^31 for K <= 32768; the weight sums come with the
// layout, the activation sums from v_dot4.  Rows of the A operand whose
// activation row is not active carry whatever the buffer holds and only
// reach outputs that are not read.
// Workgroup = KS wavefronts on one 16-output chunk, splitting the K
// chunks; every wavefront keeps PD chunks of loads in flight.  LDS
// reduction over the wavefronts, then the shared epilogue.
// ---------------------------------------------------------------------
typedef int32_t v4i __attribute__((ext_vector_type(4)));

// The A operand of lane i (< 16) of a row of lanes: 16 inputs of
// activation row i & 7, its high bytes (i < 8) or biased low bytes
// (i >= 8), element e in byte e.  Lane i holds inputs 0-7 of the 16, lane
// i + 8 inputs 8-15 (one 16-byte load each): each lane forms both byte
// planes of its 8 inputs and passes its partner's plane across (DPP row
// rotation by 8 pairs lanes i and i + 8).
__device__ __forceinline__ v4i plane16(const v4u& x, bool hi_plane) {
    const uint32_t h0 = __builtin_amdgcn_perm(x.y, x.x, 0x07050301u);
    const uint32_t h1 = __builtin_amdgcn_perm(x.w, x.z, 0x07050301u);
    const uint32_t l0 = __builtin_amdgcn_perm(x.y, x.x, 0x06040200u) ^ 0x80808080u;
    const uint32_t l1 = __builtin_amdgcn_perm(x.w, x.z, 0x06040200u) ^ 0x80808080u;
    const int32_t r0 = __builtin_amdgcn_update_dpp(0, (int32_t)(hi_plane ? l0 : h0), 0x128, 0xf,
                                                   0xf, false);
    const int32_t r1 = __builtin_amdgcn_update_dpp(0, (int32_t)(hi_plane ? l1 : h1), 0x128, 0xf,
                                                   0xf, false);
    return hi_plane ? v4i{(int32_t)h0, (int32_t)h1, r0, r1}
                    : v4i{r0, r1, (int32_t)l0, (int32_t)l1};
}
__device__ __forceinline__ int32_t byte_sum(const v4i& v, int32_t acc) {
    acc = __builtin_amdgcn_sdot4(v.x, 0x01010101, acc, false);
    acc = __builtin_amdgcn_sdot4(v.y, 0x01010101, acc, false);
    acc = __builtin_amdgcn_sdot4(v.z, 0x01010101, acc, false);
    return __builtin_amdgcn_sdot4(v.w, 0x01010101, acc, false);
}

// Operands of one K chunk as loaded: both weight planes per matrix, the
// lane's 8 activations (its half of the 16 of its A row) and, for
// EPI_STORE_NORM_IN, their 8 gammas.
template <int NM, int EPI>
struct MfChunk {
    v4i bh[NM], bl[NM];
    v4u xh;
    v4u gh;
};

template <int NM, int EPI>
__device__ __forceinline__ void mf_load(const ProjArgs& a, const int8_t* const* bp,
                                        const int16_t* xp, const int16_t* gp, uint32_t q,
                                        MfChunk<NM, EPI>& ch) {
#pragma unroll
    for (int m = 0; m < NM; m++) {
        ch.bh[m] = *(const v4i*)(bp[m] + (size_t)q * kMfRecord);
        ch.bl[m] = *(const v4i*)(bp[m] + (size_t)q * kMfRecord + 1024);
    }
    ch.xh = *(const v4u*)(xp + 64 * q);
    if (EPI == EPI_STORE_NORM_IN) {
        // unconditional: the norm table is padded by a whole k-step, and
        // past in_cols the activations are 0 and so is the normalised value
        ch.gh = *(const v4u*)(gp + 64 * q);
    }
}

// One K chunk: activations (normalised first for EPI_STORE_NORM_IN) to the
// lane's byte plane, its byte sum, two products per matrix.
template <int NM, int EPI>
__device__ __forceinline__ void mf_compute(const ProjArgs& a, const MfChunk<NM, EPI>& ch,
                                           bool hi_plane, bool ok, v4i* c1, v4i* c2,
                                           int32_t& rs) {
    v4u x = ch.xh;
    if (EPI == EPI_STORE_NORM_IN) {
        // each lane normalises its own 8 inputs; lanes i and i + 8 then
        // exchange byte planes of the normalised values
        const uint4 nm = norm8(make_uint4(x.x, x.y, x.z, x.w),
                               make_uint4(ch.gh.x, ch.gh.y, ch.gh.z, ch.gh.w), a.in_gain);
        x = v4u{nm.x, nm.y, nm.z, nm.w};
    }
    // chunks past the wavefront's last (ok false) contribute zero
    // activations; the caller computes them anyway, so that no branch
    // separates a load from its use
    const int32_t keep = (int32_t)lane_mask(ok);
    const v4i av = plane16(x, hi_plane) & v4i{keep, keep, keep, keep};
    rs = byte_sum(av, rs);
#pragma unroll
    for (int m = 0; m < NM; m++) {
        c1[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, ch.bh[m], c1[m], 0, 0, 0);
        c2[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, ch.bl[m], c2[m], 0, 0, 0);
    }
}

// Eight 4-bit high parts h of one p12 nibble word (column 2m at bits 4m,
// column 2m + 1 at bits 16 + 4m) as the signed bytes h - 8, column e in
// byte e of the pair: w + 2048 = 256 h + l makes h - 8 = w >> 8, the byte
// planes' high byte.
__device__ __forceinline__ uint2 p12_high_bytes(uint32_t w) {
    const uint32_t x = w & 0x0F0F0F0Fu;         // columns 0 4 1 5
    const uint32_t y = (w >> 4) & 0x0F0F0F0Fu;  // columns 2 6 3 7
    uint32_t c0 = __builtin_amdgcn_perm(y, x, 0x06040200u);  // columns 0 1 2 3
    uint32_t c1 = __builtin_amdgcn_perm(y, x, 0x07050301u);  // columns 4 5 6 7
    // h - 8 in every byte without borrows between bytes: (h + 128 - 8) ^ 128
    c0 = ((c0 | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
    c1 = ((c1 | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
    return make_uint2(c0, c1);
}

// Exact sum (int64) of output (r, n) from its four product sums, the weight
// sums (m0 = sum a, m1 = sum b), the activation sums and K.
__device__ __forceinline__ int64_t mf_total(int64_t ac, int64_t ad, int64_t bc, int64_t bd,
                                            int32_t m0, int32_t m1, int64_t sc, int64_t sd,
                                            int64_t k64) {
    return 65536 * ac + 256 * (ad + bc) + bd + 32768 * (int64_t)m0 + 128 * (int64_t)m1 +
           32768 * sc + 128 * sd + 16384 * k64;
}

// Epilogue operands of a matrix-core workgroup's first outputs (thread t:
// row t / 16, output 16c + t % 16), fetched when the kernel starts.
template <int NM, int EPI>
struct MfEpi {
    EpiIn ei;
    int32_t ems[NM][2];
    int16_t fill;
    CorrIn cr[NM];  // correction slots of the 12-bit copies (zero without)
};
template <int NM, int EPI>
__device__ __forceinline__ MfEpi<NM, EPI> mf_epi_fetch(const ProjArgs& a, uint32_t c) {
    const uint32_t et = threadIdx.x, er = et >> 4, en = c * kMfRows + (et & 15);
    MfEpi<NM, EPI> e{};
    if (et < 256 && en < a.n) {
        if (er < a.rows) {
            e.ei = epi_fetch<EPI>(a, er, en);
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const int32_t* ms = m == 0 ? a.ms0 : a.ms1;
                e.ems[m][0] = ms[2 * en];
                e.ems[m][1] = ms[2 * en + 1];
                const uint32_t* corr = m == 0 ? a.corr0 : a.corr1;
                if (corr) corr_slots(corr, en, e.cr[m]);  // activations at the end
            }
        } else if (EPI == EPI_RESID && a.final_out && er < 8) {
            e.fill = a.res[(size_t)er * a.ldr + en];
        }
    }
    return e;
}

// The end of a matrix-core workgroup: product sums of the wavefronts
// reduced in LDS (red, rsum), split-K partials handed to the last
// workgroup of the chunk to arrive, then the exact sums and the epilogue.
// C lane l holds rows 4 (l / 16) + s, column l % 16.
template <int NM, int KS, int EPI>
__device__ __forceinline__ void mf_finish(const ProjArgs& a, uint32_t c, uint32_t p,
                                          uint32_t parts, const v4i* c1, const v4i* c2,
                                          int32_t rs, const MfEpi<NM, EPI>& fe,
                                          v4i (*red)[NM][2][64], int32_t (*rsum)[64],
                                          uint32_t* last) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t et = threadIdx.x;
#pragma unroll
    for (int m = 0; m < NM; m++) {
        red[wave][m][0][lane] = c1[m];
        red[wave][m][1][lane] = c2[m];
    }
    rsum[wave][lane] = rs;
    __syncthreads();
    // element (row, col) of product ty of matrix m, summed over wavefronts
    auto wsum = [&](int m, int ty, uint32_t row, uint32_t col) -> int32_t {
        int32_t v = 0;
#pragma unroll
        for (int w = 0; w < KS; w++) v += red[w][m][ty][16 * (row >> 2) + col][row & 3];
        return v;
    };
    // byte sum of A row `row` (activation row row & 7, plane row >> 3)
    auto rsum_row = [&](uint32_t row) -> int32_t {
        int32_t v = 0;
#pragma unroll
        for (int w = 0; w < KS; w++)
#pragma unroll
            for (int gg = 0; gg < 4; gg++) v += rsum[w][row + 16 * gg];
        return v;
    };
    constexpr uint32_t W = mf_part_words(NM);
    if (parts > 1) {
        // this workgroup's sums: element t = 16 row + col of each product,
        // then the 16 A-row byte sums
        int32_t* part = a.mf_part + (size_t)(c * parts + p) * W;
        for (uint32_t t = threadIdx.x; t < 256; t += 64 * KS) {
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int ty = 0; ty < 2; ty++)
                    st_coherent(&part[(m * 2 + ty) * 256 + t], wsum(m, ty, t >> 4, t & 15));
            if (t < 16) st_coherent(&part[NM * 2 * 256 + t], rsum_row(t));
        }
        if (!arrive_last(&a.mf_count[c], parts, last)) return;
    }
    const int64_t k64 = (int64_t)a.kq * kMfCols;
    for (uint32_t t = threadIdx.x; t < 256; t += 64 * KS) {
        const uint32_t r = t >> 4, j = t & 15, nn = c * kMfRows + j;
        if (nn >= a.n) continue;
        if (r < a.rows) {
            int64_t s[NM][4], sc = 0, sd = 0;
            if (parts > 1) {
#pragma unroll
                for (int m = 0; m < NM; m++) s[m][0] = s[m][1] = s[m][2] = s[m][3] = 0;
                for (uint32_t pp = 0; pp < parts; pp++) {
                    const int32_t* q = a.mf_part + (size_t)(c * parts + pp) * W;
#pragma unroll
                    for (int m = 0; m < NM; m++) {
                        s[m][0] += ld_coherent(&q[(m * 2) * 256 + 16 * r + j]);
                        s[m][1] += ld_coherent(&q[(m * 2) * 256 + 16 * (8 + r) + j]);
                        s[m][2] += ld_coherent(&q[(m * 2 + 1) * 256 + 16 * r + j]);
                        s[m][3] += ld_coherent(&q[(m * 2 + 1) * 256 + 16 * (8 + r) + j]);
                    }
                    sc += ld_coherent(&q[NM * 2 * 256 + r]);
                    sd += ld_coherent(&q[NM * 2 * 256 + 8 + r]);
                }
            } else {
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    s[m][0] = wsum(m, 0, r, j);
                    s[m][1] = wsum(m, 0, 8 + r, j);
                    s[m][2] = wsum(m, 1, r, j);
                    s[m][3] = wsum(m, 1, 8 + r, j);
                }
                sc = rsum_row(r);
                sd = rsum_row(8 + r);
            }
            // later outputs of this thread (fewer than 4 wavefronts) fetch
            // their operands here
            const bool first = t == et;
            EpiIn e = first ? fe.ei : epi_fetch<EPI>(a, r, nn);
            int64_t tot[NM];
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const int32_t* ms = m == 0 ? a.ms0 : a.ms1;
                const int32_t m0 = first ? fe.ems[m][0] : ms[2 * nn];
                const int32_t m1 = first ? fe.ems[m][1] : ms[2 * nn + 1];
                tot[m] = mf_total(s[m][0], s[m][1], s[m][2], s[m][3], m0, m1, sc, sd, k64);
                const uint32_t* corr = m == 0 ? a.corr0 : a.corr1;
                if (corr) {
                    CorrIn c = fe.cr[m];
                    if (!first) corr_slots(corr, nn, c);
                    if ((c.e[0] | c.e[1] | c.e[2] | c.e[3]) != 0) {
                        corr_inputs<EPI, false>(a, r, c);
                        tot[m] += corr_sum(c);
                    }
                }
            }
            proj_out<EPI>(a, r, nn, tot[0], tot[NM - 1], e);
        } else if (EPI == EPI_RESID && a.final_out && r < 8) {
            a.final_out[(size_t)r * a.ldn + nn] =
                t == et ? fe.fill : a.res[(size_t)r * a.ldr + nn];
        }
    }
}

template <int NM, int KS, int QM, int PD, int EPI>
__global__ __launch_bounds__(64 * KS) void proj_mfma_kernel(ProjArgs a, uint32_t parts) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t c = blockIdx.x / parts, p = blockIdx.x % parts, KQ = a.kq;
    const uint32_t pq0 = p * KQ / parts, pq1 = (p + 1) * KQ / parts;
    const uint32_t q0 = pq0 + wave * (pq1 - pq0) / KS;
    const uint32_t q1 = pq0 + (wave + 1) * (pq1 - pq0) / KS;
    const uint32_t n = q1 - q0;  // <= QM (the launcher's choice)
    const uint32_t i = lane & 15, g = lane >> 4;
    const bool hi_plane = i < 8;
    // every activation buffer holds 8 rows: row i & 7 is always in bounds;
    // lane i holds inputs 8 (i / 8) .. + 7 of its 16
    const int16_t* xp = a.x + (size_t)(i & 7) * a.ldx + 16 * g + 8 * (i >> 3);
    const int16_t* gp = EPI == EPI_STORE_NORM_IN ? a.in_gamma + 16 * g + 8 * (i >> 3) : nullptr;
    const MfEpi<NM, EPI> fe = mf_epi_fetch<NM, EPI>(a, c);
    const int8_t* bp[NM];
    bp[0] = a.mf0 + (size_t)c * KQ * kMfRecord + lane * 16;
    if (NM == 2) bp[NM - 1] = a.mf1 + (size_t)c * KQ * kMfRecord + lane * 16;
    v4i c1[NM], c2[NM];
#pragma unroll
    for (int m = 0; m < NM; m++) c1[m] = c2[m] = v4i{0, 0, 0, 0};
    int32_t rs = 0;
    // Chunk u of this wavefront is q0 + u; loads past the last chunk
    // repeat it (in bounds, its products add zero).  A wavefront with no
    // chunk reads chunk pq0 and uses none.
    auto chunk_q = [&](uint32_t u) -> uint32_t {
        return n == 0 ? pq0 : q0 + (u < n ? u : n - 1);
    };
    MfChunk<NM, EPI> ring[PD];
#pragma unroll
    for (int u = 0; u < PD; u++) mf_load<NM, EPI>(a, bp, xp, gp, chunk_q(u), ring[u]);
#pragma unroll
    for (int u = 0; u < QM; u++) {
        const MfChunk<NM, EPI> cur = ring[u % PD];
        if (u + PD < QM) mf_load<NM, EPI>(a, bp, xp, gp, chunk_q(u + PD), ring[u % PD]);
        mf_compute<NM, EPI>(a, cur, hi_plane, (uint32_t)u < n, c1, c2, rs);
    }
    __shared__ v4i red[KS][NM][2][64];
    __shared__ int32_t rsum[KS][64];
    __shared__ uint32_t last;
    mf_finish<NM, KS, EPI>(a, c, p, parts, c1, c2, rs, fe, red, rsum, &last);
}

// ---------------------------------------------------------------------
// The matrix-core kernel over the 12-bit copies (p12 layout, see
// proj_p12_kernel), for matrices whose weights all fit 12 bits: 3/4 of
// the byte-plane bytes.  w + 2048 = 256 h + l makes h - 8 the byte planes'
// high byte (w >> 8) and l ^ 128 their biased low byte, so the products,
// weight sums and exact totals are the byte-plane kernel's.  The operand
// of lane l (output 16c + l % 16, inputs 64q + 16 (l / 16) .. + 15) lies in
// 64-byte pieces of four block records, so each wavefront loads whole
// 768-byte records of its four blocks instead -- 48 contiguous bytes per
// lane and step, lanes 16b .. 16b + 15 on block 4c + b -- writes them to
// its own LDS slice and reads the operands back from there (a wavefront's
// LDS operations complete in order: no barrier).  Work is split in whole
// 128-column steps (two K chunks); a half past kq carries zero activations.
// ---------------------------------------------------------------------
constexpr uint32_t kP12LoRow = 144;  // 128 low bytes of a block row + 16 of padding
constexpr uint32_t kP12NbRow = 80;   // 64 nibble-word bytes of a block row + 16
template <int NM>
struct __attribute__((aligned(16))) P12Stage {
    uint8_t lo[NM][4][4][kP12LoRow];  // [matrix][block][row][bytes]
    uint8_t nb[NM][4][4][kP12NbRow];
};

template <int NM, int EPI>
struct P12Step {
    v4i r[NM][3];  // record bytes 16 (lane % 16) + {0, 256, 512}
    v4u xh[2];     // the lane's 8 activations of the step's two K chunks
    v4u gh[2];     // their gammas (EPI_STORE_NORM_IN)
};

template <int NM, int EPI>
__device__ __forceinline__ void p12_step_load(const ProjArgs& a, const uint8_t* const* src,
                                              const int16_t* xp, const int16_t* gp, uint32_t s,
                                              P12Step<NM, EPI>& st) {
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int t = 0; t < 3; t++)
            st.r[m][t] = *(const v4i*)(src[m] + (size_t)s * kP12Step + 256 * t);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        // columns 128 s + 64 h + 16 (lane / 16) .. + 15 lie below the
        // activations' padded width (a whole number of 128-column steps)
        st.xh[h] = *(const v4u*)(xp + 128 * s + 64 * h);
        if (EPI == EPI_STORE_NORM_IN) st.gh[h] = *(const v4u*)(gp + 128 * s + 64 * h);
    }
}

template <int NM, int KS, int SM, int PDS, int EPI>
__global__ __launch_bounds__(64 * KS) void proj_mfma12_kernel(ProjArgs a, uint32_t parts) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t c = blockIdx.x / parts, p = blockIdx.x % parts, S = a.steps, KQ = a.kq;
    const uint32_t ps0 = p * S / parts, ps1 = (p + 1) * S / parts;
    const uint32_t s0 = ps0 + wave * (ps1 - ps0) / KS;
    const uint32_t s1 = ps0 + (wave + 1) * (ps1 - ps0) / KS;
    const uint32_t n = s1 - s0;  // <= SM (the launcher's choice)
    const uint32_t i = lane & 15, g = lane >> 4;
    const bool hi_plane = i < 8;
    const int16_t* xp = a.x + (size_t)(i & 7) * a.ldx + 16 * g + 8 * (i >> 3);
    const int16_t* gp = EPI == EPI_STORE_NORM_IN ? a.in_gamma + 16 * g + 8 * (i >> 3) : nullptr;
    const MfEpi<NM, EPI> fe = mf_epi_fetch<NM, EPI>(a, c);
    // load lanes: block 4c + lane / 16, clamped to the copy's last block
    // (rows past n reach only outputs that are never written)
    const uint32_t nblk = (a.n + kBlockRows - 1) / kBlockRows;
    const uint32_t lb = min(4 * c + (lane >> 4), nblk - 1);
    const uint8_t* src[NM];
    src[0] = a.p0 + (size_t)lb * S * kP12Step + 16 * (lane & 15);
    if (NM == 2) src[NM - 1] = a.p1 + (size_t)lb * S * kP12Step + 16 * (lane & 15);
    __shared__ union {
        P12Stage<NM> st[KS];
        struct {
            v4i red[KS][NM][2][64];
            int32_t rsum[KS][64];
        } fin;
    } sm;
    __shared__ uint32_t last;
    P12Stage<NM>& my = sm.st[wave];
    // where this lane's record bytes go: +0 low bytes of row (lane%16)/8,
    // +256 of row 2 + (lane%16)/8, both at column 16 ((lane%16) % 8);
    // +512 nibble words 4 (lane%16) .. + 3, row (lane%16)/4
    const uint32_t o = lane & 15, bw = lane >> 4;
    // where lane's operand is read: block i / 4, row i % 4
    const uint32_t ob = i >> 2, orow = i & 3;
    v4i c1[NM], c2[NM];
#pragma unroll
    for (int m = 0; m < NM; m++) c1[m] = c2[m] = v4i{0, 0, 0, 0};
    int32_t rs = 0;
    // Step u of this wavefront is s0 + u; loads past the last step repeat
    // it (in bounds, its products add zero).  A wavefront with no step
    // reads step ps0 and uses none.
    auto step_s = [&](uint32_t u) -> uint32_t {
        return n == 0 ? ps0 : s0 + (u < n ? u : n - 1);
    };
    P12Step<NM, EPI> ring[PDS];
#pragma unroll
    for (int u = 0; u < PDS; u++) p12_step_load<NM, EPI>(a, src, xp, gp, step_s(u), ring[u]);
#pragma unroll
    for (int u = 0; u < SM; u++) {
        const uint32_t s = step_s(u);
        P12Step<NM, EPI>& rg = ring[u % PDS];
        P12Step<NM, EPI> cur;
        // One matrix: step u's records into the slice first, so that the
        // next step's loads reuse their registers (only the activations are
        // kept; measured faster for down and Q|K|V).  Two (gate|up): the
        // next step's loads first, while step u's are still in flight.
        if (NM == 2) {
            cur = rg;
            if (u + PDS < SM) p12_step_load<NM, EPI>(a, src, xp, gp, step_s(u + PDS), rg);
        }
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const P12Step<NM, EPI>& sr = NM == 2 ? cur : rg;
            *(v4i*)&my.lo[m][bw][o >> 3][16 * (o & 7)] = sr.r[m][0];
            *(v4i*)&my.lo[m][bw][2 + (o >> 3)][16 * (o & 7)] = sr.r[m][1];
            *(v4i*)&my.nb[m][bw][o >> 2][16 * (o & 3)] = sr.r[m][2];
        }
        if (NM == 1) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                cur.xh[h] = rg.xh[h];
                cur.gh[h] = rg.gh[h];
            }
            if (u + PDS < SM) p12_step_load<NM, EPI>(a, src, xp, gp, step_s(u + PDS), rg);
        }
        // the reads below see other lanes' writes: the fences keep the
        // compiler from moving LDS accesses across (no instruction)
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int h = 0; h < 2; h++) {
            MfChunk<NM, EPI> ch;
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const v4i lo = *(const v4i*)&my.lo[m][ob][orow][64 * h + 16 * g];
                typedef uint32_t v2u __attribute__((ext_vector_type(2)));
                const v2u nw = *(const v2u*)&my.nb[m][ob][orow][32 * h + 8 * g];
                const uint2 h0 = p12_high_bytes(nw.x), h1 = p12_high_bytes(nw.y);
                ch.bh[m] = v4i{(int32_t)h0.x, (int32_t)h0.y, (int32_t)h1.x, (int32_t)h1.y};
                ch.bl[m] = lo ^ v4i{(int32_t)0x80808080u, (int32_t)0x80808080u,
                                    (int32_t)0x80808080u, (int32_t)0x80808080u};
            }
            ch.xh = cur.xh[h];
            ch.gh = cur.gh[h];
            // a half past the matrix's K chunks (odd kq) adds nothing
            mf_compute<NM, EPI>(a, ch, hi_plane, (uint32_t)u < n && 2 * s + h < KQ, c1, c2, rs);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    }
    __syncthreads();  // every wavefront's staging reads are done
    mf_finish<NM, KS, EPI>(a, c, p, parts, c1, c2, rs, fe, sm.fin.red, sm.fin.rsum, &last);
}

// ---------------------------------------------------------------------
// LM-head argmax (model_data_t::lm_head_argmax, host/host_qwen_8x64.cpp
// :937-969): exact int64 scores, strict > over increasing v.  Persistent:
// each wavefront walks 4-row blocks (all k-steps) in a grid-stride loop,
// keeps its best (score, v) per activation row, then the workgroup's best
// goes into one 64-bit atomicMax per row.  The key orders by score, then
// by smaller v, so equal scores resolve to the first index.
// ---------------------------------------------------------------------
// XS: the activation rows are staged in LDS once per workgroup (1-2 rows,
// at most kLmStageSteps k-steps) and every step reads them from there, so
// that the loads in the loop are the table's only (the four lanes of a
// column group read the same 16 bytes: an LDS broadcast).
constexpr uint32_t kLmStageSteps = 32;
template <int RT, int L, bool XS = false>
__global__ __launch_bounds__(256) void lm_argmax_kernel(const int16_t* __restrict__ w,
                                                        uint32_t S, uint32_t n,
                                                        const int16_t* __restrict__ x,
                                                        uint32_t ldx, uint32_t rows,
                                                        unsigned long long* keys) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane >> 4, j = lane & 15;
    const uint32_t nblocks = (n + 3) / 4;
    const uint32_t stride = gridDim.x * 4;
    unsigned long long best[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) best[r] = 0;
    static_assert(!XS || RT <= 2, "staged rows: 1-2");
    __shared__ __attribute__((aligned(16))) int16_t xs[XS ? RT : 1][XS ? kLmStageSteps * 128 : 8];
    if constexpr (XS) {
        // rows beyond `rows` stage row 0 (in bounds; ignored); S <= kLmStageSteps
        for (uint32_t e = threadIdx.x; e < S * 16; e += 256)
#pragma unroll
            for (int r = 0; r < RT; r++)
                *(uint4*)&xs[r][8 * e] =
                    *(const uint4*)(x + (size_t)(r < (int)rows ? r : 0) * ldx + 8 * e);
        __syncthreads();
    }
    for (uint32_t b = blockIdx.x * 4 + wave; b < nblocks; b += stride) {
        const int16_t* wp = w + ((size_t)b * S * 4 + i) * 128 + j * 8;
        const int16_t* xp = x + j * 8;
        int64_t acc[RT];
        int32_t part[RT];
#pragma unroll
        for (int r = 0; r < RT; r++) acc[r] = 0, part[r] = 0;
        for (uint32_t s = 0; s < S;) {
            const uint32_t lim = (L == 0) ? S : (s + L < S ? s + L : S);
#pragma unroll 4
            for (; s < lim; s++) {
                const uint4 wv = *(const uint4*)(wp + (size_t)s * 512);
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    // rows beyond `rows` read row 0 (in bounds; ignored)
                    const uint4 xv = XS ? *(const uint4*)&xs[XS ? r : 0][s * 128 + j * 8]
                                        : *(const uint4*)(xp + (size_t)(r < (int)rows ? r : 0) * ldx +
                                                          s * 128);
                    if (L == 0) {
                        acc[r] += dot2_wide(wv.x, xv.x) + dot2_wide(wv.y, xv.y) +
                                  dot2_wide(wv.z, xv.z) + dot2_wide(wv.w, xv.w);
                    } else {
                        int32_t p = part[r];
                        p = dot2(wv.x, xv.x, p);
                        p = dot2(wv.y, xv.y, p);
                        p = dot2(wv.z, xv.z, p);
                        p = dot2(wv.w, xv.w, p);
                        part[r] = p;
                    }
                }
            }
            if (L != 0) {
#pragma unroll
                for (int r = 0; r < RT; r++) acc[r] += part[r], part[r] = 0;
            }
        }
        const uint32_t v = b * 4 + i;
#pragma unroll
        for (int r = 0; r < RT; r++) {
            acc[r] = row16_sum(acc[r]);
            const unsigned long long k = argmax_key(acc[r], v);
            if (j == 15 && v < n && k > best[r]) best[r] = k;
        }
    }
    __shared__ unsigned long long wbest[4][4][RT];
    if (j == 15) {
#pragma unroll
        for (int r = 0; r < RT; r++) wbest[wave][i][r] = best[r];
    }
    __syncthreads();
    if (threadIdx.x < RT && threadIdx.x < rows) {
        const int r = threadIdx.x;
        unsigned long long k = 0;
        for (int ww = 0; ww < 4; ww++)
            for (int ii = 0; ii < 4; ii++) k = wbest[ww][ii][r] > k ? wbest[ww][ii][r] : k;
        atomicMax(&keys[r], k);
    }
}

template <int RT>
static hipError_t launch_lm_rt(const int16_t* w, uint32_t steps, uint32_t n,
                               const int16_t* x, uint32_t ldx, uint32_t rows, int L,
                               unsigned long long* keys, hipStream_t st) {
    const uint32_t nblocks = (n + 3) / 4;
    uint32_t grid = (nblocks + 3) / 4;
    if (grid > 2048) grid = 2048;
    if (RT <= 2 && steps <= kLmStageSteps) {
        constexpr bool XS = RT <= 2;
        switch (L) {
        case 0: lm_argmax_kernel<RT, 0, XS><<<grid, 256, 0, st>>>(w, steps, n, x, ldx, rows, keys); break;
        case 1: lm_argmax_kernel<RT, 1, XS><<<grid, 256, 0, st>>>(w, steps, n, x, ldx, rows, keys); break;
        case 4: lm_argmax_kernel<RT, 4, XS><<<grid, 256, 0, st>>>(w, steps, n, x, ldx, rows, keys); break;
        case 8: lm_argmax_kernel<RT, 8, XS><<<grid, 256, 0, st>>>(w, steps, n, x, ldx, rows, keys); break;
        default: lm_argmax_kernel<RT, 16, XS><<<grid, 256, 0, st>>>(w, steps, n, x, ldx, rows, keys); break;
        }
        return hipGetLastError();
    }
    switch (L) {
    case 0: lm_argmax_kernel<RT, 0><<<grid, 256, 0, st>>>(w, steps, n, x, ldx, rows, keys); break;
    case 1: lm_argmax_kernel<RT, 1><<<grid, 256, 0, st>>>(w, steps, n, x, ldx, rows, keys); break;
    case 4: lm_argmax_kernel<RT, 4><<<grid, 256, 0, st>>>(w, steps, n, x, ldx, rows, keys); break;
    case 8: lm_argmax_kernel<RT, 8><<<grid, 256, 0, st>>>(w, steps, n, x, ldx, rows, keys); break;
    default: lm_argmax_kernel<RT, 16><<<grid, 256, 0, st>>>(w, steps, n, x, ldx, rows, keys); break;
    }
    return hipGetLastError();
}

hipError_t launch_lm_argmax(const int16_t* w, uint32_t steps, uint32_t n,
                            const int16_t* x, uint32_t ldx, uint32_t rows, int L,
                            unsigned long long* keys, hipStream_t st) {
    if (rows <= 1) return launch_lm_rt<1>(w, steps, n, x, ldx, rows, L, keys, st);
    if (rows <= 2) return launch_lm_rt<2>(w, steps, n, x, ldx, rows, L, keys, st);
    if (rows <= 4) return launch_lm_rt<4>(w, steps, n, x, ldx, rows, L, keys, st);
    return launch_lm_rt<8>(w, steps, n, x, ldx, rows, L, keys, st);
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
template <int RT, int EPI, int W, int SPW>
static void launch_proj_s(const ProjArgs& a, int L, uint32_t blocks, hipStream_t st) {
    // SPW <= 4: with L >= 4 the int32 sums of a wavefront's steps widen
    // once at the end; L 1..3 widens after every step, L 0 every product
    if (L >= 4) proj_kernel<RT, 4, EPI, W, SPW><<<blocks, 64 * W, 0, st>>>(a);
    else if (L >= 1) proj_kernel<RT, 1, EPI, W, SPW><<<blocks, 64 * W, 0, st>>>(a);
    else proj_kernel<RT, 0, EPI, W, SPW><<<blocks, 64 * W, 0, st>>>(a);
}

template <int RT, int EPI, int W>
static hipError_t launch_proj_w(const ProjArgs& a, int L, uint32_t blocks,
                                hipStream_t st) {
    // all loads at once pays for up to 4 steps per wavefront; longer
    // reductions (the down projection: 6) measured faster with the loop,
    // two steps of loads at a time, at lower register use
    const uint32_t spw = (a.steps + W - 1) / W;
    if (RT <= 2 && spw <= 4) {
        if (spw <= 2) launch_proj_s<RT, EPI, W, 2>(a, L, blocks, st);
        else launch_proj_s<RT, EPI, W, 4>(a, L, blocks, st);
        return hipGetLastError();
    }
    switch (L) {
    case 0: proj_kernel<RT, 0, EPI, W, 0><<<blocks, 64 * W, 0, st>>>(a); break;
    case 1: proj_kernel<RT, 1, EPI, W, 0><<<blocks, 64 * W, 0, st>>>(a); break;
    case 4: proj_kernel<RT, 4, EPI, W, 0><<<blocks, 64 * W, 0, st>>>(a); break;
    case 8: proj_kernel<RT, 8, EPI, W, 0><<<blocks, 64 * W, 0, st>>>(a); break;
    default: proj_kernel<RT, 16, EPI, W, 0><<<blocks, 64 * W, 0, st>>>(a); break;
    }
    return hipGetLastError();
}

template <int RT, int EPI>
static hipError_t launch_proj_rt(const ProjArgs& a, int L, uint32_t blocks,
                                 hipStream_t st) {
    if (EPI == EPI_SILU) return launch_proj_w<RT, EPI, LLM_PROJ_WPB_SILU>(a, L, blocks, st);
    // long reductions (the down projection) keep more loads in flight per
    // block with 16 wavefronts (measured: 11.9 -> 9.7 us at configs[1])
    if (RT <= 2 && a.steps >= LLM_PROJ_LONG_STEPS)
        return launch_proj_w<RT, EPI, 16>(a, L, blocks, st);
    return launch_proj_w<RT, EPI, LLM_PROJ_WPB>(a, L, blocks, st);
}

// The p12 kernel (one or two rows): gate|up with 8 wavefronts per block,
// long reductions (the down projection) with 16 and the others (Q|K|V, O)
// with LLM_P12_WPB = 8 (4 in the 16-bit kernel), and 16 wherever fewer
// would take more than 8 k-steps each; every wavefront's steps loaded at
// once (proj_uses_p12 bounds the steps by 16 x 8).
template <int RT, int EPI, int W, bool CORR>
static void launch_p12_c(const ProjArgs& a, uint32_t blocks, hipStream_t st) {
    const uint32_t spw = (a.steps + W - 1) / W;
    // the smallest variant that holds the steps (registers decide how many
    // 16-wavefront blocks a compute unit holds)
    if (spw <= 2) proj_p12_kernel<RT, EPI, W, 2, CORR><<<blocks, 64 * W, 0, st>>>(a);
    else if (spw <= 4) proj_p12_kernel<RT, EPI, W, 4, CORR><<<blocks, 64 * W, 0, st>>>(a);
    else if (spw <= 6) proj_p12_kernel<RT, EPI, W, 6, CORR><<<blocks, 64 * W, 0, st>>>(a);
    else proj_p12_kernel<RT, EPI, W, 8, CORR><<<blocks, 64 * W, 0, st>>>(a);
}
template <int RT, int EPI, int W>
static hipError_t launch_p12_w(const ProjArgs& a, uint32_t blocks, hipStream_t st) {
    if (a.corr0 || a.corr1)
        launch_p12_c<RT, EPI, W, true>(a, blocks, st);
    else
        launch_p12_c<RT, EPI, W, false>(a, blocks, st);
    return hipGetLastError();
}
template <int RT, int EPI>
static hipError_t launch_p12_rt(const ProjArgs& a, uint32_t blocks, hipStream_t st) {
    if constexpr (EPI == EPI_SILU) {
        if (a.steps > 8 * LLM_PROJ_WPB_SILU) return launch_p12_w<RT, EPI, 16>(a, blocks, st);
        return launch_p12_w<RT, EPI, LLM_PROJ_WPB_SILU>(a, blocks, st);
    } else {
        if (a.steps >= LLM_PROJ_LONG_STEPS || a.steps > 8 * LLM_P12_WPB)
            return launch_p12_w<RT, EPI, 16>(a, blocks, st);
        return launch_p12_w<RT, EPI, LLM_P12_WPB>(a, blocks, st);
    }
}

template <int EPI>
static hipError_t launch_proj_epi(const ProjArgs& a, int L, uint32_t blocks,
                                  hipStream_t st) {
    if (proj_uses_p12(a, EPI))
        return a.rows <= 1 ? launch_p12_rt<1, EPI>(a, blocks, st)
                           : launch_p12_rt<2, EPI>(a, blocks, st);
    // the 16-bit copy (absent for matrices held in 12 bits only)
    if (!a.w0 || (EPI == EPI_SILU && !a.w1)) return hipErrorInvalidValue;
    if (a.rows <= 1) return launch_proj_rt<1, EPI>(a, L, blocks, st);
    if (a.rows <= 2) return launch_proj_rt<2, EPI>(a, L, blocks, st);
    if (a.rows <= 4) return launch_proj_rt<4, EPI>(a, L, blocks, st);
    return launch_proj_rt<8, EPI>(a, L, blocks, st);
}

// Largest K-chunk count of one wavefront: parts split kq, wavefronts
// split a part, each by floor division of the boundaries.
static uint32_t mf_chunks_per_wave(uint32_t kq, uint32_t parts, uint32_t ks) {
    const uint32_t per_part = (kq + parts - 1) / parts;
    return (per_part + ks - 1) / ks;
}

MfSplit mf_split(uint32_t nc, uint32_t kq) {
    // LLM_MF_KS wavefronts per workgroup (fewer when K is short), the K
    // range split over workgroups only while the chunks alone give fewer
    // than LLM_MF_WG_TARGET workgroups and each wavefront keeps two K
    // chunks, or when a wavefront would get more than LLM_MF_QMAX
    MfSplit s{LLM_MF_KS, 1};
    while (s.ks > 4 && kq < 2 * s.ks) s.ks /= 2;
    while (nc * s.parts < LLM_MF_WG_TARGET && kq / (s.parts * 2) >= s.ks * 2) s.parts *= 2;
    while (mf_chunks_per_wave(kq, s.parts, s.ks) > LLM_MF_QMAX) s.parts *= 2;
    return s;
}

template <int NM, int KS, int QM, int EPI>
static void launch_mfma_k(const ProjArgs& a, uint32_t parts, hipStream_t st) {
    constexpr int PD0 = NM == 2 ? LLM_MF_PD2 : LLM_MF_PD1;
    constexpr int PD = PD0 < QM ? PD0 : QM;
    proj_mfma_kernel<NM, KS, QM, PD, EPI><<<a.nc * parts, 64 * KS, 0, st>>>(a, parts);
}

template <int NM, int KS, int EPI>
static hipError_t launch_mfma_q(const ProjArgs& a, uint32_t parts, hipStream_t st) {
    const uint32_t qm = mf_chunks_per_wave(a.kq, parts, KS);
    if (qm <= 2)
        launch_mfma_k<NM, KS, 2, EPI>(a, parts, st);
    else if (qm <= 4)
        launch_mfma_k<NM, KS, 4, EPI>(a, parts, st);
    else if (qm <= 8)
        launch_mfma_k<NM, KS, 8, EPI>(a, parts, st);
    else if (qm <= 12)
        launch_mfma_k<NM, KS, 12, EPI>(a, parts, st);
    else
        return hipErrorInvalidConfiguration;  // mf_split keeps qm <= LLM_MF_QMAX <= 12
    return hipGetLastError();
}

// The 12-bit matrix-core kernel splits whole 128-column steps the same
// way: wavefronts keep at least one step, at most LLM_MF_QMAX / 2.  Two
// matrices (gate|up) take fewer wavefronts per workgroup below 4 steps
// each: more workgroups resident (measured faster at K = 2048; slower for
// one matrix, and for K = 11008).  One matrix with a long K (down, K =
// 11008) takes 16 wavefronts of ~3 steps over at least 256 workgroups
// (P8 down 11.5 -> 11.1 us against 8 wavefronts of ~6 steps over 128
// chunks x 2; Q|K|V and O, K = 2048, are slower so).  Not splitting K
// costs more than the partial sums' hand-off saves: 16 wavefronts of ~6
// steps over 128 workgroups took 14.2 us against 11.7, and 8-output
// chunks over 256 workgroups without a split (the MFMA's columns 8-15
// repeating 0-7) 14.1 us, 13.3 with 3 steps of loads in flight: the
// longer per-wavefront chain of steps, not the hand-off, sets the time.
MfSplit mf12_split(uint32_t nc, uint32_t steps, uint32_t nm) {
    MfSplit s{LLM_MF12_KS, 1};
    uint32_t target = LLM_MF12_WG_TARGET;
    while (nm == 2 && s.ks > 4 && steps < LLM_MF12_MIN_STEPS * s.ks) s.ks /= 2;
    if (nm == 1 && steps >= LLM_MF12_LONG_STEPS) {
        s.ks = 16;
        target = 256;
    }
    while (nc * s.parts < target && steps / (s.parts * 2) >= s.ks) s.parts *= 2;
    while (mf_chunks_per_wave(steps, s.parts, s.ks) > LLM_MF_QMAX / 2) s.parts *= 2;
    return s;
}

template <int NM, int KS, int SM, int EPI>
static void launch_mfma12_k(const ProjArgs& a, uint32_t parts, hipStream_t st) {
    // normalising on load holds the gammas too: one step in flight
    constexpr int PD0 = NM == 2 ? LLM_MF12_PD2 : EPI == EPI_STORE_NORM_IN ? 1 : LLM_MF12_PD1;
    constexpr int PD = PD0 < SM ? PD0 : SM;
    proj_mfma12_kernel<NM, KS, SM, PD, EPI><<<a.nc * parts, 64 * KS, 0, st>>>(a, parts);
}

template <int NM, int KS, int EPI>
static hipError_t launch_mfma12_s(const ProjArgs& a, uint32_t parts, hipStream_t st) {
    const uint32_t sm = mf_chunks_per_wave(a.steps, parts, KS);
    if (sm <= 1)
        launch_mfma12_k<NM, KS, 1, EPI>(a, parts, st);
    else if (sm <= 2)
        launch_mfma12_k<NM, KS, 2, EPI>(a, parts, st);
    else if (sm <= 3)
        launch_mfma12_k<NM, KS, 3, EPI>(a, parts, st);
    else if (sm <= 4)
        launch_mfma12_k<NM, KS, 4, EPI>(a, parts, st);
    else if (sm <= 6)
        launch_mfma12_k<NM, KS, 6, EPI>(a, parts, st);
    else
        return hipErrorInvalidConfiguration;  // mf12_split keeps sm <= LLM_MF_QMAX / 2 <= 6
    return hipGetLastError();
}

bool proj_mfma_reads_p12(const ProjArgs& a, int epi) {
    return a.mf_p12 && a.p0 && (epi != EPI_SILU || a.p1);
}

template <int NM, int EPI>
static hipError_t launch_mfma_epi(const ProjArgs& a, hipStream_t st) {
    if (proj_mfma_reads_p12(a, EPI) || !a.mf0 || (NM == 2 && !a.mf1)) {
        if (!proj_mfma_reads_p12(a, EPI)) return hipErrorInvalidValue;
        const MfSplit sp = mf12_split(a.nc, a.steps, NM);
        if (sp.ks >= 16) return launch_mfma12_s<NM, 16, EPI>(a, sp.parts, st);
        if (sp.ks == 8) return launch_mfma12_s<NM, 8, EPI>(a, sp.parts, st);
        return launch_mfma12_s<NM, 4, EPI>(a, sp.parts, st);
    }
    const MfSplit sp = mf_split(a.nc, a.kq);
    if (sp.ks >= 16) return launch_mfma_q<NM, 16, EPI>(a, sp.parts, st);
    if (sp.ks == 8) return launch_mfma_q<NM, 8, EPI>(a, sp.parts, st);
    return launch_mfma_q<NM, 4, EPI>(a, sp.parts, st);
}

bool proj_uses_mfma(const ProjArgs& a, int epi) {
    return a.rows >= kMfMinRows && (a.mf0 || proj_mfma_reads_p12(a, epi)) && a.mf_part &&
           a.kq * kMfCols <= 32768;
}

bool proj_uses_p12(const ProjArgs& a, int epi) {
    // blocks of one or two rows with every matrix of the launch in 12 bits
    // and at most 8 k-steps per wavefront (launch_p12_rt's wavefronts)
    return a.rows <= LLM_P12_MAX_ROWS && a.p0 && (epi != EPI_SILU || a.p1) &&
           a.steps <= kP12MaxSteps;
}

hipError_t launch_proj(const ProjArgs& a, int epi, int L, uint32_t blocks,
                       hipStream_t st) {
    if (epi == EPI_SILU && !a.silu8) return hipErrorInvalidValue;  // the SiLU epilogue's table
    if (proj_uses_mfma(a, epi)) {
        switch (epi) {
        case EPI_STORE: return launch_mfma_epi<1, EPI_STORE>(a, st);
        case EPI_RESID: return launch_mfma_epi<1, EPI_RESID>(a, st);
        case EPI_STORE_NORM_IN: return launch_mfma_epi<1, EPI_STORE_NORM_IN>(a, st);
        default: return launch_mfma_epi<2, EPI_SILU>(a, st);
        }
    }
    switch (epi) {
    case EPI_STORE: return launch_proj_epi<EPI_STORE>(a, L, blocks, st);
    case EPI_RESID: return launch_proj_epi<EPI_RESID>(a, L, blocks, st);
    case EPI_STORE_NORM_IN: return launch_proj_epi<EPI_STORE_NORM_IN>(a, L, blocks, st);
    default: return launch_proj_epi<EPI_SILU>(a, L, blocks, st);
    }
}

// Every weight of a 12-bit copy set to 0 (h = 8, l = 0): the nibble words
// of each 768-byte record to 0x88888888, the low bytes to 0.
__global__ void p12_zero_kernel(uint32_t* p, size_t records) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= records * 192) return;
    const size_t r = i / 192, w = i % 192;
    p[r * 192 + w] = w < 128 ? 0u : 0x88888888u;
}

hipError_t launch_p12_zero(uint8_t* p, size_t records, hipStream_t st) {
    const size_t words = records * 192;
    p12_zero_kernel<<<(unsigned)((words + 255) / 256), 256, 0, st>>>((uint32_t*)p, records);
    return hipGetLastError();
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
