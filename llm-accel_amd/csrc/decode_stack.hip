// decode_stack.hip -- decode rows (1-2) through a run of sublayers in one
// persistent launch (see decode_stack.h for the scheme).
//
// The arithmetic is that of the separate kernels: the projections are the
// reference's exact int sums with double rounding (golden_projection,
// host/host_qwen_8x64.cpp:3105-3142) over the tile4x128 weights, lane
// (i, j) of a wavefront owning row i and columns 8j..8j+7 of a k-step and
// the four wavefronts splitting the k-steps; the norms are the constant-gain
// RMSNorm (hidden >= 128); the attention is split_head_body (split_head.h).
// Activation rows go through LDS: every workgroup stages the rows a phase
// reads (device-coherent loads: other workgroups of this launch wrote
// them), normalised on the way in where the phase starts with an RMSNorm.
//
// Ordering: a phase's outputs are written with device-coherent stores;
// each workgroup then waits for all of its memory operations and adds one
// to its counter line of the phase (arrive, coherent.h); a phase that
// reads them polls every line of the group until each holds its target.
// Every workgroup arrives once per phase occurrence, so occurrence k of a
// group is complete when line l holds start + (k + 1) * cnt(l).  Every
// wait is bounded; one that gives up ends the launch (see wait_counts).
#include "decode_stack.h"

#include <algorithm>

#include "attn_common.h"
#include "coherent.h"
#include "fixed_point.h"
#include "proj_common.h"
#include "split_head.h"

namespace llm {
namespace {

constexpr int WPB = 4;                          // wavefronts per workgroup
constexpr int NTH = 64 * WPB;
constexpr int SPW_H = kStackMaxStepsH / WPB;    // k-steps per wavefront, hidden width
constexpr int SPW_I = kStackMaxStepsI / WPB;    // intermediate width
constexpr uint32_t G_QKV = 0, G_ATT = 1, G_O = 2, G_GU = 3, G_DN = 4;
constexpr int D = kStackHeadDim;
static_assert(NTH == 2 * D, "the attention runs on one workgroup of 2 * head_dim threads");

template <int NM, int SPW>
struct WRegs {
    uint4 w[NM][SPW];
};

// The thread index, opaque to the compiler: every lane-dependent offset
// is recomputed where it is used instead of being hoisted out of the step
// loop and held (or spilled) across the whole kernel.
__device__ __forceinline__ uint32_t tid_now() {
    uint32_t t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
// The wavefront's index as a uniform (scalar) value: its k-step range and
// every address derived from it stay in scalar registers.
__device__ __forceinline__ uint32_t wave_id() {
    return __builtin_amdgcn_readfirstlane(tid_now() >> 6);
}

// The k-steps [s0, s0 + cnt) of wavefront `wave` over S steps.
__device__ __forceinline__ void wave_steps(uint32_t S, uint32_t wave, uint32_t& s0,
                                           uint32_t& cnt) {
    s0 = wave * S / WPB;
    cnt = (wave + 1) * S / WPB - s0;
}

// Weight loads of 4-row block b (clamped to the matrix; a repeat is not
// used) over this wavefront's k-steps; loads past its last step repeat
// that step and are masked where they are used.
template <int NM, int SPW>
__device__ __forceinline__ void issue_block(const int16_t* w0, const int16_t* w1, uint32_t S,
                                            uint32_t b, uint32_t nblocks, WRegs<NM, SPW>& R) {
    const uint32_t lane = tid_now() & 63, wave = wave_id();
    const uint32_t i = lane >> 4, j = lane & 15;
    uint32_t s0, cnt;
    wave_steps(S, wave, s0, cnt);
    const uint32_t bb = b < nblocks ? b : nblocks - 1;
#pragma unroll
    for (int m = 0; m < NM; m++) {
        const int16_t* wp =
            (m == 0 ? w0 : w1) + ((size_t)(bb * S + s0) * 4 + i) * 128 + j * 8;
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const uint32_t du = cnt == 0 ? 0 : ((uint32_t)u < cnt ? u : cnt - 1);
            R.w[m][u] = *(const uint4*)(wp + (size_t)du * 512);
        }
    }
}

// This lane's sums of its block row over its wavefront's k-steps,
// activations from LDS xs [RT][ldx]; summed over the 16 lanes of the row.
// The int32 sums widen every LW k-steps (1 or 4: the matrix's widening
// interval allows 8 LW products of any activation).
template <int RT, int NM, int SPW, int LW>
__device__ __forceinline__ void block_dot(const WRegs<NM, SPW>& R, const int16_t* xs,
                                          uint32_t ldx, uint32_t S, int64_t (&acc)[NM][RT]) {
    const uint32_t lane = tid_now() & 63, wave = wave_id();
    const uint32_t j = lane & 15;
    uint32_t s0, cnt;
    wave_steps(S, wave, s0, cnt);
    int32_t part[NM][RT];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < RT; r++) part[m][r] = 0, acc[m][r] = 0;
#pragma unroll
    for (int u = 0; u < SPW; u++) {
        const uint32_t keep = lane_mask((uint32_t)u < cnt);
        const uint32_t du = cnt == 0 ? 0 : ((uint32_t)u < cnt ? u : cnt - 1);
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const uint4 x = *(const uint4*)(xs + (size_t)r * ldx + (s0 + du) * 128 + j * 8);
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const uint4 w = and4(R.w[m][u], keep);
                int32_t p = part[m][r];
                p = dot2(w.x, x.x, p);
                p = dot2(w.y, x.y, p);
                p = dot2(w.z, x.z, p);
                p = dot2(w.w, x.w, p);
                part[m][r] = p;
            }
        }
        if ((u + 1) % LW == 0) {
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int r = 0; r < RT; r++) acc[m][r] += part[m][r], part[m][r] = 0;
        }
        // the LDS reads of at most four steps ahead: hoisting all of them
        // would hold SPW x 4 registers more
        if ((u + 1) % 4 == 0) __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < RT; r++) {
            acc[m][r] += part[m][r];
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) acc[m][r] += __shfl_xor(acc[m][r], off, 64);
        }
}

// The block's exact sums: thread et < 4 RT gets those of block row et / RT,
// activation row et % RT (red: LDS [WPB][NM][4][RT], alternated by the
// caller between consecutive blocks so that one barrier suffices).
template <int RT, int NM>
__device__ __forceinline__ void block_reduce(int64_t* red, const int64_t (&acc)[NM][RT],
                                             int64_t (&tot)[NM]) {
    const uint32_t lane = tid_now() & 63, wave = wave_id();
    const uint32_t i = lane >> 4, j = lane & 15;
    if (j == 0) {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < RT; r++) red[((wave * NM + m) * 4 + i) * RT + r] = acc[m][r];
    }
    lds_barrier();
    const uint32_t et = tid_now();
#pragma unroll
    for (int m = 0; m < NM; m++) {
        tot[m] = 0;
        if (et < 4 * RT) {
            const uint32_t ii = et / RT, r = et % RT;
#pragma unroll
            for (int ww = 0; ww < WPB; ww++) tot[m] += red[((ww * NM + m) * 4 + ii) * RT + r];
        }
    }
}

// Rows [rows][kvalid] of src (row stride ld) into LDS xs [RT][ldx] over kpad
// columns (zero past kvalid and in rows >= rows), with device-coherent
// loads, all issued before the first is used; normalised with a constant
// gain when gamma != null (the norm table is padded to whole k-steps).
template <int RT, int NIT, bool NORM>
__device__ __forceinline__ void stage_rows(int16_t* xs, uint32_t ldx, const int16_t* src,
                                           uint32_t ld, uint32_t rows, uint32_t kpad,
                                           uint32_t kvalid, const int16_t* gamma,
                                           int32_t gain) {
    const uint32_t cpr = kpad / 8;  // 16-byte chunks per row
    uint4 v[NIT], g[NORM ? NIT : 1];
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const uint32_t u = tid_now() + it * NTH;
        const uint32_t r = u / cpr, c = (u % cpr) * 8;
        const bool ok = u < RT * cpr && r < rows && c < kvalid;
        v[it] = ld_coherent16(src + (ok ? (size_t)r * ld + c : 0));
        v[it] = and4(v[it], lane_mask(ok));
        if (NORM) g[NORM ? it : 0] = *(const uint4*)(gamma + (u < RT * cpr ? c : 0));
    }
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const uint32_t u = tid_now() + it * NTH;
        if (u < RT * cpr) {
            const uint32_t r = u / cpr, c = (u % cpr) * 8;
            *(uint4*)(xs + (size_t)r * ldx + c) = NORM ? norm8(v[it], g[NORM ? it : 0], gain)
                                                       : v[it];
        }
    }
    lds_barrier();
}

// Bytes of the LDS shared by the staged rows and the attention.
template <int RT>
constexpr size_t smem_bytes() {
    const size_t rows = (size_t)RT * kStackMaxStepsI * 128 * 2;
    const size_t att = sizeof(SplitSmem<D>);
    return rows > att ? rows : att;
}

template <int RT, int LW>
__global__ __launch_bounds__(NTH, 2) void decode_stack_kernel(StackArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[smem_bytes<RT>()];
    __shared__ int64_t red[2][WPB * 2 * 4 * RT];
    __shared__ uint32_t flag;
    __shared__ __attribute__((aligned(16))) int16_t e8s[2056];  // Q8.8 exp table (SiLU)
    int16_t* const xs = (int16_t*)smem;
    SplitSmem<D>& sm = *(SplitSmem<D>*)smem;

    const uint32_t w = blockIdx.x, nwg = gridDim.x;
    const uint32_t line = w % kStackLines;
    const uint32_t R = a.rows;
    const uint32_t SH = a.Hp / 128, SI = a.Ip / 128;
    const uint32_t nbq = (a.Nqkv + 3) / 4, nbo = (a.H + 3) / 4, nbg = (a.I + 3) / 4;
    const uint32_t na = R * a.at.num_heads;
    uint32_t occ[kStackGroups] = {0, 0, 0, 0, 0};
    uint32_t par = 0;  // parity of the reduction buffer

    auto wait_group = [&](uint32_t g) -> bool {
        const uint32_t k = a.occ[g] + occ[g];
        return wait_counts(
            a.sync + g * kStackLines * kStackStride, kStackStride, kStackLines,
            [&](uint32_t l) {
                const uint32_t cnt = nwg / kStackLines + (l < nwg % kStackLines ? 1u : 0u);
                return a.start + k * cnt;
            },
            a.wait_limit, a.abort, a.host_abort, &flag);
    };
    auto arrive_group = [&](uint32_t g) {
        arrive(a.sync + (g * kStackLines + line) * kStackStride);
        occ[g]++;
    };

    uint32_t prev = kStackGroups;  // the group the next step's input comes from

    // the SiLU exp table goes to LDS (the gate|up epilogue looks it up per
    // output, between one block's reduction and the next): its loads are
    // issued here, the LDS writes follow the first staged rows
    uint4 e8v[2];
    bool e8_pending = true;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const uint32_t c = tid_now() + u * NTH;
        e8v[u] = *(const uint4*)(a.exp8 + 8 * (c < 257 ? c : 0));
    }
    auto e8_commit = [&] {
        if (!e8_pending) return;
        e8_pending = false;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const uint32_t c = tid_now() + u * NTH;
            if (c < 257) *(uint4*)(e8s + 8 * c) = e8v[u];
        }
    };

    // One iteration: an attention sublayer and, when one follows, its FFN
    // sublayer (whose first gate|up blocks stream during the attention), or
    // an FFN sublayer alone.  Every prefetch register set lives within one
    // iteration.
    for (uint32_t s = 0; s < a.nsteps; s++) {
        WRegs<2, SPW_H> ga, gb;
        if (!a.steps[s].ffn) {
            // ---------------- attention sublayer ----------------
            const StackStep st = a.steps[s];
            const size_t lo = (size_t)st.layer * a.layer_stride;
            const int16_t* wq = a.w[0] + lo;
            const int16_t* wo = a.w[1] + lo;
            {
                WRegs<1, SPW_H> q0, q1;
                issue_block<1, SPW_H>(wq, nullptr, SH, w, nbq, q0);
                issue_block<1, SPW_H>(wq, nullptr, SH, w + nwg, nbq, q1);
                if (prev < kStackGroups && !wait_group(prev)) return;
                stage_rows<RT, RT, true>(xs, a.Hp, st.in, a.Hp, R, a.Hp, a.H,
                                         a.norms + (size_t)(2 * st.layer) * a.H, a.gain);
                e8_commit();
                auto qkv_block = [&](const WRegs<1, SPW_H>& q, uint32_t b) {
                    if (b >= nbq) return;
                    int64_t acc[1][RT], tot[1];
                    block_dot<RT, 1, SPW_H, LW>(q, xs, a.Hp, SH, acc);
                    block_reduce<RT, 1>(red[par], acc, tot);
                    par ^= 1;
                    const uint32_t et = tid_now(), n = b * 4 + et / RT, r = et % RT;
                    if (et < 4 * RT && r < R && n < a.Nqkv)
                        st_coherent(&a.qkv[(size_t)r * a.Nqkv + n],
                                    fx_narrow_projection(tot[0]));
                };
                qkv_block(q0, w);
                qkv_block(q1, w + nwg);
            }
            arrive_group(G_QKV);

            if (w < na) {
                AttnArgs at = a.at;
                const size_t kvo = (size_t)st.layer * a.kv_layer_stride;
                at.kcache = a.at.kcache + kvo;
                at.vcache = a.at.vcache + kvo;
                if (!split_head_body<D, true>(at, w / at.num_heads, w % at.num_heads, sm,
                                              [&] { return wait_group(G_QKV); }))
                    return;
            }
            arrive_group(G_ATT);

            // the O weights and the first gate|up blocks of the FFN sublayer
            // that follows (else of this layer, unused) stream while the
            // attention runs
            const bool pair = s + 1 < a.nsteps && a.steps[s + 1].ffn;
            const size_t ln = (size_t)a.steps[pair ? s + 1 : s].layer * a.layer_stride;
            WRegs<1, SPW_H> o0, o1;
            issue_block<1, SPW_H>(wo, nullptr, SH, w, nbo, o0);
            issue_block<1, SPW_H>(wo, nullptr, SH, w + nwg, nbo, o1);
            issue_block<2, SPW_H>(a.w[2] + ln, a.w[3] + ln, SH, w, nbg, ga);
            if (!wait_group(G_ATT)) return;
            stage_rows<RT, RT, false>(xs, a.Hp, a.attn, a.Hp, R, a.Hp, a.H, nullptr, 0);
            auto o_block = [&](const WRegs<1, SPW_H>& q, uint32_t b) {
                if (b >= nbo) return;
                const uint32_t et = tid_now(), n = b * 4 + et / RT, r = et % RT;
                const bool mine = et < 4 * RT && r < R && n < a.H;
                int32_t res = 0;
                if (mine) res = ld_coherent(&st.in[(size_t)r * a.Hp + n]);
                int64_t acc[1][RT], tot[1];
                block_dot<RT, 1, SPW_H, LW>(q, xs, a.Hp, SH, acc);
                block_reduce<RT, 1>(red[par], acc, tot);
                par ^= 1;
                if (mine)
                    st_coherent(&st.out[(size_t)r * a.Hp + n],
                                fx_sat16((int32_t)fx_narrow_projection(tot[0]) + res));
            };
            o_block(o0, w);
            o_block(o1, w + nwg);
            arrive_group(G_O);
            prev = G_O;
            issue_block<2, SPW_H>(a.w[2] + ln, a.w[3] + ln, SH, w + nwg, nbg, gb);
            if (!pair) continue;
            s++;  // the FFN sublayer of this iteration
        } else {
            const size_t lo = (size_t)a.steps[s].layer * a.layer_stride;
            issue_block<2, SPW_H>(a.w[2] + lo, a.w[3] + lo, SH, w, nbg, ga);
            issue_block<2, SPW_H>(a.w[2] + lo, a.w[3] + lo, SH, w + nwg, nbg, gb);
        }
        // ---------------- FFN sublayer ----------------
        const StackStep st = a.steps[s];
        const size_t lo = (size_t)st.layer * a.layer_stride;
        const int16_t* wg = a.w[2] + lo;
        const int16_t* wu = a.w[3] + lo;
        const int16_t* wd = a.w[4] + lo;
        if (prev < kStackGroups && !wait_group(prev)) return;
        stage_rows<RT, RT, true>(xs, a.Hp, st.in, a.Hp, R, a.Hp, a.H,
                                 a.norms + (size_t)(2 * st.layer + 1) * a.H, a.gain);
        e8_commit();
        lds_barrier();  // the table before the first epilogue reads it
        // this workgroup's blocks b = w + k nwg, k < ngu, two in flight
        const uint32_t ngu = w < nbg ? (nbg - w + nwg - 1) / nwg : 0;
        auto gu_block = [&](const WRegs<2, SPW_H>& q, uint32_t k) {
            if (k >= ngu) return;
            const uint32_t b = w + k * nwg;
            int64_t acc[2][RT], tot[2];
            block_dot<RT, 2, SPW_H, LW>(q, xs, a.Hp, SH, acc);
            block_reduce<RT, 2>(red[par], acc, tot);
            par ^= 1;
            const uint32_t et = tid_now(), n = b * 4 + et / RT, r = et % RT;
            if (et < 4 * RT && r < R && n < a.I) {
                const int16_t g = fx_narrow_projection(tot[0]);
                const int16_t u = fx_narrow_projection(tot[1]);
                st_coherent(&a.act[(size_t)r * a.Ip + n],
                            fx_sat16(fx_rnd((int64_t)fx_silu(g, e8s) * u, 8)));
            }
        };
        const uint32_t last = ngu ? ngu - 1 : 0;
        for (uint32_t k = 0; k < ngu; k += 2) {
            gu_block(ga, k);
            issue_block<2, SPW_H>(wg, wu, SH, w + std::min(k + 2, last) * nwg, nbg, ga);
            gu_block(gb, k + 1);
            issue_block<2, SPW_H>(wg, wu, SH, w + std::min(k + 3, last) * nwg, nbg, gb);
        }
        arrive_group(G_GU);
        // the down projection's weights stream while the others finish
        WRegs<1, SPW_I> dw;
        issue_block<1, SPW_I>(wd, nullptr, SI, w, nbo, dw);
        if (!wait_group(G_GU)) return;
        stage_rows<RT, (RT * kStackMaxStepsI * 16 + NTH - 1) / NTH, false>(
            xs, a.Ip, a.act, a.Ip, R, a.Ip, a.I, nullptr, 0);
        const bool fin = a.final_out && s + 1 == a.nsteps;
        for (uint32_t b = w; b < nbo; b += nwg) {
            const uint32_t et = tid_now(), n = b * 4 + et / RT, r = et % RT;
            const bool mine = et < 4 * RT && r < R && n < a.H;
            int32_t res = 0, gf = 0;
            if (mine) {
                res = ld_coherent(&st.in[(size_t)r * a.Hp + n]);
                if (fin) gf = a.norms[(size_t)(2 * a.L) * a.H + n];
            }
            // rows >= R of the final-norm buffer copy the input pair
            const uint32_t fe = et - 64, fr = fe / 4, fn = b * 4 + fe % 4;
            if (fin && et >= 64 && et < 96 && fr >= R && fn < a.H)
                a.final_out[(size_t)fr * a.Hp + fn] = ld_coherent(&st.in[(size_t)fr * a.Hp + fn]);
            int64_t acc[1][RT], tot[1];
            block_dot<RT, 1, SPW_I, LW>(dw, xs, a.Ip, SI, acc);
            block_reduce<RT, 1>(red[par], acc, tot);
            par ^= 1;
            if (b + nwg < nbo) issue_block<1, SPW_I>(wd, nullptr, SI, b + nwg, nbo, dw);
            if (mine) {
                const int16_t y = fx_sat16((int32_t)fx_narrow_projection(tot[0]) + res);
                st_coherent(&st.out[(size_t)r * a.Hp + n], y);
                if (fin)
                    a.final_out[(size_t)r * a.Hp + n] =
                        fx_sat16(fx_rnd((int64_t)y * a.gain * gf, 16));
            }
        }
        arrive_group(G_DN);
        prev = G_DN;
    }
}

template <int RT>
static int stack_occupancy() {
    int o4 = 0, o1 = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o4, decode_stack_kernel<RT, 4>, NTH, 0) !=
            hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&o1, decode_stack_kernel<RT, 1>, NTH, 0) !=
            hipSuccess)
        return 0;
    return std::min(o4, o1);
}

}  // namespace

uint32_t stack_workgroups(int cus, uint32_t rows) {
    const int per_cu = rows <= 1 ? stack_occupancy<1>() : stack_occupancy<2>();
    return (uint32_t)(std::min(per_cu, 2) * cus);
}

hipError_t launch_decode_stack(const StackArgs& a, uint32_t nwg, int lw, hipStream_t st) {
    if (a.rows <= 1) {
        if (lw >= 4) decode_stack_kernel<1, 4><<<nwg, NTH, 0, st>>>(a);
        else decode_stack_kernel<1, 1><<<nwg, NTH, 0, st>>>(a);
    } else {
        if (lw >= 4) decode_stack_kernel<2, 4><<<nwg, NTH, 0, st>>>(a);
        else decode_stack_kernel<2, 1><<<nwg, NTH, 0, st>>>(a);
    }
    return hipGetLastError();
}

}  // namespace llm
