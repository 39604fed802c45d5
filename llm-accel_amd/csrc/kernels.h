// kernels.h -- launch interface of the HIP kernels (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llm {

// Epilogues: STORE the narrowed sums; RESID add a residual row (and
// optionally write a constant-gain RMSNorm of the result); SILU store
// silu(gate) * up; STORE_NORM_IN like STORE on inputs normalised while they
// are loaded (constant-gain RMSNorm of the raw rows).
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_STORE_NORM_IN = 3 };

// Rows per weight block and columns per k-step of the "tile4x128" layout.
constexpr uint32_t kBlockRows = 4;
constexpr uint32_t kStepCols = 128;
constexpr uint32_t kTile = 64;  // attention tile = KV page (positions)

struct ProjArgs {
    const int16_t* w0;  // tile4x128 weights (gate for EPI_SILU)
    const int16_t* w1;  // up weights (EPI_SILU only)
    uint32_t steps;     // K_pad / 128
    const int16_t* x;   // activations [rows][ldx], ldx >= K_pad
    uint32_t ldx;
    int16_t* out;       // [rows][ldo]
    uint32_t ldo;
    const int16_t* res; // residual [rows][ldr] (EPI_RESID)
    uint32_t ldr;
    uint32_t n;         // valid output columns
    uint32_t rows;      // active rows (1..8)
    const int16_t* exp8;    // Q8.8 exp table, x = -2048..0
    const uint32_t* silu8;  // EPI_SILU: per exp-table entry e, e | recip(256 + e) << 16
    // EPI_RESID only, optional: RMSNorm of the output rows with a constant
    // gain (norm_out[r][n] = rnd(out * gain * gamma[n], 16)).
    int16_t* norm_out;
    uint32_t ldn;
    const int16_t* norm_gamma;
    int32_t norm_gain;
    // EPI_RESID, optional: the final RMSNorm (constant gain norm_gain) of
    // the output rows into final_out [8][ldn]; its rows rows..7 copy the
    // same rows of the residual, so final_out holds a whole pair.
    int16_t* final_out;
    const int16_t* final_gamma;
    // EPI_STORE_NORM_IN: x[r][k] is replaced by rnd(x * in_gain * in_gamma[k],
    // 16); in_gamma is read in whole k-steps (the table is padded), and past
    // in_cols the rows themselves are 0.
    const int16_t* in_gamma;
    int32_t in_gain;
    uint32_t in_cols;
    // Byte-plane copies of the weights for the matrix-core path ("mfma16x64",
    // see proj_mfma_kernel) and their per-output (sum hi, sum lo) pairs;
    // null when absent.  kq = K_pad / 64, nc = N_pad / 16.
    const int8_t* mf0;
    const int8_t* mf1;
    const int32_t* ms0;
    const int32_t* ms1;
    uint32_t kq, nc;
    // Split of the K chunks over workgroups (matrix-core path): partial
    // sums of part p of chunk c go to mf_part, the last workgroup of a
    // chunk to arrive (mf_count) finishes it.
    int32_t* mf_part;
    uint32_t* mf_count;
    // 12-bit copies of w0 / w1 ("p12", see proj_p12_kernel), for matrices
    // whose weights all lie in [-2048, 2047]; null when absent.
    const uint8_t* p0;
    const uint8_t* p1;
    // The matrix-core path reads p0 (and p1) instead of the byte planes
    // when set and present (proj_mfma12_kernel).
    uint32_t mf_p12;
    // Sparse corrections of the 12-bit copies p0 / p1 (null: none): per
    // output row kCorrSlots words (k << 16) | (uint16) delta, delta =
    // w - clamp(w, -2048, 2047) for the row's weights outside 12 bits, whose
    // copy holds the clamped value; unused words are 0.
    const uint32_t* corr0;
    const uint32_t* corr1;
};
constexpr uint32_t kCorrSlots = 4;
// Bytes of the p12 copy per 4-row block and k-step.
constexpr uint32_t kP12Step = 768;
// Sets every weight of a p12 copy of `records` records to 0.
hipError_t launch_p12_zero(uint8_t* p, size_t records, hipStream_t st);

// Matrix-core layout: record (c, q) of 2048 bytes holds outputs 16c..16c+15
// and inputs 64q..64q+63: bytes [0, 1024) the high bytes w >> 8, bytes
// [1024, 2048) the low bytes (w & 255) - 128, both as int8; lane l, byte b
// of a plane is output 16c + l % 16, input 64q + 16 (l / 16) + b.  Records
// are ordered [c][q].
constexpr uint32_t kMfRows = 16;
constexpr uint32_t kMfCols = 64;
constexpr uint32_t kMfRecord = 2048;

// Records `msg` as the text llm_last_error() returns; returns `code`.
int set_last_error(int code, const char* msg);

hipError_t launch_copy(const uint4* src, uint4* dst, size_t n16,
                       hipStream_t st);

// LM-head argmax: for each of `rows` activation rows x[r] (stride ldx),
// argmax over v < n of the exact int64 sum_k x[r][k] * W[v][k] (tile4x128
// weights w with `steps` k-steps, widening interval L), first index on
// ties.  keys[r] must be zero on entry; it receives
// ((score + 2^45) << 18) | (2^18 - 1 - v) of the winner.
constexpr uint32_t kArgmaxVocabMax = (1u << 18) - 1;
__device__ __forceinline__ unsigned long long argmax_key(int64_t score, uint32_t v) {
    return ((unsigned long long)(score + ((int64_t)1 << 45)) << 18) |
           (unsigned long long)(kArgmaxVocabMax - v);
}
hipError_t launch_lm_argmax(const int16_t* w, uint32_t steps, uint32_t n,
                            const int16_t* x, uint32_t ldx, uint32_t rows, int L,
                            unsigned long long* keys, hipStream_t st);
// Blocks of at least kMfMinRows rows run on the matrix cores when the
// byte-plane layout is present; others on the VALU dot2 kernel.
#ifndef LLM_MF_MIN_ROWS
#define LLM_MF_MIN_ROWS 3
#endif
constexpr uint32_t kMfMinRows = LLM_MF_MIN_ROWS;
// Workgroup shape of the matrix-core kernel for a matrix: KS wavefronts
// per workgroup, P workgroups per 16-output chunk.
struct MfSplit {
    uint32_t ks, parts;
};
MfSplit mf_split(uint32_t nc, uint32_t kq);
// The same for the matrix-core kernel over the 12-bit copy, in k-steps,
// and whether a launch of the matrix-core path takes that kernel.
MfSplit mf12_split(uint32_t nc, uint32_t steps, uint32_t nm);
bool proj_mfma_reads_p12(const ProjArgs& a, int epi);
// int32 words of partial sums per (chunk, part) record.
constexpr uint32_t mf_part_words(uint32_t nm) { return nm * 2 * 256 + 32; }
bool proj_uses_mfma(const ProjArgs& a, int epi);
// Blocks of one or two rows read the p12 copy when every matrix of the
// launch has one and K is at most kP12MaxSteps k-steps.
constexpr uint32_t kP12MaxSteps = 128;
bool proj_uses_p12(const ProjArgs& a, int epi);
hipError_t launch_proj(const ProjArgs& a, int epi, int L, uint32_t blocks,
                       hipStream_t st);
// RMSNorm of `rows` rows; const_gain > 0 selects the elementwise kernel
// (the gain does not depend on the data when hidden >= 128).
hipError_t launch_rmsnorm(const int16_t* x, uint32_t ldx, const int16_t* gamma,
                          uint32_t cols, int16_t* y, uint32_t ldy, uint32_t rows,
                          int32_t const_gain, hipStream_t st);

}  // namespace llm
