// noalloc.hip -- the LM-head argmax for callers that cannot allocate.
//
// llm_lm_head_argmax_static() computes what llm_lm_head_argmax() computes
// (model_data_t::lm_head_argmax, host/host_qwen_8x64.cpp:937-969: the exact
// int64 score of every vocabulary row, strict > over increasing index) on
// memory the caller owns: the table in the reference's row-major
// [vocab][hidden] form, the hidden rows and the outputs, all in device
// memory, on the caller's stream.  It calls no allocating routine; its one
// scratch buffer, the per-row argmax keys, is the file-scope array
// `scratch` below, whose device address is looked up once per device.
//
// Three launches in stream order: clear the keys, the argmax (each
// workgroup's best goes into one 64-bit atomicMax per row), and the decode
// of the keys into tokens and scores.  Every call on a device shares that
// device's keys, so calls that overlap on one device race.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "kernels.h"
#include "llm_accel.h"
#include "proj_common.h"

namespace {

constexpr uint32_t kStaticRows = 8;           // rows per call
constexpr uint32_t kStaticHiddenMax = 16384;  // keeps |score| < 2^45 in the key
constexpr int kMaxDevices = 64;

// Argmax keys of up to 8 rows: 64 bytes per device, held until the
// process ends.  Host code uses the address from hipGetSymbolAddress, never
// this name.
static __device__ __align__(256) unsigned long long scratch[kStaticRows];

std::mutex g_scratch_mu;
unsigned long long* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device.
int scratch_of_current_device(unsigned long long** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return llm::set_last_error(LLM_E_HIP, hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return llm::set_last_error(LLM_E_ARG, "device id beyond the static scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return llm::set_last_error(
                LLM_E_HIP, (std::string("hipGetSymbolAddress(scratch): ") +
                            hipGetErrorString(e)).c_str());
        g_scratch_ptr[dev] = (unsigned long long*)p;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

__global__ void static_keys_clear_kernel(unsigned long long* keys) {
    if (threadIdx.x < kStaticRows) keys[threadIdx.x] = 0;
}

// Row-major table: wavefront `wave` of a workgroup scores vocabulary rows
// v = 4 * blockIdx.x + wave, 4 * gridDim.x apart; lane l reads the 16-byte
// chunks l, l + 64, ... of the row (coalesced 1 KiB per wavefront load) and
// the same chunks of each activation row.  Products are exact in int32
// (|x w| <= 2^30) and summed in int64.
template <int RT>
__global__ __launch_bounds__(256) void lm_argmax_rows_kernel(
    const int16_t* __restrict__ w, uint32_t vocab, uint32_t chunks,
    const int16_t* __restrict__ x, uint32_t ldx, uint32_t rows,
    unsigned long long* keys) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    unsigned long long best[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) best[r] = 0;
    for (uint32_t v = blockIdx.x * 4 + wave; v < vocab; v += gridDim.x * 4) {
        const uint4* wp = (const uint4*)(w + (size_t)v * chunks * 8);
        int64_t acc[RT];
#pragma unroll
        for (int r = 0; r < RT; r++) acc[r] = 0;
        for (uint32_t c = lane; c < chunks; c += 64) {
            const uint4 wv = wp[c];
#pragma unroll
            for (int r = 0; r < RT; r++) {
                // rows beyond `rows` read row 0 (in bounds; ignored)
                const uint4 xv =
                    ((const uint4*)(x + (size_t)(r < (int)rows ? r : 0) * ldx))[c];
                acc[r] += llm::dot2_wide(wv.x, xv.x) + llm::dot2_wide(wv.y, xv.y) +
                          llm::dot2_wide(wv.z, xv.z) + llm::dot2_wide(wv.w, xv.w);
            }
        }
#pragma unroll
        for (int r = 0; r < RT; r++) {
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) acc[r] += __shfl_xor(acc[r], off, 64);
            const unsigned long long k = llm::argmax_key(acc[r], v);
            if (k > best[r]) best[r] = k;
        }
    }
    __shared__ unsigned long long wbest[4][RT];
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RT; r++) wbest[wave][r] = best[r];
    }
    __syncthreads();
    if (threadIdx.x < RT && threadIdx.x < rows) {
        const int r = threadIdx.x;
        unsigned long long k = 0;
        for (int ww = 0; ww < 4; ww++) k = wbest[ww][r] > k ? wbest[ww][r] : k;
        atomicMax(&keys[r], k);
    }
}

__global__ void static_keys_decode_kernel(const unsigned long long* keys, uint32_t rows,
                                          uint32_t* tokens, int64_t* scores) {
    const uint32_t r = threadIdx.x;
    if (r >= rows) return;
    const unsigned long long k = keys[r];
    tokens[r] = llm::kArgmaxVocabMax - (uint32_t)(k & llm::kArgmaxVocabMax);
    if (scores) scores[r] = (int64_t)(k >> 18) - ((int64_t)1 << 45);
}

template <int RT>
hipError_t launch_rows(const int16_t* w, uint32_t vocab, uint32_t chunks, const int16_t* x,
                       uint32_t ldx, uint32_t rows, unsigned long long* keys,
                       hipStream_t st) {
    uint32_t grid = (vocab + 3) / 4;
    if (grid > 2048) grid = 2048;
    lm_argmax_rows_kernel<RT><<<grid, 256, 0, st>>>(w, vocab, chunks, x, ldx, rows, keys);
    return hipGetLastError();
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace

extern "C" int llm_lm_head_argmax_static(const int16_t* table, uint32_t vocab,
                                         uint32_t hidden, const int16_t* rows,
                                         uint32_t ld, uint32_t row_count,
                                         uint32_t* tokens, int64_t* scores,
                                         void* stream) {
    // Sizes first, before any HIP call.
    if (!table || !rows || !tokens)
        return llm::set_last_error(LLM_E_ARG, "null table, rows or tokens");
    if (row_count == 0 || row_count > kStaticRows)
        return llm::set_last_error(LLM_E_ARG,
                                   "row_count must be 1..8 (the static scratch holds 8 keys)");
    if (vocab == 0 || vocab > llm::kArgmaxVocabMax)
        return llm::set_last_error(LLM_E_ARG, "vocab must be 1..262143");
    if (hidden == 0 || hidden > kStaticHiddenMax || hidden % 8 != 0)
        return llm::set_last_error(LLM_E_ARG,
                                   "hidden must be a multiple of 8 and at most 16384");
    if (ld < hidden || ld % 8 != 0)
        return llm::set_last_error(LLM_E_ARG, "ld must be >= hidden and a multiple of 8");
    if (!aligned(table, 16) || !aligned(rows, 16) || !aligned(tokens, 4) ||
        (scores && !aligned(scores, 8)))
        return llm::set_last_error(LLM_E_ARG,
                                   "table and rows must be 16-byte aligned device memory");
    unsigned long long* keys = nullptr;
    if (int rc = scratch_of_current_device(&keys)) return rc;
    hipStream_t st = (hipStream_t)stream;
    static_keys_clear_kernel<<<1, 64, 0, st>>>(keys);
    hipError_t e = hipGetLastError();
    const uint32_t chunks = hidden / 8;
    if (e == hipSuccess) {
        if (row_count <= 1) e = launch_rows<1>(table, vocab, chunks, rows, ld, row_count, keys, st);
        else if (row_count <= 2) e = launch_rows<2>(table, vocab, chunks, rows, ld, row_count, keys, st);
        else if (row_count <= 4) e = launch_rows<4>(table, vocab, chunks, rows, ld, row_count, keys, st);
        else e = launch_rows<8>(table, vocab, chunks, rows, ld, row_count, keys, st);
    }
    if (e == hipSuccess) {
        static_keys_decode_kernel<<<1, 64, 0, st>>>(keys, row_count, tokens, scores);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return llm::set_last_error(LLM_E_HIP, hipGetErrorString(e));
    return 0;
}
