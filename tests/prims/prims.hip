// prims.hip -- test-only evaluation of the library's fixed-point
// primitives on the GPU (tests/test_gpu_primitives.py compares them with
// the oracle over whole input ranges).  Built from the library's own
// headers, so the code under test is the code the kernels inline.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_common.h"
#include "fixed_point.h"

namespace {

enum Which {
    P_RECIP = 0,    // fx_recip(x), x int16
    P_RSQRT = 1,    // fx_rsqrt(x), x int32 (Q16.16)
    P_SILU = 2,     // fx_silu(x, e8), x int16
    P_INV_SUM = 3,  // fx_inv_sum(x), x int32
    P_TERM = 4,     // one product term as the QK / PV banks form it: x = a | b << 16
    P_PROB = 5,     // prob(e14, x), x int32 <= 0
};

__global__ void prims_kernel(int which, const int32_t* in, int32_t* out, uint32_t n,
                             const int16_t* table) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += gridDim.x * blockDim.x) {
        const int32_t x = in[i];
        int32_t y = 0;
        switch (which) {
        case P_RECIP: y = fx_recip((int16_t)x); break;
        case P_RSQRT: y = fx_rsqrt(x); break;
        case P_SILU: y = fx_silu((int16_t)x, table); break;
        case P_INV_SUM: y = fx_inv_sum(x); break;
        case P_TERM: {
            // b staged clamped to [-2048, 2048]; a staged 2048 adds c(a)
            // (the kernels' clamp4 / sat_mask / sat_corr)
            const uint32_t a = (uint32_t)x & 0xffffu;
            const uint32_t b = llm::clamp_word((uint32_t)x >> 16);
            const uint32_t ca = (uint16_t)(int16_t)llm::sat_corr((int16_t)a);
            y = llm::dot2(b, a, 0) + llm::dot2(llm::sat_mask(b), ca, 0);
            break;
        }
        // the kernels call prob with x <= 0 only (score - running max);
        // x > 0 would index past the 2049-entry table
        case P_PROB: y = x <= 0 ? llm::prob(table, x) : 0; break;
        default: break;
        }
        out[i] = y;
    }
}

}  // namespace

// Host buffers in and out (n values), `table` (table_len int16, the exp
// table the primitive reads, or NULL).  Returns 0, or a hipError_t.
extern "C" int prims_eval(int which, const int32_t* in, int32_t* out, uint32_t n,
                          const int16_t* table, uint32_t table_len) {
    if (which < P_RECIP || which > P_PROB || n == 0 || !in || !out) return -1;
    if ((which == P_SILU || which == P_PROB) && (!table || table_len < 2049)) return -1;
    int32_t *din = nullptr, *dout = nullptr;
    int16_t* dt = nullptr;
    hipError_t e = hipMalloc((void**)&din, (size_t)n * 4);
    if (e == hipSuccess) e = hipMalloc((void**)&dout, (size_t)n * 4);
    if (e == hipSuccess) e = hipMalloc((void**)&dt, 4096 * 2);
    if (e == hipSuccess) e = hipMemset(dt, 0, 4096 * 2);
    if (e == hipSuccess && table)
        e = hipMemcpy(dt, table, (size_t)(table_len < 4096 ? table_len : 4096) * 2,
                      hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(din, in, (size_t)n * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        prims_kernel<<<1024, 256>>>(which, din, dout, n, dt);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(out, dout, (size_t)n * 4, hipMemcpyDeviceToHost);
    if (din) (void)hipFree(din);
    if (dout) (void)hipFree(dout);
    if (dt) (void)hipFree(dt);
    return (int)e;
}
