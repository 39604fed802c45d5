// coherent.h -- hand-off of partial results between workgroups of one
// launch without device-wide cache flushes.
//
// A workgroup that publishes partial results for another workgroup of the
// same launch writes them with device-coherent stores (sc1: performed at
// the device coherence point, not held in one XCD's L2), waits until they
// have completed, and only then increments the arrival counter.  The
// workgroup that arrives last reads them with device-coherent loads.  A
// __threadfence() would instead write back and invalidate the whole L2 of
// the XCD for every workgroup, which dominates when hundreds of workgroups
// publish.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llm {

template <typename T>
__device__ __forceinline__ void st_coherent(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_coherent(const T* p) {
    return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every thread's coherent stores have completed; then one arrival per
// workgroup on *counter.  Returns (uniformly) whether this workgroup is the
// last of `expected` to arrive; that workgroup also resets the counter.
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t expected,
                                            uint32_t* lds_flag) {
    __builtin_amdgcn_s_waitcnt(0);  // all counters: stores performed
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        const bool last = prev == expected - 1;
        if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *lds_flag = last;
    }
    __syncthreads();
    return *lds_flag != 0;
}

}  // namespace llm
