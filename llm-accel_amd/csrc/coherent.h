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
//
// Why relaxed atomics suffice (an argument at the level of the gfx9 ISA,
// not of the C++ memory model):
//   - producer: every value is a relaxed agent-scope atomic store
//     (global_store ... sc1).  s_waitcnt vmcnt(0) returns only when the
//     memory system has acknowledged each of the wavefront's stores, i.e.
//     when each is performed at the coherence point; __syncthreads() then
//     puts every wavefront of the workgroup past its own wait before one
//     thread issues the counter's atomic add.  The add is therefore issued
//     after the values are globally visible at the coherence point;
//   - consumer: the counter is polled with relaxed agent-scope atomic
//     loads (sc1: read at the coherence point, not from a stale L2 line).
//     The value loads are issued only after the poll's result has decided a
//     branch; the hardware issues a wavefront's memory instructions in
//     order and does not execute past an unresolved branch, and both kinds
//     of load are served by the same coherence point, so they see the
//     values written before the counter reached its target.
// The release / acquire formulation would make the compiler surround each
// counter atomic with write-back / invalidation of the XCD's whole L2
// (agent scope spans XCDs whose L2s are not coherent with each other),
// which is the per-workgroup cost this scheme avoids.
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

// 16 bytes read with two device-coherent 8-byte loads (p 16-byte aligned).
__device__ __forceinline__ uint4 ld_coherent16(const int16_t* p) {
    const uint64_t lo = ld_coherent((const uint64_t*)p);
    const uint64_t hi = ld_coherent((const uint64_t*)p + 1);
    return make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32));
}

// Every thread's coherent stores have completed; then one arrival per
// workgroup on each of the `copies` counters counter[0], counter[stride], ...
__device__ __forceinline__ void arrive(uint32_t* counter, uint32_t copies = 1,
                                       uint32_t stride = 0) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x < copies)
        __hip_atomic_fetch_add(counter + threadIdx.x * stride, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

// Default bound of one wait, in ticks of the 100 MHz constant clock
// (20 ms): a wait that legitimately ends takes microseconds.
constexpr uint32_t kWaitLimitTicks = 2000000;

// Waits until counter[l * stride] has reached target(l) for every l < n
// (n <= 64; counters grow across launches and are compared modulo 2^32),
// the workgroup held at a barrier while wavefront 0 polls, lane l reading
// counter l.  Every wait ends: past `limit` ticks, or when another
// workgroup has given up (*abort != 0), it returns false (uniformly) and
// the workgroup must leave; the one that gives up sets *abort and
// *host_abort (host-visible memory read by the library after its next
// synchronisation).  Progress needs the awaited workgroups to be
// dispatched: the launcher only uses this in grids whose waiting
// workgroups alone cannot fill the device.
template <typename Target>
__device__ __forceinline__ bool wait_counts(const uint32_t* counter, uint32_t stride, uint32_t n,
                                            Target&& target, uint32_t limit, uint32_t* abort,
                                            uint32_t* host_abort, uint32_t* lds_flag) {
    if (threadIdx.x < 64) {
        const uint32_t l = threadIdx.x;
        const bool mine = l < n;
        const uint32_t want = mine ? target(l) : 0u;
        const uint32_t* p = counter + (mine ? l : 0u) * stride;
        uint32_t ok = 1;
        const uint64_t t0 = wall_clock64();
        while (true) {
            const uint32_t v = ld_coherent(p);
            if (__all(!mine || (int32_t)(v - want) >= 0)) break;
            if (ld_coherent(abort) != 0) {
                ok = 0;
                break;
            }
            if (wall_clock64() - t0 > limit) {
                if (l == 0) {
                    st_coherent(abort, 1u);
                    __hip_atomic_store(host_abort, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
                }
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (l == 0) *lds_flag = ok;
    }
    __syncthreads();
    return *lds_flag != 0;
}

// Words tagged with the launch that wrote them: a word published during a
// launch carries the launch's epoch above bit `shift` and its value below,
// written by one 32-bit coherent store, so a reader that sees the epoch has
// the value.  Epochs are never 0 and differ from every launch since the
// words were last cleared.
__device__ __forceinline__ bool tag_ok(uint32_t word, uint32_t shift, uint32_t tag) {
    return (word >> shift) == tag;
}

// Bounded wait of one wavefront: keep_waiting() sleeps briefly and returns
// true, or returns false when another workgroup has given up or `limit`
// ticks have passed (then, once, setting *abort and *host_abort).
struct TagWait {
    uint64_t t0;
    uint32_t limit;
    uint32_t* abort;
    uint32_t* host_abort;
    __device__ __forceinline__ bool keep_waiting() const {
        if (ld_coherent(abort) != 0) return false;
        if ((uint64_t)wall_clock64() - t0 > limit) {
            if ((threadIdx.x & 63) == 0) {
                st_coherent(abort, 1u);
                __hip_atomic_store(host_abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
            return false;
        }
        __builtin_amdgcn_s_sleep(2);
        return true;
    }
};

// Waits until each of the n <= 64 words p[l * stride] (l < n) has a bit of
// `valid` set, wavefront 0's lane l reading word l with device-coherent
// loads; then lane l of wavefront 0 holds word l in *val (the word is both
// the flag and the value: no separate arrival).  Bounded as wait_counts:
// returns (uniformly) false when the wait gave up or another workgroup
// did.  Progress needs the workgroups that write the words to be running.
// `done(v)` runs in wavefront 0 with each lane's word once every flag is
// set, before the workgroup barrier (results it writes to LDS are visible
// to every wavefront on return).
template <typename Done>
__device__ __forceinline__ bool poll_flags(const uint32_t* p, uint32_t stride, uint32_t n,
                                           uint32_t valid, uint32_t* val, uint32_t limit,
                                           uint32_t* abort, uint32_t* host_abort,
                                           uint32_t* lds_flag, Done done) {
    if (threadIdx.x < 64) {
        const uint32_t l = threadIdx.x;
        const bool mine = l < n;
        const uint32_t* q = p + (mine ? l : 0u) * stride;
        uint32_t v = 0, ok = 1;
        const uint64_t t0 = wall_clock64();
        while (true) {
            v = ld_coherent(q);
            v = mine ? v : valid;
            if (__all((v & valid) != 0)) break;
            if (ld_coherent(abort) != 0) {
                ok = 0;
                break;
            }
            if (wall_clock64() - t0 > limit) {
                if (l == 0) {
                    st_coherent(abort, 1u);
                    __hip_atomic_store(host_abort, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
                }
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        *val = v;
        if (ok) done(v);
        if (l == 0) *lds_flag = ok;
    }
    __syncthreads();
    return *lds_flag != 0;
}
__device__ __forceinline__ bool poll_flags(const uint32_t* p, uint32_t stride, uint32_t n,
                                           uint32_t valid, uint32_t* val, uint32_t limit,
                                           uint32_t* abort, uint32_t* host_abort,
                                           uint32_t* lds_flag) {
    return poll_flags(p, stride, n, valid, val, limit, abort, host_abort, lds_flag,
                      [](uint32_t) {});
}

}  // namespace llm
