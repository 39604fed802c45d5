// decode_stack.h -- launch interface of the persistent decode kernel
// (internal to the library).
//
// One launch runs a run of decode sublayers (Task 18 / Task 19 of the
// same 1-2 rows at the same position, any layers and pair bindings) on a
// grid of workgroups that are all resident at once.  Every workgroup walks
// every phase of every step -- QKV, attention, O of an attention sublayer;
// gate|up, down of an FFN sublayer -- and takes a fixed share of each
// phase's 4-row blocks; a phase starts when the phase it reads has been
// completed by every workgroup (arrival counters).  Before it waits, a
// workgroup issues the weight loads of the phase it is about to run (and,
// while the attention runs, of the first gate|up blocks), so HBM streams
// weights across the phase boundaries instead of draining at each one.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attention.h"
#include "kernels.h"

namespace llm {

constexpr uint32_t kStackMaxSteps = 72;   // 36 layers x (Task 18, Task 19)
constexpr uint32_t kStackGroups = 5;      // QKV, attention, O, gate|up, down
constexpr uint32_t kStackLines = 32;      // counter lines per group
constexpr uint32_t kStackStride = 32;     // words between counter lines
constexpr uint32_t kStackSyncWords = kStackGroups * kStackLines * kStackStride;
constexpr uint32_t kStackHeadDim = 128;   // head_dim of this kernel
constexpr uint32_t kStackMaxStepsH = 16;  // k-steps over the hidden width
constexpr uint32_t kStackMaxStepsI = 88;  // k-steps over the intermediate width
constexpr uint32_t kStackThreads = 256;   // four wavefronts per workgroup

struct StackStep {
    const int16_t* in;  // input pair rows (ld = ldh)
    int16_t* out;       // output pair rows
    uint32_t layer;
    uint32_t ffn;       // 0: attention sublayer (Task 18), 1: FFN (Task 19)
};

struct StackArgs {
    StackStep steps[kStackMaxSteps];
    uint32_t nsteps, rows, pos0;
    uint32_t H, I, Hp, Ip, Nqkv;        // widths (Hp, Ip padded to 128)
    // weights: matrix m of layer l (tile4x128) at w[m] + l * layer_stride
    const int16_t* w[5];                // QKV, O, gate, up, down of layer 0
    size_t layer_stride;
    const int16_t* norms;               // [(2L + 1)][H], padded to whole k-steps
    int32_t gain;                       // constant RMSNorm gain
    uint32_t L;                         // layers of the model (final norm row 2L)
    const int16_t* exp8;                // Q8.8 exp table (SiLU)
    AttnArgs at;                        // layer 0's attention arguments
    size_t kv_layer_stride;             // elements between layers' KV pages
    int16_t* qkv;                       // [8][Nqkv]
    int16_t* attn;                      // [8][Hp]
    int16_t* act;                       // [8][Ip]
    // final RMSNorm of the last step (an FFN sublayer) into final_out
    // [8][Hp], rows >= rows copying the step's input pair
    int16_t* final_out;
    // arrival counters: group g, line l at sync[(g * kStackLines + l) *
    // kStackStride]; occurrence k of group g (counted over the context)
    // completes at start + (k + 1) * cnt(l), cnt(l) = arrivals per line
    uint32_t* sync;
    uint32_t occ[kStackGroups];         // occurrences before this launch
    uint32_t start;
    uint32_t* abort;                    // device word: a wait gave up
    uint32_t* host_abort;               // host-visible copy
    uint32_t wait_limit;
};

// Workgroups of the launch (every one resident: occupancy x CUs, at most
// two per CU); 0 when the kernel cannot run on this device.  A workgroup
// takes at most two 4-row blocks of the QKV, O and down projections, so
// the launch needs at least a half of the larger block count.
uint32_t stack_workgroups(int cus, uint32_t rows);
// lw: the int32 sums widen every 4 k-steps (4), every step (1).
hipError_t launch_decode_stack(const StackArgs& a, uint32_t nwg, int lw, hipStream_t st);

}  // namespace llm
