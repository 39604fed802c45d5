// ops.h -- kernels of the operator-level commands (internal to the library).
//
// The controller's per-operator scheduler (kernel/control_cache_8x64.cpp
// :6497-7500 of the reference) runs one operator per command: the seven
// projections, RMSNorm, SiLU*up, residual add, the attention building
// blocks QK, PV and softmax over one 64-position tile, flash attention
// over the cache for one decode position (with or without appending that
// position's K / V) and block attention for up to 8 prefill tokens.  The
// projections and RMSNorm reuse the resident path's kernels; the rest are
// here.  Port tensors are tight row-major int16 in the order of the
// reference's two ports (port 0 = KV head 0, then KV head 1, ...).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llm {

// ATTN_QK: out[h][g][p] (p < 64) = the scaled score of query row q[h][g]
// against K row k[h][p] for p < tile_len, 0 for p >= tile_len.
hipError_t launch_op_qk(const int16_t* q, const int16_t* k, uint32_t kv_heads,
                        uint32_t group, uint32_t head_dim, uint32_t tile_len,
                        int32_t qk_scale, int16_t* out, hipStream_t st);
// ATTN_PV: out[h][g][e] = sum over p < tile_len of p[h][g][p] (row stride
// 64) times v[h][p][e], four p-mod-4 banks.
hipError_t launch_op_pv(const int16_t* p, const int16_t* v, uint32_t kv_heads,
                        uint32_t group, uint32_t head_dim, uint32_t tile_len,
                        int16_t* out, hipStream_t st);
// SOFTMAX: rows of 64 (first tile_len valid) -> rows of tile_len.
hipError_t launch_op_softmax(const int16_t* x, uint32_t rows, uint32_t tile_len,
                             const int16_t* exp8, int16_t* out, hipStream_t st);
// SILU_MUL and RESIDUAL_ADD over n elements.
hipError_t launch_op_silu_mul(const int16_t* gate, const int16_t* up, uint32_t n,
                              const int16_t* exp8, int16_t* out, hipStream_t st);
hipError_t launch_op_residual(const int16_t* a, const int16_t* b, uint32_t n,
                              int16_t* out, hipStream_t st);

// Flash attention of query rows over cache pages (one layer's kcache /
// vcache, the paged layout of attention.h).  q and out are
// [kv_heads][tokens][group][head_dim]; token t of the block sees positions
// [0, pos0 + t].  legacy = 1: Q8.8 probabilities from the exp8 table, PV
// without rescaling (ATTN_FLASH / DECODE_SMOKE); 0: Q2.14 probabilities
// from exp14, PV rescaled by 1/64 (ATTN_PREFILL_BLOCK).
struct OpFlashArgs {
    const int16_t* q;
    const int16_t* kcache;
    const int16_t* vcache;
    uint32_t tiles;  // pages per (layer, KV head)
    uint32_t kv_heads, tokens, group, head_dim;
    uint32_t pos0;
    int32_t qk_scale;
    const int16_t* exp8;
    const int16_t* exp14;
    int legacy;
    int16_t* out;
};
hipError_t launch_op_flash(const OpFlashArgs& a, hipStream_t st);
// Writes k[h] / v[h] (head_dim each) as position pos of every KV head's
// pages of one layer.
hipError_t launch_op_kv_append(int16_t* kcache, int16_t* vcache, uint32_t tiles,
                               uint32_t kv_heads, uint32_t head_dim, uint32_t pos,
                               const int16_t* k, const int16_t* v, hipStream_t st);

}  // namespace llm
