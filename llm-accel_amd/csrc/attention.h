// attention.h -- launch interface of the attention kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llm {

struct AttnArgs {
    const int16_t* qkv;   // projections of the active rows: q | k | v
    uint32_t ldqkv;
    const int16_t* rope;  // [max_seq][head_dim] = cos d/2 | sin d/2 (Q8.8)
    int16_t* kcache;      // this layer's K pages [kv_heads][tiles][64][head_dim]
                          // (after RoPE, rows bank-paired)
    int16_t* vcache;      // this layer's V pages [kv_heads][tiles][head_dim][64]
                          // (positions bank-paired)
    uint32_t tiles;       // pages per (layer, KV head)
    uint32_t pos0;        // absolute position of active row 0
    uint32_t num_heads, num_kv_heads, group, head_dim;
    int32_t qk_scale;     // fm(1/sqrt(head_dim)) raw
    const int16_t* exp14; // Q2.14 exp table, x = -2048..0
    int16_t* out;         // [rows][ldo] attention outputs, head-major
    uint32_t ldo;
    // split path
    uint32_t chunk_tiles; // tiles per workgroup
    uint32_t max_tiles;   // scratch stride in tiles
    int16_t* s_scores;    // [8][kv_heads][max_tiles][group][64]
    int16_t* s_tmax;      // [8][kv_heads][max_tiles][group]
    int32_t* s_tsum;      // [8][kv_heads][max_tiles][group]
    int16_t* s_tval;      // [8][kv_heads][max_tiles][group][head_dim]
    uint32_t* counters;   // [8][num_heads], zero between launches
    // split path, per chunk of tiles and query head: whether the running
    // max rises inside the chunk, sum of its tile sums << 2, and per
    // element the sum of its tile PV values << 8 (the whole chunk's effect
    // on the recurrence when the max does not rise)
    uint32_t max_chunks;
    int32_t* c_flag;      // [8][kv_heads][max_chunks][group]
    int32_t* c_tsum;      // [8][kv_heads][max_chunks][group]
    int32_t* c_sum;       // [8][kv_heads][max_chunks][group][head_dim]
};

// Tiles per split-path workgroup: at most kMaxChunkTiles.
constexpr uint32_t kMaxChunkTiles = 8;

// chunks = max over active rows of ceil(tiles / chunk_tiles); 1 selects
// the fused single-workgroup path.
hipError_t launch_attention(const AttnArgs& a, uint32_t rows, uint32_t kv_heads,
                            uint32_t chunks, hipStream_t st);

}  // namespace llm
