// kernels.h -- launch interface of the HIP kernels (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llm {

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SILU = 2 };

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
    const int16_t* exp8;  // Q8.8 exp table, x = -2048..0 (EPI_SILU)
};

struct RopeArgs {
    const int16_t* qkv;  // [rows][ldqkv]: q | k | v projections
    uint32_t ldqkv;
    int16_t* q;          // rotated q [rows][ldq]
    uint32_t ldq;
    int16_t* kcache;     // page pool [pages][64][head_dim]
    int16_t* vcache;
    const int32_t* page_table;  // this layer: [kv_heads][tiles]
    uint32_t tiles;
    const int16_t* rope;  // [max_seq][head_dim] = cos d/2 | sin d/2
    uint32_t pos0;
    uint32_t num_heads, num_kv_heads, head_dim;
};

struct AttnArgs {
    const int16_t* q;  // rotated q [rows][ldq]
    uint32_t ldq;
    const int16_t* kcache;
    const int16_t* vcache;
    const int32_t* page_table;  // this layer: [kv_heads][tiles]
    uint32_t tiles;
    uint32_t pos0;
    uint32_t group, head_dim;
    int32_t qk_scale;      // fm(1/sqrt(head_dim)) raw
    const int16_t* exp14;  // Q2.14 exp table, x = -2048..0
    int16_t* out;          // [rows][ldo]
    uint32_t ldo;
};

hipError_t launch_proj(const ProjArgs& a, int epi, int L, uint32_t blocks,
                       hipStream_t st);
hipError_t launch_rmsnorm(const int16_t* x, uint32_t ldx, const int16_t* gamma,
                          uint32_t cols, int16_t* y, uint32_t ldy, uint32_t rows,
                          hipStream_t st);
hipError_t launch_rope_append(const RopeArgs& a, uint32_t rows, hipStream_t st);
hipError_t launch_attention(const AttnArgs& a, uint32_t rows, uint32_t kv_heads,
                            hipStream_t st);

}  // namespace llm
