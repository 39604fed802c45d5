// attention.h -- launch interface of the attention kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

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
    uint32_t grid_rows, grid_tiles;  // tile path: rows and tiles of the launch
    uint32_t use_gqa;     // long contexts take the GQA tile path when it applies
    uint32_t* counters;   // zero between launches: chunked path [8][kv_heads];
                          // tile path kCounterStride words apart, per (row,
                          // query head) 1 + tile_groups(max_tiles) of them
    // split path, per chunk of tiles and query head: whether the running
    // max rises inside the chunk, sum of its tile sums << 2, and per
    // element the sum of its tile PV values << 8 (the whole chunk's effect
    // on the recurrence when the max does not rise)
    uint32_t max_chunks;
    int32_t* c_flag;      // [8][kv_heads][max_chunks][group]
    int32_t* c_tsum;      // [8][kv_heads][max_chunks][group]
    int32_t* c_sum;       // [8][kv_heads][max_chunks][group][head_dim]
    // tile path in one launch (up to 64 tiles): tile maxima published
    // during the launch (flag | value, zero between launches; the flagged
    // tile sums use s_tsum), the bounded wait's abort words and limit, and
    // the device's compute units
    uint32_t tile_fused;
    int32_t* s_tmax32;    // [8][kv_heads][max_tiles][group]
    // GQA path in one launch (scores and PV): the tile maxima go into
    // s_gmax32 [8][kv_heads][max_tiles][group] tagged with the launch's
    // epoch (epoch << 16 | (uint16) max; 1..kGqaEpochMax, different from
    // every launch since s_gmax32 was last cleared)
    uint32_t epoch;
    int32_t* s_gmax32;
    // ... and, with the scan in the same launch, the tile sums as
    // s_gsum64 [8][kv_heads][max_tiles][group] = epoch << 32 | sum, stored
    // after the tile's values (null: the scan is a launch of its own)
    uint64_t* s_gsum64;
    uint32_t* abort;      // device word set when a wait gave up
    uint32_t* host_abort; // host-visible copy
    uint32_t wait_limit;  // bound of one wait (100 MHz ticks)
    uint32_t cus;
    // one-launch tile path with the O projection in the same launch: the
    // combining workgroups' arrival counters (kSyncAttnLines of them,
    // kSyncStride words apart; null otherwise)
    uint32_t* attn_arrive;
    // one-launch kernels go through hipLaunchCooperativeKernel, which
    // refuses a grid the device cannot hold at once (other work holding
    // compute units included); the launcher then takes the separate launches
    uint32_t coop;
};

// Tile-path arrivals: the tiles of a (row, query head) arrive in groups of
// kArriveGroup on counters one 128-byte line apart, the last tile of each
// group on the (row, query head)'s top counter (no line takes more than
// kArriveGroup atomics: arrivals on one line serialise).
constexpr uint32_t kArriveGroup = 16, kCounterStride = 32;
constexpr uint32_t tile_groups(uint32_t tiles) { return (tiles + kArriveGroup - 1) / kArriveGroup; }
// Words of `counters` for a context of `tiles` tiles per (layer, KV head).
constexpr size_t counter_words(uint32_t num_heads, uint32_t tiles) {
    return (size_t)8 * num_heads * (1 + tile_groups(tiles)) * kCounterStride;
}

// Epochs of the GQA path's tagged maxima and sums run 1..kGqaEpochMax;
// then the host clears s_gmax32 and s_gsum64 and starts again.
constexpr uint32_t kGqaEpochMax = 65535;

// Tiles per split-path workgroup: at most kMaxChunkTiles.
constexpr uint32_t kMaxChunkTiles = 8;

// Long contexts with the query heads of a GQA group sharing each K / V
// page (attention_gqa.hip): head_dim 64 or 128, at most 8 query heads per
// KV head, at most 1024 tiles.
bool attention_gqa_ok(const AttnArgs& a, uint32_t rows);
hipError_t launch_attention_gqa(const AttnArgs& a, uint32_t rows, hipStream_t st);

// chunks = max over active rows of ceil(tiles / chunk_tiles); 1 selects
// the fused single-workgroup path.
hipError_t launch_attention(const AttnArgs& a, uint32_t rows, uint32_t kv_heads,
                            uint32_t chunks, hipStream_t st);

// Attention sublayer of decode rows in one launch: workgroups [0, nq) are
// the QKV projection's 4-row blocks, [nq, nq + na) the attention of (row,
// query head), the rest the O projection's blocks (with its residual and
// FFN-norm epilogue).  Each later role issues its weight / cache loads,
// then waits for the arrivals of the role it reads.
struct SublayerArgs {
    ProjArgs qkv, o;
    AttnArgs at;
    uint32_t nq, na, no;
    // Arrival counters (kSyncWords words) grow across launches: QKV
    // workgroup b adds 1 to line b % kSyncQkvLines, which held qkv_base[l]
    // before the launch; every attention workgroup adds 1 to each of
    // kSyncAttnLines lines, which held attn_base.  The host keeps the
    // bases (mod 2^32).
    uint32_t* sync;
    uint32_t qkv_base[32];
    uint32_t attn_base;
    uint32_t* host_abort;  // host-visible word, set when a wait gave up
    uint32_t wait_limit;   // bound of one wait (100 MHz ticks)
};
constexpr uint32_t kSyncStride = 32;  // words between counters (one 128-byte line)
constexpr uint32_t kSyncQkvLines = 32, kSyncAttnLines = 16;
static_assert(sizeof(SublayerArgs::qkv_base) == kSyncQkvLines * 4, "one base per QKV line");
constexpr uint32_t kSyncAttn = kSyncQkvLines * kSyncStride;
// Word of `sync` set when a wait gave up (cleared by the host).
constexpr uint32_t kSyncAbort = kSyncAttn + kSyncAttnLines * kSyncStride;
constexpr uint32_t kSyncWords = kSyncAbort + kSyncStride;

// Whether the fused launch serves `rows` rows with this shape: head_dim
// 64 or 128, the split-head attention path, every wavefront of both
// projections within 4 k-steps, and the waiting workgroups fewer than the
// `capacity` the device holds at once (so that the workgroups they wait
// for can always be dispatched).
bool sublayer_fused_ok(const SublayerArgs& s, uint32_t rows, int qkv_epi, int L_qkv, int L_o,
                       int capacity);
// Whether the fused launch reads the two projections' 12-bit copies.
bool sublayer_reads_p12(const SublayerArgs& s);

// The one-launch tile path (5-64 tiles, decode rows) and the O projection
// in one launch: tile workgroups first, then O blocks that wait for every
// (row, query head) of the attention (arrivals on the kSyncAttn counters,
// which held attn_base before the launch; the host adds `arrivals` to its
// copy after the launch).
struct TileOArgs {
    AttnArgs at;
    ProjArgs o;
    uint32_t ntile, no;     // tile workgroups (the tile grid), O workgroups
    uint32_t arrivals;      // rows x query heads
    uint32_t* sync;
    uint32_t attn_base;
    uint32_t* host_abort;
    uint32_t wait_limit;
};
// The variant of the tile + O launch for an O projection of widening
// interval L, and the workgroups of a variant the device holds at once.
int tile_o_variant(const ProjArgs& o, int L);
int tile_o_capacity(uint32_t head_dim, uint32_t rows, int variant, int cus);
// Fills the launch shape of s (grid, arrivals) and returns whether the
// launch serves `rows` rows: head_dim 64 or 128, 1-2 rows, the attention
// on the one-launch tile path (5-64 tiles, not the GQA path, not
// cooperative), O within 4 k-steps per wavefront, the whole grid within
// `capacity`.
bool tile_o_prepare(TileOArgs& s, uint32_t rows, int capacity);
hipError_t launch_attention_tile_o(const TileOArgs& s, uint32_t rows, int L, hipStream_t st);
// QKV and O workgroups of the fused launch for `blocks` 4-row blocks.
uint32_t sublayer_qkv_workgroups(uint32_t blocks);
uint32_t sublayer_o_workgroups(uint32_t blocks);
// Workgroups of the fused launch for (head_dim, rows, QKV epilogue) that
// the device holds at once (`cus` compute units); 0 when unsupported.
int sublayer_capacity(uint32_t head_dim, uint32_t rows, int qkv_epi, int cus);
// L: the smaller widening interval of the QKV and O matrices.
hipError_t launch_attention_sublayer(const SublayerArgs& s, uint32_t rows, int qkv_epi,
                                     int L, hipStream_t st);

}  // namespace llm
