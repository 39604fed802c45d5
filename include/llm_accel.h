/*
 * llm_accel.h -- C ABI of the MI355X resident decoder-layer path.
 *
 * Drop-in for LLM-ACCEL's coarse-task boundary: the host hands the device
 * an operator id, layer, active row count (1..8) and first position; the
 * device runs the whole sublayer with hidden state, KV cache and all
 * intermediates resident in HBM, and returns the controller's 64-byte
 * status record.  Plain pointers and sizes only.
 *
 * Reference interfaces replaced (paths under the reference repository):
 *   - device kernel control_cache_8x64_dual_core_nk + status sink
 *     (include/vitis_stream_8x64.hpp:219-258, kernel/control_cache_8x64.cpp
 *     :5767-6481) -> llm_task();
 *   - accelerator_t construction, persistent aux tables and one-time weight
 *     migration (host/host_qwen_8x64.cpp:1026-1086, :2144-2190, :2458-2478)
 *     -> llm_ctx_create(), llm_load_*();
 *   - feature-pair H2D / D2H migration and port rebinding
 *     (host/host_qwen_8x64.cpp:1283-1445, :1846-1888, :2062-2103)
 *     -> llm_hidden_upload*(), llm_hidden_download*(), pair ids of
 *     llm_task();
 *   - KV cache preload / inspection (host/host_qwen_8x64.cpp:1729-1843)
 *     -> llm_kv_write(), llm_kv_read().
 *
 * Threading: one host thread per context; every call is synchronous with
 * respect to the caller (work runs on the context's own HIP stream).
 * Return values: >= 0 is a reference status code (llm_task) or 0; < 0 is an
 * error of this library (LLM_E_*), with a message in llm_last_error().
 */
#ifndef LLM_ACCEL_H
#define LLM_ACCEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Operator ids (include/control_cache_8x64.hpp:253-276).  llm_task() is
 * the resident-layer image: ids 1..15 and 17 return
 * LLM_STATUS_BAD_OPERATOR exactly as that image does
 * (kernel/control_cache_8x64.cpp:6483-6494); llm_op() runs them as the
 * controller's full image does. */
enum {
    LLM_OP_NOP = 0,
    LLM_OP_Q_PROJECTION = 1,       /* operator-level (llm_op)          */
    LLM_OP_K_PROJECTION = 2,
    LLM_OP_V_PROJECTION = 3,
    LLM_OP_O_PROJECTION = 4,
    LLM_OP_FFN_GATE = 5,
    LLM_OP_FFN_UP = 6,
    LLM_OP_FFN_DOWN = 7,
    LLM_OP_RMSNORM = 8,
    LLM_OP_SILU_MUL = 9,
    LLM_OP_RESIDUAL_ADD = 10,
    LLM_OP_ATTN_QK = 11,
    LLM_OP_ATTN_PV = 12,
    LLM_OP_SOFTMAX = 13,
    LLM_OP_ATTN_FLASH = 14,
    LLM_OP_DECODE_SMOKE = 15,
    LLM_OP_DECODER_LAYER = 16,     /* attention + FFN sublayers        */
    LLM_OP_ATTN_PREFILL_BLOCK = 17, /* operator-level (llm_op)         */
    LLM_OP_ATTENTION_SUBLAYER = 18, /* Task 18                         */
    LLM_OP_FFN_SUBLAYER = 19,       /* Task 19                         */
    LLM_OP_FINAL_NORM = 20          /* Task 20                         */
};

/* Status codes (include/control_cache_8x64.hpp:279-286). */
enum {
    LLM_STATUS_OK = 0,
    LLM_STATUS_BAD_OPERATOR = 1,
    LLM_STATUS_BAD_TOKEN_COUNT = 2,
    LLM_STATUS_BAD_TILE_LENGTH = 3,
    LLM_STATUS_BAD_POSITION = 4,
    LLM_STATUS_BAD_LAYER = 5
};

/* Library errors (never produced by the reference). */
enum {
    LLM_E_ARG = -1,    /* bad argument / shape                   */
    LLM_E_HIP = -2,    /* HIP runtime error                      */
    LLM_E_NOMEM = -3,  /* device allocation failed               */
    LLM_E_STATE = -4   /* missing weights / tables               */
};

/* Projection ids, in the reference's packed order
 * (host/host_qwen_8x64.cpp:325-376, kernel/mm_controller.cpp:51-102). */
enum {
    LLM_PROJ_Q = 0,
    LLM_PROJ_K = 1,
    LLM_PROJ_V = 2,
    LLM_PROJ_O = 3,
    LLM_PROJ_GATE = 4,
    LLM_PROJ_UP = 5,
    LLM_PROJ_DOWN = 6
};

/* Model shape (model_shape_t, host/host_qwen_8x64.cpp:110-118).
 * Requirements of this build: num_kv_heads >= 1, num_heads % num_kv_heads
 * == 0, head_dim a multiple of 16 and <= 128, heads per KV group <= 16,
 * hidden a multiple of 8, intermediate a multiple of 4 (every reference
 * profile qualifies: host/host_qwen_8x64.cpp:309-343). */
typedef struct {
    uint32_t vocab_size;
    uint32_t hidden_size;
    uint32_t intermediate_size;
    uint32_t num_layers;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t max_seq_len;
    double rope_theta; /* 1e6 in the reference (host:47) */
} llm_shape_t;

/* The controller's 64-byte status record (kernel/cc8_status_sink.cpp:4-15,
 * decoded at host/host_qwen_8x64.cpp:670-684).  op, code, token_count and
 * last_task follow the reference exactly; the four schedule counters are
 * the values the 8x64 controller would report for the same command,
 * computed from its formulas (kernel/control_cache_8x64.cpp:5974-6481). */
typedef struct {
    uint32_t op;
    uint32_t code;
    uint32_t token_count;
    uint32_t output_waves;
    uint32_t mm_tasks;
    uint32_t vector_tasks;
    uint32_t completed_packets;
    uint32_t last_task;
    uint32_t reserved[8];
} llm_status_t;

typedef struct llm_ctx llm_ctx_t;

/* Create a context on HIP device `device`: allocates weights, norm table,
 * RoPE table (built here from rope_theta exactly as the reference host
 * builds aux1), a zeroed KV cache for max_seq_len positions of every
 * layer, `num_pairs` hidden-state pairs of 8 rows, and scratch.  The
 * reference binds 4 feature buffers (two pairs); num_pairs >= 2. */
int llm_ctx_create(const llm_shape_t* shape, int device, uint32_t num_pairs,
                   llm_ctx_t** out);
void llm_ctx_destroy(llm_ctx_t* ctx);
const char* llm_last_error(void);

/* Weights of one projection of one layer, row-major [out_dim][in_dim]
 * Q4.12 raw int16 (the values projection_weight_raw returns,
 * host/host_qwen_8x64.cpp:899-935). */
int llm_load_projection(llm_ctx_t* ctx, uint32_t layer, uint32_t proj,
                        const int16_t* weights);
/* The reference's 16 packed weight shards (host/host_qwen_8x64.cpp:842-869,
 * :899-935): shard i holds `shard_words` 64-byte words of 32 int16 lanes
 * covering every layer's 16x16 tiles. */
int llm_load_packed_shards(llm_ctx_t* ctx, const int16_t* const shards[16],
                           uint64_t shard_words);
/* A packed Fix16 checkpoint directory (model_data_t::load,
 * host/host_qwen_8x64.cpp:736-840): layer_weights_shard00..15.fix16.bin
 * (the llm_load_packed_shards layout, weight_shard_words 64-byte words
 * each for the context's num_layers), norm_weights.fix16.bin
 * ((2L+1)*hidden int16), token_embedding.fix16.bin (vocab*hidden int16,
 * read into `embedding`, host memory of the caller, when not NULL) and,
 * unless LLM_CKPT_TIE_EMBEDDINGS (the embedding is then the LM head),
 * lm_head.fix16.bin into the LM head when present.  Every file must have
 * exactly its expected size ("<what> size mismatch: <path> expected=N
 * actual=M", LLM_E_ARG; sizes are all checked before anything loads);
 * with LLM_CKPT_REQUIRE_LM_HEAD a missing, untied LM head is an error. */
#define LLM_CKPT_TIE_EMBEDDINGS 1u
#define LLM_CKPT_REQUIRE_LM_HEAD 2u
int llm_load_checkpoint_dir(llm_ctx_t* ctx, const char* dir, uint32_t flags,
                            int16_t* embedding);
/* Norm table, [(2*num_layers + 1)][hidden] Q8.8: rows 2l (attention),
 * 2l+1 (FFN), 2L (final) (include/control_cache_8x64.hpp:111-123). */
int llm_load_norms(llm_ctx_t* ctx, const int16_t* norms);

/* Hidden-state pairs: rows are [rows][hidden] int16 Q8.8. */
int llm_hidden_upload(llm_ctx_t* ctx, uint32_t pair, const int16_t* rows,
                      uint32_t row_count);
int llm_hidden_download(llm_ctx_t* ctx, uint32_t pair, int16_t* rows,
                        uint32_t row_count);
/* The reference's packed feature ports (host/host_qwen_8x64.cpp:2062-2103):
 * rows 0-3 in port0, rows 4-7 in port1, row stride `stride_words` 64-byte
 * words (ceil(max(H, I) / 32) in the reference). */
int llm_hidden_upload_ports(llm_ctx_t* ctx, uint32_t pair,
                            const int16_t* port0, const int16_t* port1,
                            uint32_t row_count, uint32_t stride_words);
int llm_hidden_download_ports(llm_ctx_t* ctx, uint32_t pair, int16_t* port0,
                              int16_t* port1, uint32_t row_count,
                              uint32_t stride_words);

/* One coarse task: the controller invocation with scalar arguments
 * operator_kind, layer_id, token_count, position, tile_len
 * (kernel/control_cache_8x64.cpp:5767-5797), reading pair `in_pair` and
 * writing pair `out_pair` (the reference's port rebinding; equal pairs are
 * allowed).  Returns the status code (also in *status when non-NULL). */
int llm_task(llm_ctx_t* ctx, uint32_t op, uint32_t layer,
             uint32_t token_count, uint32_t position, uint32_t tile_len,
             uint32_t in_pair, uint32_t out_pair, llm_status_t* status);

/* Operator-level commands: the per-operator scheduler of the
 * controller's full image (kernel/control_cache_8x64.cpp:6497-7500) as the
 * reference host drives it through run_feature, run_attention and
 * run_prefill_attention_block (host/host_qwen_8x64.cpp:1088-1133,
 * :1556-1675).  Replaces launch() of those host paths (:2500-2757) with
 * ops 1..15 and 17; ops 16 and 18..20 are llm_task()'s (LLM_E_ARG here).
 *
 * in, aux and out are device memory, each holding what the reference's
 * two ports of that name hold (input_port0/1, aux_port0/1,
 * output_port0/1), concatenated and tight (rows not padded to 64-byte
 * words); NULL selects the context's own port buffer (llm_port()).  With
 * H = hidden, I = intermediate, C = num_kv_heads * head_dim, G = query
 * heads per KV head, d = head_dim, T = token_count, and [a][b] row-major
 * int16 Q8.8:
 *   1-3, 5, 6 (Q, K, V, gate, up projection of `layer`): in [T][H] ->
 *        out [T][H | C | C | I | I];
 *   4 (O): in [T][H] -> out [T][H];   7 (down): in [T][I] -> out [T][H];
 *   8 RMSNORM: in [T][H], aux [1][H] gains -> out [T][H];
 *   9 SILU_MUL: in gate [T][I], aux up [T][I] -> out [T][I];
 *   10 RESIDUAL_ADD: in [T][H], aux [T][H] -> out [T][H];
 *   11 ATTN_QK (1 <= tile_len <= 64): in q [Hkv][G][d], aux K panels
 *        [Hkv][tile_len][d] -> out scores [Hkv][G][64] (0 past tile_len);
 *   12 ATTN_PV: in probabilities [Hkv][G][64] (Q8.8, first tile_len
 *        used), aux V panels [Hkv][tile_len][d] -> out [Hkv][G][d];
 *   13 SOFTMAX: in [Hkv][G][64] -> out [Hkv][G][tile_len];
 *   14 ATTN_FLASH (T = G): in q [Hkv][G][d] -> out [Hkv][G][d], attention
 *        over cache positions [0, position] of `layer`;
 *   15 DECODE_SMOKE (T = G): as 14 after writing aux = K [Hkv][d] then
 *        V [Hkv][d] as cache position `position`;
 *   17 ATTN_PREFILL_BLOCK (1 <= T <= 8): in q [Hkv][T][G][d] -> out the
 *        same shape; token t attends to cache positions [0, position + t].
 * Returns the reference status code (also in *status, with the
 * controller's counters); work is enqueued on the context stream and not
 * waited for (llm_sync()).  tile_len != 0 on a projection is the FPGA
 * MM wave-profile encoding and returns LLM_E_ARG. */
enum { LLM_PORT_IN = 0, LLM_PORT_AUX = 1, LLM_PORT_OUT = 2 };
int llm_op(llm_ctx_t* ctx, uint32_t op, uint32_t layer, uint32_t token_count,
           uint32_t position, uint32_t tile_len, const int16_t* in,
           const int16_t* aux, int16_t* out, llm_status_t* status);
/* The context's port buffer `port` (device memory of *elems int16,
 * enough for every operator's tensor); allocated on first use.  Replaces
 * the reference host's six data buffers data_words_ (two per port name,
 * host/host_qwen_8x64.cpp:3060, packed by :2062-2123). */
int llm_port(llm_ctx_t* ctx, uint32_t port, void** dev, size_t* elems);
/* Synchronous host copies into / out of a port buffer (the migrations
 * around launch(), host/host_qwen_8x64.cpp:2500-2757). */
int llm_port_write(llm_ctx_t* ctx, uint32_t port, const int16_t* host, size_t elems);
int llm_port_read(llm_ctx_t* ctx, uint32_t port, int16_t* host, size_t elems);

/* KV cache rows of one layer and KV head, positions [pos0, pos0 + n):
 * k / v are [n][head_dim] Q8.8 (K stored after RoPE, V raw). */
int llm_kv_read(llm_ctx_t* ctx, uint32_t layer, uint32_t kv_head,
                uint32_t pos0, uint32_t n, int16_t* k, int16_t* v);
int llm_kv_write(llm_ctx_t* ctx, uint32_t layer, uint32_t kv_head,
                 uint32_t pos0, uint32_t n, const int16_t* k,
                 const int16_t* v);
/* Zero the whole KV cache (accelerator_t constructor, host:1073-1074). */
int llm_kv_clear(llm_ctx_t* ctx);

/* Device pointer of a pair's [8][hidden] rows (for zero-copy callers). */
void* llm_pair_device_ptr(llm_ctx_t* ctx, uint32_t pair);
/* The context's HIP stream (hipStream_t) and a full synchronisation. */
void* llm_stream(llm_ctx_t* ctx);
int llm_sync(llm_ctx_t* ctx);

/* HIP-event timing on the context stream: record into slot (0..1023), and
 * the elapsed milliseconds between two recorded slots (synchronises). */
int llm_event_record(llm_ctx_t* ctx, uint32_t slot);
int llm_event_elapsed_ms(llm_ctx_t* ctx, uint32_t slot_a, uint32_t slot_b,
                         float* ms);

/* Per-kernel timing for measurement: when enabled, every kernel launch of
 * llm_task is bracketed by HIP events on the context stream; stats sum
 * the measured durations per kernel kind since the last enable. */
enum {
    LLM_K_RMSNORM = 0,   /* attention / FFN / final RMSNorm          */
    LLM_K_QKV = 1,       /* fused Q | K | V projection                */
    LLM_K_ROPE = 2,      /* RoPE + KV-cache append                     */
    LLM_K_ATTENTION = 3, /* tiled online-softmax attention             */
    LLM_K_OPROJ = 4,     /* O projection + residual                    */
    LLM_K_GATEUP = 5,    /* gate | up projection + SiLU * up           */
    LLM_K_DOWN = 6,      /* down projection + residual                 */
    LLM_K_ATTN_SUBLAYER = 7, /* QKV + attention + O in one launch (decode) */
    LLM_K_COUNT = 8
};
int llm_kernel_timing(llm_ctx_t* ctx, int enable);
int llm_kernel_stats(llm_ctx_t* ctx, uint32_t kernel, uint64_t* launches,
                     double* total_ms);

/* Back-to-back launches of one projection kernel (kernel = LLM_K_QKV,
 * LLM_K_OPROJ, LLM_K_GATEUP or LLM_K_DOWN) on `rows` resident rows,
 * cycling over layers [0, layers); *avg_us is the mean duration of one
 * launch measured with HIP events on the context stream.  Outputs go to
 * scratch; hidden pairs and the KV cache are untouched. */
int llm_bench_projection(llm_ctx_t* ctx, uint32_t kernel, uint32_t rows,
                         uint32_t layers, uint32_t iters, float* avg_us);

/* Device memory held by the decoder-layer weights, all layouts together
 * (16-bit tiles, byte planes, 12-bit copies, per-output byte sums), and
 * the number of layer matrices (Q|K|V, O, gate, up, down per layer) held
 * in 16 bits.  A matrix whose weights all lie in [-2048, 2047] is held in
 * 12 bits only; one with any weight outside keeps the 16-bit tiles and
 * byte planes.  No counterpart in the reference (its weights are one
 * packed image in device DDR); for capacity planning. */
int llm_weight_bytes(llm_ctx_t* ctx, uint64_t* bytes, uint32_t* wide_matrices);

/* A plain device-to-device copy of `bytes` repeated `iters` times on the
 * context stream (calibration reference for HBM counters and achievable
 * bandwidth); *ms is the average duration of one copy. */
int llm_bench_copy(llm_ctx_t* ctx, uint64_t bytes, uint32_t iters, float* ms);

/* LM head for the device argmax: [vocab][hidden] raw int16 (the tied
 * embedding table, or lm_head.fix16.bin; model_data_t::lm_head_argmax,
 * host/host_qwen_8x64.cpp:937-969).  vocab < 2^18, hidden <= 16384. */
int llm_load_lm_head(llm_ctx_t* ctx, const int16_t* table, uint32_t vocab);
/* For rows [row0, row0 + rows) of `pair`: argmax over v of the exact int64
 * sum_k h[k] * W[v][k], first index on ties (the reference's strict >
 * scan), into tokens[]; scores[] (optional) receives the winning sums.
 * Replaces the host-side lm_head_argmax of the reference. */
int llm_lm_head_argmax(llm_ctx_t* ctx, uint32_t pair, uint32_t row0,
                       uint32_t rows, uint32_t* tokens, int64_t* scores);

/* No counterpart in the reference.  For callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops): the
 * argmax of llm_lm_head_argmax() over memory the caller owns, with no
 * context and no allocation.  table is device memory [vocab][hidden] raw
 * int16 (the reference's row-major LM head); rows is device memory
 * [row_count][ld]; tokens (uint32 [row_count]) and scores (int64
 * [row_count], optional) are device memory.  Work is enqueued on `stream`
 * (a hipStream_t; NULL = the null stream) and not waited for.  Limits:
 * row_count <= 8, vocab < 2^18, hidden <= 16384 and a multiple of 8, ld a
 * multiple of 8, table and rows 16-byte aligned; larger sizes return
 * LLM_E_ARG.  Its scratch is 64 bytes of static device memory per device,
 * shared by every call on that device: calls that overlap on one device
 * race. */
int llm_lm_head_argmax_static(const int16_t* table, uint32_t vocab,
                              uint32_t hidden, const int16_t* rows,
                              uint32_t ld, uint32_t row_count,
                              uint32_t* tokens, int64_t* scores, void* stream);

/* Report of llm_generate (the QWEN_8X64_E2E_PROFILE fields of the
 * reference's generate mode, host/host_qwen_8x64.cpp:9264-9336).  Forward
 * and LM-head times are stream-event times on the device (a forward from
 * before its rows' copy to after its last task); the generate loop waits
 * only for each sampled token's argmax keys. */
typedef struct {
    uint32_t prompt_tokens;
    uint32_t generated_tokens;
    uint32_t prompt_forward_passes;
    uint32_t generated_forward_passes;
    uint32_t coarse_task_count;       /* ceil(P/B)*2L + 1 + (G-1)*(2L+1) */
    uint32_t output_materializations;
    uint32_t released_prompt_blocks;
    uint32_t wait_reruns;             /* runs re-done on launches without
                                         waits between workgroups after a
                                         bounded wait gave up (0 normally) */
    double prompt_forward_ms;         /* all prompt blocks */
    double time_to_first_token_ms;    /* host clock, call to first token */
    double generated_forward_ms;      /* sum over the sampled tokens' forwards */
    double lm_head_ms;                /* sum over the argmax launches */
    double total_ms;                  /* host clock of the call */
    double generated_wall_ms;         /* host clock from the first token to the
                                         last (the generated forwards and their
                                         argmaxes) */
    /* Residency (tests/test_coarse_task_residency_contract.sh:63-80 of the
     * reference): host -> device copies of hidden rows (one per forward),
     * device -> host copies of hidden rows (0: the argmax runs on the
     * device and returns 8-byte keys), KV transfers (0), key read-backs
     * (one per sampled token). */
    uint32_t input_migrations;
    uint32_t output_migrations;
    uint32_t kv_migrations;
    uint32_t argmax_readbacks;
} llm_generate_stats_t;

/* Line sink of the request loop.  With a sink set, llm_generate brackets
 * every task with stream events, synchronises after every forward and
 * passes the reference's report lines (host/host_qwen_8x64.cpp:1342-1352,
 * :7684-7711, :7885-7909, :9264-9336): COARSE_TASK_PROGRESS per task,
 * COARSE_TASK_PREFILL_BLOCK per prompt block, COARSE_TASK_STACK per
 * sampled-token forward and one QWEN_8X64_E2E_PROFILE line, key=value
 * fields separated by spaces.  NULL removes the sink. */
typedef void (*llm_log_fn)(const char* line, void* user);
int llm_set_log(llm_ctx_t* ctx, llm_log_fn fn, void* user);

/* The reference's generate loop with coarse tasks (host/host_qwen_8x64.cpp
 * :9016-9136 with run_prompt_block :7840-7884 and run_token :7665-7712):
 * the prompt in blocks of block_size (<= 8) tokens through layers
 * [0, layer_count) (Task 18 from pair 1 into pair 0, Task 19 back, per
 * layer), Task 20 only after the final block; then max_new_tokens sampled
 * tokens, each the LM-head argmax of the last row, with a one-row forward
 * (Tasks 18/19 per layer and 20) for every sampled token but the last.
 * Embedding rows are gathered on the host from `embedding` [vocab][hidden]
 * and uploaded, as in the reference.  Requires llm_load_lm_head first.
 * A one-launch kernel whose bounded wait between workgroups gives up
 * (e.g. a device shared with other work) does not fail the request: the
 * forwards since the previous synchronisation run again on launches
 * without such waits (counted in stats->wait_reruns), as the reference's
 * controller completes every command it accepts
 * (kernel/control_cache_8x64.cpp:5892-5957).  llm_task reports the same
 * event as LLM_E_HIP at its caller's next synchronisation. */
int llm_generate(llm_ctx_t* ctx, const int16_t* embedding, uint32_t vocab,
                 const uint32_t* prompt, uint32_t n_prompt, uint32_t block_size,
                 uint32_t layer_count, uint32_t max_new_tokens,
                 uint32_t* out_tokens, llm_generate_stats_t* stats);

/* The two exp tables the kernels use, 2049 entries for x = -8 .. 0 in
 * Q8.8 steps: q8_8 = the reference's hls::exp on ap_fixed<16,8> (SiLU and
 * the Q8.8 softmax / flash operators; golden_exp, host/host_qwen_8x64.cpp
 * :578-586), q2_14 = floor(e^x * 16384) (attention probabilities,
 * hls::exp on ap_fixed<18,4>, host:588-596). */
int llm_exp_tables(int16_t* q8_8, int16_t* q2_14);

#ifdef __cplusplus
}
#endif
#endif
