/*
 * llm_oracle.h -- CPU restatement of LLM-ACCEL's fixed-point golden model.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * MI355X path: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product (liballm_accel / the HIP
 * kernels) never links, loads or calls it.
 *
 * Every function restates one golden_* routine of the reference host
 * (host/host_qwen_8x64.cpp) on raw integers.  The ap_fixed semantics used
 * (documented Xilinx ap_fixed behaviour, UG1399):
 *   - expression temporaries are exact;
 *   - AP_RND rounds half toward +inf: raw = floor(x * 2^F + 1/2);
 *   - AP_SAT clamps to the signed W-bit range;
 *   - quantisation happens only on assignment / construction.
 * Formats: Q8.8 activations and gammas (fm_t), Q4.12 weights (wt_linear_t),
 * Q16.16 accumulators (fm_accum_t), Q2.14 attention probabilities.
 *
 * Parity pinning (see tests/test_oracle_*.py):
 *   - mt19937 / uniform_int_distribution: std::mt19937 10000th-output
 *     check, and a cross-check against this container's libstdc++;
 *   - projection / residual / rmsnorm / recip / rsqrt / rope / QK / PV:
 *     closed forms, exhaustive tables, brute-force ap_fixed model in
 *     Python (exact rationals), and the reference's published known-answer
 *     values (results/ logs, transcribed in tests/golden/kat.json);
 *   - the two hls::exp instantiations: restated from the structure the
 *     reference's HLS build log shows and pinned end-to-end by those
 *     known-answer values (the HLS math library is not available here).
 */
#ifndef LLM_ORACLE_H
#define LLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model shape (host/host_qwen_8x64.cpp:110-118, model_shape_t). */
typedef struct {
    uint32_t vocab_size;
    uint32_t hidden_size;
    uint32_t intermediate_size;
    uint32_t num_layers;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t max_seq_len;
} orc_shape_t;

/* Projection ids, in the reference's packed order (host:325-376). */
enum {
    ORC_PROJ_Q = 0,
    ORC_PROJ_K = 1,
    ORC_PROJ_V = 2,
    ORC_PROJ_O = 3,
    ORC_PROJ_GATE = 4,
    ORC_PROJ_UP = 5,
    ORC_PROJ_DOWN = 6,
    ORC_PROJ_COUNT = 7
};

/* hls::exp candidate policies (the library itself is absent here). */
enum {
    ORC_EXP_FLOOR = 0, /* floor(e^x * 2^F)                              */
    ORC_EXP_ROUND = 1, /* floor(e^x * 2^F + 1/2)                        */
    ORC_EXP_HLS = 2    /* the reference's instantiations (default):
                          Q8.8 = three-table hls::exp<16,8> restatement,
                          Q2.14 = floor(e^x * 2^14) (hls::exp<18,4>)   */
};

/* uniform_int_distribution<int> algorithms of libstdc++. */
enum {
    ORC_UID_DIVREJ = 0, /* libstdc++ <= 10: divide and reject        */
    ORC_UID_LEMIRE = 1  /* libstdc++ >= 11: Lemire nearly-divisionless */
};

/* ---- exp tables ------------------------------------------------------ */
void orc_set_exp_policy(int q8_8_policy, int q2_14_policy);
/* golden_exp (host:578-586): Q8.8 in, Q8.8 out. */
int16_t orc_exp_q8_8(int16_t x);
/* golden_attention_probability (host:588-596): Q8.8 in, Q2.14 out. */
int16_t orc_attn_prob(int16_t x);
/* Install explicit tables (q8_8: x raw -2048..2048, 4097 entries;
 * q2_14: x raw -2048..0, 2049 entries); NULL keeps a table. */
void orc_set_exp_tables(const int16_t* q8_8, const int16_t* q2_14);
/* Copy the 2049-entry tables for x = -8 .. 0 (raw -2048 .. 0). */
void orc_get_exp_tables(int16_t* q8_8_table, int16_t* q2_14_table);

/* ---- scalar primitives ---------------------------------------------- */
int16_t orc_recip(int16_t x);          /* golden_recip host:537-576   */
int16_t orc_rsqrt(int32_t v);          /* golden_rsqrt host:621-656   */
int16_t orc_silu(int16_t x);           /* golden_silu  host:658-668   */
int16_t orc_quantize_fix16(double v);  /* quantize_fix16 host:496-505 */
int16_t orc_inv_sum(int32_t sum);      /* fm(accum(1)/max(sum,2^-12)) */
/* rnd(a * golden_weight_t(b), 4): one QK / raw-payload PV product term */
int32_t orc_fm_wt_term(int16_t a, int16_t b);

/* ---- vector / matrix ops -------------------------------------------- */
/* golden_projection (host:3105-3142); w row-major [out_dim][in_dim]. */
void orc_projection(const int16_t* x, uint32_t rows, uint32_t in_dim,
                    const int16_t* w, uint32_t out_dim, int16_t* y);
/* golden_residual (host:3144-3160). */
void orc_residual(const int16_t* a, const int16_t* b, size_t n, int16_t* y);
/* golden_rmsnorm (host:3162-3197). */
void orc_rmsnorm(const int16_t* x, uint32_t rows, uint32_t cols,
                 const int16_t* gamma, int16_t* y);
/* golden_silu_mul (host:3199-3217). */
void orc_silu_mul(const int16_t* gate, const int16_t* up, size_t n,
                  int16_t* y);
/* RoPE table row per position: [cos d/2 | sin d/2], Q8.8
 * (initialize_persistent_auxiliary_data, host:2159-2189). */
void orc_rope_table(uint32_t max_seq, uint32_t head_dim, double theta,
                    int16_t* table);
/* rotate_fix16_pair_with_quantized_rope over `heads` heads
 * (host:4765-4852), using a table row. */
void orc_rope_apply(int16_t* vec, uint32_t heads, uint32_t head_dim,
                    const int16_t* table_row);

/* Tiled online-softmax attention of one GQA group over n cached
 * positions (host:3609-3760).  semantics: 0 = Q2.14 raw payload
 * (production), 1 = Q2.14 direct multiply, 2 = legacy Q8.8 probabilities
 * (golden_tiled_flash_attention, host:3419-3575).  q [G][d], k/v [n][d],
 * out [G][d]. */
void orc_attention(const int16_t* q, uint32_t G, uint32_t d,
                   const int16_t* k, const int16_t* v, uint32_t n,
                   int semantics, int16_t* out);
/* QK scores of one group against one 64-position tile (host:3219-3278). */
void orc_qk_scores(const int16_t* q, uint32_t G, uint32_t d,
                   const int16_t* k, uint32_t n, int16_t* scores);

/* ATTN_PV of one group over one tile: golden_attention_mm(p, v, d, false)
 * (host:3219-3278).  p [G][ldp] Q8.8 (first n used), v [n][d], out [G][d]. */
void orc_attention_pv(const int16_t* p, uint32_t G, uint32_t ldp,
                      const int16_t* v, uint32_t n, uint32_t d, int16_t* out);
/* SOFTMAX rows (kernel/compute_stream.cpp:388-478): x [rows][ldx], first
 * n of each row, out [rows][n]. */
void orc_softmax_rows(const int16_t* x, uint32_t rows, uint32_t ldx,
                      uint32_t n, int16_t* out);

/* ---- model ---------------------------------------------------------- */
typedef struct orc_model orc_model_t;

orc_model_t* orc_model_create(const orc_shape_t* shape, uint32_t kept_layers,
                              int with_embedding);
void orc_model_destroy(orc_model_t* m);
/* Raw access to the row-major arrays. */
int16_t* orc_model_weight(orc_model_t* m, uint32_t layer, uint32_t proj);
int16_t* orc_model_norms(orc_model_t* m);     /* [(2L+1)][H] */
int16_t* orc_model_embedding(orc_model_t* m); /* [vocab][H]  */
uint32_t orc_proj_in_dim(const orc_shape_t* s, uint32_t proj);
uint32_t orc_proj_out_dim(const orc_shape_t* s, uint32_t proj);

/* model_data_t::initialize_random_model (host:842-869): mt19937(seed),
 * embedding U[-128,128], norms U[224,288], 16 packed shards U[-64,64]
 * drawn word by word; weights are scattered through the packed-tile
 * accessor projection_weight_raw (host:899-935).  Draws for every layer
 * of the shape are consumed; only kept_layers are stored. */
void orc_model_init_reference_random(orc_model_t* m, uint32_t seed,
                                     int uid_algorithm);
/* Weights from the reference's 16 packed shards (the layout
 * projection_weight_raw reads, host:899-935): shard i is `shard_words`
 * words of 32 int16 lanes.  Returns -1 when shard_words is too small. */
int orc_model_load_shards(orc_model_t* m, const int16_t* const shards[16],
                          uint64_t shard_words);
/* The 16 weight shards initialize_random_model fills (host:842-869), in
 * the reference's draw order (the embedding and norm draws are consumed
 * first); shard_words must equal orc_shard_words(s). */
int orc_reference_random_shards(const orc_shape_t* s, uint32_t seed, int alg,
                                uint64_t shard_words, int16_t* const out[16]);
/* Words per shard of a shape: ceil(layers * tiles per layer / 2). */
uint64_t orc_shard_words(const orc_shape_t* s);
/* make_random_tensor (host:3089-3103). */
void orc_make_random_tensor(uint32_t rows, uint32_t cols, uint32_t seed,
                            int32_t lo, int32_t hi, int uid_algorithm,
                            int16_t* out);
/* model_data_t::lm_head_argmax (host:937-969) over a [vocab][H] table. */
uint32_t orc_lm_head_argmax(const int16_t* table, uint32_t vocab,
                            uint32_t hidden, const int16_t* h);
/* tensor_checksum, FNV-1a-64 over uint16 values (host:8542-8549). */
uint64_t orc_checksum(const int16_t* v, size_t n);
/* n-th output (1-based) of std::mt19937(seed). */
uint32_t orc_mt19937_nth(uint32_t seed, uint64_t n);
/* n draws of uniform_int_distribution<int>(lo, hi) from mt19937(seed). */
void orc_uniform_ints(uint32_t seed, int32_t lo, int32_t hi, int alg,
                      size_t n, int32_t* out);
/* OpenMP threads for projections (0 = runtime default, 1 = serial). */
void orc_set_threads(int n);

/* ---- incremental resident tasks ------------------------------------- */
/* KV cache arrays are [layer][kv_head][max_seq][d] int16 (logical). */
typedef struct {
    uint32_t op, code, token_count, output_waves;
    uint32_t mm_tasks, vector_tasks, completed_packets, last_task;
} orc_status_t;

/* One coarse task (control_cache_8x64.cpp:5767-6481 / golden composition
 * host:4854-5017): op 18 (attention sublayer), 19 (FFN sublayer),
 * 20 (final RMSNorm), 16 (18 then 19).  in/out are [rows][H].  `semantics`
 * selects the attention arithmetic as in orc_attention.  Returns the
 * reference status code. */
int orc_task(const orc_model_t* m, int16_t* kcache, int16_t* vcache,
             uint32_t op, uint32_t layer, uint32_t token_count,
             uint32_t position, const int16_t* in, int16_t* out,
             int semantics, orc_status_t* status);

/* golden_prefill_decoder_layer_sequence (host:4854-4978) at position 0,
 * rows = all positions (full-prefix recompute).  post_attention may be
 * NULL.  Uses its own temporary KV. */
void orc_prefill_layer_sequence(const orc_model_t* m, const int16_t* hidden,
                                uint32_t rows, uint32_t layer, int semantics,
                                int16_t* post_attention, int16_t* out);

#ifdef __cplusplus
}
#endif
#endif
