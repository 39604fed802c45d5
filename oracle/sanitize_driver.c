/*
 * sanitize_driver.c -- TEST INFRASTRUCTURE ONLY: drives the oracle
 * (llm_oracle.c) through its whole API on small shapes, for a build with
 * AddressSanitizer and UndefinedBehaviorSanitizer (tests/test_oracle_sanitize.py
 * builds `make -C oracle sanitize` into a temporary directory and runs it;
 * any report fails the run).  Exit status 0 and "sanitize OK" on success.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "llm_oracle.h"

static int16_t* alloc16(size_t n) {
    int16_t* p = calloc(n ? n : 1, sizeof(int16_t));
    if (!p) {
        fprintf(stderr, "out of memory\n");
        exit(2);
    }
    return p;
}

/* P8 at position 0, then three decode rows, through every layer; Task 20
 * after each; the LM-head argmax of the last row. */
static uint64_t run_model(const orc_shape_t* s, uint32_t seed, int semantics) {
    const uint32_t H = s->hidden_size, d = H / s->num_heads;
    orc_model_t* m = orc_model_create(s, s->num_layers, 1);
    orc_model_init_reference_random(m, seed, ORC_UID_DIVREJ);
    const size_t kv = (size_t)s->num_layers * s->num_kv_heads * s->max_seq_len * d;
    int16_t *kc = alloc16(kv), *vc = alloc16(kv);
    int16_t *a = alloc16((size_t)8 * H), *b = alloc16((size_t)8 * H);
    orc_make_random_tensor(8, H, seed ^ 0x55u, -48, 48, ORC_UID_DIVREJ, a);
    uint64_t sum = 0;
    orc_status_t st;
    uint32_t pos = 0;
    for (uint32_t step = 0; step < 4; step++) {
        const uint32_t rows = step == 0 ? 8 : 1;
        for (uint32_t l = 0; l < s->num_layers; l++) {
            if (orc_task(m, kc, vc, 18, l, rows, pos, a, b, semantics, &st) ||
                orc_task(m, kc, vc, 19, l, rows, pos, b, a, semantics, &st)) {
                fprintf(stderr, "task failed\n");
                exit(3);
            }
        }
        orc_task(m, kc, vc, 20, 0, rows, pos, a, b, semantics, &st);
        sum ^= orc_checksum(b, (size_t)rows * H);
        const uint32_t tok = orc_lm_head_argmax(orc_model_embedding(m), s->vocab_size, H,
                                                b + (size_t)(rows - 1) * H);
        memcpy(a, orc_model_embedding(m) + (size_t)tok * H, (size_t)H * 2);
        pos += rows;
    }
    /* op 16 and the prefill sequence */
    orc_task(m, kc, vc, 16, 0, 1, pos, a, b, semantics, &st);
    int16_t* seq = alloc16((size_t)8 * H);
    orc_make_random_tensor(8, H, seed ^ 0x77u, -48, 48, ORC_UID_LEMIRE, seq);
    orc_prefill_layer_sequence(m, seq, 8, 0, semantics, a, b);
    sum ^= orc_checksum(b, (size_t)8 * H);
    free(seq);
    free(kc);
    free(vc);
    free(a);
    free(b);
    orc_model_destroy(m);
    return sum;
}

int main(void) {
    /* scalar primitives over their whole int16 ranges */
    int64_t acc = 0;
    for (int32_t x = -32768; x < 32768; x++) {
        acc += orc_recip((int16_t)x) + orc_silu((int16_t)x) + orc_exp_q8_8((int16_t)x) +
               orc_attn_prob((int16_t)x) + orc_fm_wt_term((int16_t)x, (int16_t)(x * 7));
        const int32_t wide = (int32_t)((uint32_t)x * 65537u);
        acc += orc_rsqrt(wide) + orc_inv_sum(wide);
    }
    /* shards: generate, load, and the exact-size words */
    const orc_shape_t small = {64, 64, 128, 2, 4, 2, 32};
    const uint64_t words = orc_shard_words(&small);
    int16_t* shards[16];
    for (int i = 0; i < 16; i++) shards[i] = alloc16((size_t)words * 32);
    orc_reference_random_shards(&small, 20260718u, ORC_UID_DIVREJ, words, shards);
    orc_model_t* m = orc_model_create(&small, 2, 0);
    if (orc_model_load_shards(m, (const int16_t* const*)shards, words) != 0 ||
        orc_model_load_shards(m, (const int16_t* const*)shards, words - 1) == 0) {
        fprintf(stderr, "shard load checks failed\n");
        return 4;
    }
    orc_model_destroy(m);
    for (int i = 0; i < 16; i++) free(shards[i]);
    /* attention in the three semantics beyond one tile */
    const uint32_t G = 4, d = 32, n = 150;
    int16_t *q = alloc16(G * d), *k = alloc16((size_t)n * d), *v = alloc16((size_t)n * d),
            *o = alloc16(G * d);
    orc_make_random_tensor(G, d, 1, -300, 300, ORC_UID_LEMIRE, q);
    orc_make_random_tensor(n, d, 2, -4000, 4000, ORC_UID_LEMIRE, k);
    orc_make_random_tensor(n, d, 3, -4000, 4000, ORC_UID_LEMIRE, v);
    for (int sem = 0; sem < 3; sem++) {
        orc_attention(q, G, d, k, v, n, sem, o);
        acc += orc_checksum(o, G * d) & 0xffff;
    }
    free(q);
    free(k);
    free(v);
    free(o);
    /* models: the small and medium profiles, every attention semantics */
    const orc_shape_t medium = {128, 128, 256, 2, 4, 2, 64};
    uint64_t sum = 0;
    for (int sem = 0; sem < 3; sem++) {
        sum ^= run_model(&small, 20260718u, sem);
        sum ^= run_model(&medium, 7u, sem);
    }
    printf("sanitize OK %lld %016llx\n", (long long)acc, (unsigned long long)sum);
    return 0;
}
