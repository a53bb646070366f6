/*
 * host_main.c - the C host logic above the sampler ABI, run on the CPU
 * against fake_sampler.c (O1 behind the ABI) under AddressSanitizer and
 * UBSan by tests/test_c_host.py:
 *   1. INTEGRATION.md's snippet (snippet.c, extracted from the document):
 *      generatorSetSampling -> resetGeneratorWindow (zero fill) ->
 *      prefillFinalPass -> two decode groups (4 and 3 passes);
 *   2. pgl_generate (pss_generate.c) over two rows, 11 tokens.
 * Each is compared with a direct O1 chain over the same logits (tokens and
 * final state).  Exit status 0 when everything matches.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pss_oracle.h"
#include "pumice_generate.h"
#include "snippet.c"

#define V 4099u
#define NPASS 12u

static uint64_t lcg = 0x9E3779B97F4A7C15ull;
static double urand(void) {
    lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
    return ((lcg >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}
static float nrand(void) { return (float)(3.0 * sqrt(-2.0 * log(urand())) * cos(6.283185307179586 * urand())); }

static int fails = 0;
#define CHECK(c, ...) do { if (!(c)) { fprintf(stderr, __VA_ARGS__); fputc('\n', stderr); ++fails; } } while (0)

static int emit_count = 0;
static uint32_t emitted[64];
static int emit_cb(void* ctx, uint32_t tok) {
    (void)ctx;
    if (emit_count < 64) emitted[emit_count] = tok;
    ++emit_count;
    return 0;
}

int main(void) {
    float* x = (float*)malloc(sizeof(float) * (size_t)NPASS * 2u * V); /* [pass][row][V] */
    uint32_t* hist = (uint32_t*)malloc(4u * PSS_MAX_PENALTY_LEN);
    uint32_t* hist2 = (uint32_t*)malloc(4u * 2u * PSS_MAX_PENALTY_LEN);
    if (!x || !hist || !hist2) return 2;
    for (size_t i = 0; i < (size_t)NPASS * 2u * V; ++i) x[i] = nrand();
    sample_params p = {0.8f, 1.1f, 64u, 40u, 0.95f, 0.05f, 0.5f};
    const void* rowp[NPASS];
    for (uint32_t k = 0; k < NPASS; ++k) rowp[k] = x + (size_t)k * 2u * V;

    /* 1. the snippet: seed 7, zero-filled window, prefill at P = 5, groups of 4 and 3 */
    generator g;
    CHECK(generatorCreateSampler(&g, V) == PSS_OK, "create");
    CHECK(generatorSetSampling(&g, &p, 7u) == PSS_OK, "set sampling");
    CHECK(resetGeneratorWindow(&g) == PSS_OK, "reset window");
    uint32_t got[8], t0 = 0;
    CHECK(prefillFinalPass(&g, rowp[0], 5u, &t0) == PSS_OK, "prefill");
    got[0] = t0;
    uint32_t grp[PSS_RESULT_SLOTS];
    CHECK(decodeGroup(&g, rowp + 1, 4u, grp) == PSS_OK, "group 1");
    for (int k = 0; k < 4; ++k) got[1 + k] = grp[k];
    CHECK(decodeGroup(&g, rowp + 5, 3u, grp) == PSS_OK, "group 2");
    for (int k = 0; k < 3; ++k) got[5 + k] = grp[k];
    /* the O1 chain */
    memset(hist, 0, 4u * PSS_MAX_PENALTY_LEN);
    oracle_row_state st = {hist, 5u, 7u, 0u};
    for (uint32_t k = 0; k < 8; ++k) {
        const uint32_t want = oracle_o1_row((const float*)rowp[k], V, &p, &st, 0u, PSS_MODE_SAMPLE,
                                            PSS_RNG_XORSHIFT32, k == 0 ? 0u : 1u, NULL, NULL, NULL, NULL, NULL);
        CHECK(got[k] == want, "snippet pass %u: token %u, O1 %u", k, got[k], want);
    }
    uint32_t pos = 0, rng = 0, step = 0;
    CHECK(pss_read_state(g.smp, 1, hist2, &pos, &rng, &step) == PSS_OK, "read state");
    CHECK(pos == st.position && rng == st.rng && step == st.step, "snippet state: pos %u/%u rng %u/%u", pos,
          st.position, rng, st.rng);
    CHECK(memcmp(hist2, hist, 4u * PSS_MAX_PENALTY_LEN) == 0, "snippet history ring");
    pss_destroy(g.smp);

    /* 2. pgl_generate: two rows stepped together, row 0 emitted, 11 tokens */
    pss_sampler* s = NULL;
    CHECK(pss_create(&s, V, 2, NULL) == PSS_OK, "create 2");
    sample_params pp[2] = {p, p};
    pp[1].topK = 5u;
    const uint32_t seeds[2] = {11u, 12u};
    CHECK(pss_set_params(s, 0, 2, pp, seeds) == PSS_OK, "params 2");
    CHECK(pss_reset_history(s, 0, 2, 0xFFFFFFFFu) == PSS_OK, "reset 2");
    pgl_logits_table tab = {rowp, NPASS};
    pgl_config cfg = {11u, 0xFFFFFFFFu, 2u, PSS_DTYPE_F32, V, PSS_MODE_SAMPLE, PSS_RNG_XORSHIFT32, 3u};
    pgl_result res;
    CHECK(pgl_generate(s, &cfg, pgl_table_logits, &tab, emit_cb, NULL, &res) == PSS_OK, "pgl_generate");
    CHECK(res.emitted == 11u && emit_count == 11, "emitted %u", res.emitted);
    memset(hist2, 0xFF, 4u * 2u * PSS_MAX_PENALTY_LEN);
    oracle_row_state s0 = {hist2, 3u, 11u, 0u}, s1 = {hist2 + PSS_MAX_PENALTY_LEN, 3u, 12u, 0u};
    for (uint32_t k = 0; k < 11u; ++k) {
        /* pass k reads the logits at position start_pos + k (the table wraps) */
        const float* l = (const float*)rowp[(3u + (k == 0 ? 0u : k - 1u)) % NPASS];
        const uint32_t w0 = oracle_o1_row(l, V, &pp[0], &s0, 0u, PSS_MODE_SAMPLE, PSS_RNG_XORSHIFT32,
                                          k == 0 ? 0u : 1u, NULL, NULL, NULL, NULL, NULL);
        (void)oracle_o1_row(l + V, V, &pp[1], &s1, 1u, PSS_MODE_SAMPLE, PSS_RNG_XORSHIFT32, k == 0 ? 0u : 1u,
                            NULL, NULL, NULL, NULL, NULL);
        CHECK(emitted[k] == w0, "pgl_generate token %u: %u, O1 %u", k, emitted[k], w0);
    }
    uint32_t pos2[2], rng2[2], step2[2];
    uint32_t* h2 = (uint32_t*)malloc(4u * 2u * PSS_MAX_PENALTY_LEN);
    CHECK(h2 && pss_read_state(s, 2, h2, pos2, rng2, step2) == PSS_OK, "read state 2");
    CHECK(pos2[0] == s0.position && pos2[1] == s1.position && rng2[0] == s0.rng && rng2[1] == s1.rng,
          "pgl_generate state");
    CHECK(h2 && memcmp(h2, hist2, 4u * 2u * PSS_MAX_PENALTY_LEN) == 0, "pgl_generate history rings");
    free(h2);
    pss_destroy(s);
    free(x);
    free(hist);
    free(hist2);
    if (fails) fprintf(stderr, "%d check(s) failed\n", fails);
    else printf("host logic ok: snippet 8 passes, pgl_generate 11 tokens match O1\n");
    return fails ? 1 : 0;
}
