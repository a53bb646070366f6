/*
 * snippet_harness.c - INTEGRATION.md's drop-in snippet (snippet.c, extracted
 * from the document by extract_snippet.py) linked to the real sampler
 * library, for tests/test_gpu_integration_snippet.py: one request as the
 * reference runs it -- generatorSetSampling, resetGenerator's zero-filled
 * window, the prefill-final pass at position P, then decode groups of four
 * passes -- with the tokens and the final state handed back to the test.
 */
#include "snippet.c"

int snippet_chain(uint32_t vocab, const sample_params* p, uint32_t seed, uint32_t P,
                  const void* const* logits_dev, uint32_t ngroups, uint32_t* tokens_out,
                  uint32_t* history_out, uint32_t* state_out /* position, rng, step */) {
    generator g;
    pss_status st = generatorCreateSampler(&g, vocab);
    if (st != PSS_OK) return (int)st;
    if (st == PSS_OK) st = generatorSetSampling(&g, p, seed);
    if (st == PSS_OK) st = resetGeneratorWindow(&g);
    if (st == PSS_OK) st = prefillFinalPass(&g, logits_dev[0], P, &tokens_out[0]);
    for (uint32_t k = 0; k < ngroups && st == PSS_OK; ++k) {
        uint32_t grp[PSS_RESULT_SLOTS];
        st = decodeGroup(&g, logits_dev + 1 + PSS_RESULT_SLOTS * k, PSS_RESULT_SLOTS, grp);
        for (uint32_t j = 0; j < PSS_RESULT_SLOTS; ++j) tokens_out[1 + PSS_RESULT_SLOTS * k + j] = grp[j];
    }
    if (st == PSS_OK) st = pss_read_state(g.smp, 1, history_out, &state_out[0], &state_out[1], &state_out[2]);
    const pss_status d = pss_destroy(g.smp);
    return (int)(st != PSS_OK ? st : d);
}
