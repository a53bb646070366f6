/*
 * fake_sampler.c - a host stand-in for the sampler C ABI, built only by the
 * tests (tests/test_c_host.py), so that the C host logic above the ABI
 * (pss_generate.c, the INTEGRATION.md snippet) runs on the CPU under
 * AddressSanitizer.  "Device" pointers are host pointers here; every step
 * runs the O1 oracle row by row with the sampler's per-row state, as the GPU
 * kernels do.  Entry points the loops under test do not reach return
 * PSS_ERR_UNSUPPORTED.
 */
#include <stdlib.h>
#include <string.h>

#include "pss_oracle.h"
#include "pumice_sampler.h"

struct pss_sampler {
    uint32_t V, max_rows;
    sample_params* params;
    uint32_t *rng, *step, *pos, *hist, *result, *tokens;
};

pss_status pss_create(pss_sampler** out, uint32_t vocab, uint32_t max_rows, void* stream) {
    (void)stream;
    if (!out || vocab == 0 || max_rows == 0) return PSS_ERR_INVALID_ARG;
    pss_sampler* s = (pss_sampler*)calloc(1, sizeof *s);
    if (!s) return PSS_ERR_ALLOC;
    s->V = vocab;
    s->max_rows = max_rows;
    s->params = (sample_params*)calloc(max_rows, sizeof(sample_params));
    s->rng = (uint32_t*)calloc(max_rows, 4);
    s->step = (uint32_t*)calloc(max_rows, 4);
    s->pos = (uint32_t*)calloc(max_rows, 4);
    s->tokens = (uint32_t*)calloc(max_rows, 4);
    s->result = (uint32_t*)calloc((size_t)max_rows * PSS_RESULT_SLOTS, 4);
    s->hist = (uint32_t*)malloc((size_t)max_rows * PSS_MAX_PENALTY_LEN * 4);
    if (!s->params || !s->rng || !s->step || !s->pos || !s->tokens || !s->result || !s->hist) {
        pss_destroy(s);
        return PSS_ERR_ALLOC;
    }
    memset(s->hist, 0xFF, (size_t)max_rows * PSS_MAX_PENALTY_LEN * 4);
    *out = s;
    return PSS_OK;
}

pss_status pss_destroy(pss_sampler* s) {
    if (!s) return PSS_ERR_INVALID_ARG;
    free(s->params);
    free(s->rng);
    free(s->step);
    free(s->pos);
    free(s->tokens);
    free(s->result);
    free(s->hist);
    free(s);
    return PSS_OK;
}

static int rows_ok(const pss_sampler* s, uint32_t row0, uint32_t rows) {
    return s && rows > 0 && row0 < s->max_rows && rows <= s->max_rows - row0;
}

pss_status pss_set_params(pss_sampler* s, uint32_t row0, uint32_t rows, const sample_params* params,
                          const uint32_t* seeds) {
    if (!rows_ok(s, row0, rows) || !params) return PSS_ERR_INVALID_ARG;
    memcpy(s->params + row0, params, rows * sizeof(sample_params));
    for (uint32_t i = 0; i < rows; ++i) {
        s->rng[row0 + i] = seeds ? seeds[i] : 0u;
        s->step[row0 + i] = 0u;
    }
    return PSS_OK;
}

pss_status pss_reset_history(pss_sampler* s, uint32_t row0, uint32_t rows, uint32_t fill) {
    if (!rows_ok(s, row0, rows)) return PSS_ERR_INVALID_ARG;
    for (size_t i = (size_t)row0 * PSS_MAX_PENALTY_LEN; i < (size_t)(row0 + rows) * PSS_MAX_PENALTY_LEN; ++i)
        s->hist[i] = fill;
    return PSS_OK;
}

pss_status pss_set_history(pss_sampler* s, uint32_t row0, uint32_t rows, const uint32_t* hist,
                           uint32_t count) {
    if (!rows_ok(s, row0, rows) || !hist || count > PSS_MAX_PENALTY_LEN) return PSS_ERR_INVALID_ARG;
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t k = 0; k < PSS_MAX_PENALTY_LEN; ++k)
            s->hist[(size_t)(row0 + r) * PSS_MAX_PENALTY_LEN + k] = k < count ? hist[(size_t)r * count + k] : 0xFFFFFFFFu;
    return PSS_OK;
}

pss_status pss_set_position(pss_sampler* s, uint32_t row0, uint32_t rows, const uint32_t* pos) {
    if (!rows_ok(s, row0, rows) || !pos) return PSS_ERR_INVALID_ARG;
    memcpy(s->pos + row0, pos, 4u * rows);
    return PSS_OK;
}

pss_status pss_enqueue(pss_sampler* s, const void* logits, uint32_t dtype, uint64_t row_stride,
                       uint32_t rows, uint32_t mode, uint32_t do_increment, uint32_t pass_idx,
                       uint32_t rng_mode) {
    if (!s || !logits || rows == 0 || rows > s->max_rows || dtype != PSS_DTYPE_F32 ||
        (mode != PSS_MODE_GREEDY && mode != PSS_MODE_SAMPLE) || pass_idx >= PSS_RESULT_SLOTS ||
        row_stride < s->V)
        return PSS_ERR_INVALID_ARG;
    for (uint32_t r = 0; r < rows; ++r) {
        oracle_row_state st = {s->hist + (size_t)r * PSS_MAX_PENALTY_LEN, s->pos[r], s->rng[r], s->step[r]};
        const uint32_t tok = oracle_o1_row((const float*)logits + (size_t)r * row_stride, s->V, &s->params[r], &st,
                                           r, mode, rng_mode, do_increment, NULL, NULL, NULL, NULL, NULL);
        s->pos[r] = st.position;
        s->rng[r] = st.rng;
        s->step[r] = st.step;
        s->tokens[r] = tok;
        s->result[(size_t)r * PSS_RESULT_SLOTS + pass_idx] = tok;
    }
    return PSS_OK;
}

pss_status pss_enqueue_ex(pss_sampler* s, const void* logits, uint32_t dtype, uint64_t row_stride,
                          uint32_t rows, uint32_t mode, uint32_t do_increment, uint32_t pass_idx,
                          uint32_t rng_mode, const pss_enqueue_opts* opts) {
    if (opts && (opts->flags || opts->row_info || opts->kept_mask || opts->probs || opts->host_tokens))
        return PSS_ERR_UNSUPPORTED;
    return pss_enqueue(s, logits, dtype, row_stride, rows, mode, do_increment, pass_idx, rng_mode);
}

pss_status pss_read_results(pss_sampler* s, uint32_t rows, uint32_t* results, uint32_t* tokens) {
    if (!s || rows == 0 || rows > s->max_rows) return PSS_ERR_INVALID_ARG;
    if (results) memcpy(results, s->result, 4u * rows * PSS_RESULT_SLOTS);
    if (tokens) memcpy(tokens, s->tokens, 4u * rows);
    return PSS_OK;
}

pss_status pss_read_state(pss_sampler* s, uint32_t rows, uint32_t* history, uint32_t* position,
                          uint32_t* rng, uint32_t* step) {
    if (!s || rows == 0 || rows > s->max_rows) return PSS_ERR_INVALID_ARG;
    if (history) memcpy(history, s->hist, 4u * rows * PSS_MAX_PENALTY_LEN);
    if (position) memcpy(position, s->pos, 4u * rows);
    if (rng) memcpy(rng, s->rng, 4u * rows);
    if (step) memcpy(step, s->step, 4u * rows);
    return PSS_OK;
}

pss_status pss_reset_gate(pss_sampler* s) {
    (void)s;
    return PSS_ERR_UNSUPPORTED;
}

pss_status pss_set_score_targets(pss_sampler* s, uint32_t row0, uint32_t rows, uint32_t slots,
                                 const uint32_t* ids) {
    (void)s, (void)row0, (void)rows, (void)slots, (void)ids;
    return PSS_ERR_UNSUPPORTED;
}
