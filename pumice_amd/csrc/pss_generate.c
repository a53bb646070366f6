/*
 * pss_generate.c - C generate-loop call site of the sampler
 * (include/pumice_generate.h).  Mirrors the token-consumption structure of
 * src/generate.c:1027-1159: a prefill-final pass (runPrefill's finalOps,
 * doIncrement 0, :640-644 / :1009-1016), then decode groups of DECODE_GROUP
 * passes whose result slots are read back per group (:1118-1156).  Plain C over
 * the sampler C ABI; no HIP types.
 */
#define _POSIX_C_SOURCE 199309L
#include "pumice_generate.h"

#include <stddef.h>
#include <string.h>
#include <time.h>

static double now_us(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec * 1e6 + (double)ts.tv_nsec * 1e-3;
}

const void* pgl_table_logits(void* ctx, uint32_t position) {
    const pgl_logits_table* t = (const pgl_logits_table*)ctx;
    return t->rows[position % t->count];
}

pss_status pgl_generate(pss_sampler* s, const pgl_config* cfg, pgl_logits_fn logits, void* lctx,
                        pgl_emit_fn emit, void* ectx, pgl_result* out) {
    if (!s || !cfg || !logits || !emit || !out || cfg->max_new == 0 || cfg->rows == 0 ||
        cfg->rows > 256)
        return PSS_ERR_INVALID_ARG;
    pgl_result r = {0, 1, 0, 0.0};
    double t0 = now_us();
    uint32_t pos = cfg->start_pos;
    uint32_t results[256 * PGL_DECODE_GROUP];
    pss_status st;

    /* prefill-final pass: slot 0, no position increment (generate.c:642) */
    uint32_t posv[256];
    for (uint32_t i = 0; i < cfg->rows; ++i) posv[i] = pos;
    st = pss_set_position(s, 0, cfg->rows, posv);
    if (st != PSS_OK) return st;
    st = pss_enqueue(s, logits(lctx, pos), cfg->dtype, cfg->row_stride, cfg->rows, cfg->mode, 0, 0,
                     cfg->rng_mode);
    if (st != PSS_OK) return st;
    st = pss_read_results(s, cfg->rows, results, NULL);
    if (st != PSS_OK) return st;
    uint32_t tok = results[0];
    r.emitted = 1;
    int stop = emit(ectx, tok);
    if (tok == cfg->eos || stop) {
        r.finish_reason = 0;
        r.wall_us = now_us() - t0;
        *out = r;
        return PSS_OK;
    }

    uint32_t remaining = cfg->max_new - 1;
    while (remaining > 0) {
        uint32_t cur = remaining < PGL_DECODE_GROUP ? remaining : PGL_DECODE_GROUP;
        for (uint32_t p = 0; p < cur; ++p) {
            st = pss_enqueue(s, logits(lctx, pos + p), cfg->dtype, cfg->row_stride, cfg->rows,
                             cfg->mode, 1, p, cfg->rng_mode);
            if (st != PSS_OK) return st;
        }
        r.groups++;
        st = pss_read_results(s, cfg->rows, results, NULL);
        if (st != PSS_OK) return st;
        pos += cur;
        for (uint32_t j = 0; j < cur; ++j) {
            tok = results[j]; /* row 0, slot j */
            r.emitted++;
            remaining--;
            stop = emit(ectx, tok);
            if (tok == cfg->eos || stop) {
                r.finish_reason = 0;
                remaining = 0;
                break;
            }
        }
    }
    r.wall_us = now_us() - t0;
    *out = r;
    return PSS_OK;
}

/* Spin until pinned[0] differs from the sentinel; 0 when it landed, else the
 * stream's status after 2 s (a failed stream reports it; otherwise
 * PSS_ERR_HIP). */
static pss_status wait_token(pss_sampler* s, uint32_t rows, volatile uint32_t* pinned) {
    double t0 = 0.0;
    for (uint32_t n = 1;; ++n) {
        if (__atomic_load_n(pinned, __ATOMIC_ACQUIRE) != 0xFFFFFFFFu) return PSS_OK;
        if ((n & 4095u) == 0u) {
            const double t = now_us();
            if (t0 == 0.0) t0 = t;
            else if (t - t0 > 2e6) {
                const pss_status st = pss_read_results(s, rows, NULL, NULL);
                if (__atomic_load_n(pinned, __ATOMIC_ACQUIRE) != 0xFFFFFFFFu) return PSS_OK;
                return st != PSS_OK ? st : PSS_ERR_HIP;
            }
        }
    }
}

pss_status pgl_generate_pinned(pss_sampler* s, const pgl_config* cfg, pgl_logits_fn logits, void* lctx,
                               pgl_emit_fn emit, void* ectx, uint32_t* pinned_dev,
                               volatile uint32_t* pinned_host, pgl_result* out) {
    if (!s || !cfg || !logits || !emit || !out || !pinned_dev || !pinned_host || cfg->max_new == 0 ||
        cfg->rows == 0 || cfg->rows > 256)
        return PSS_ERR_INVALID_ARG;
    const uint32_t rows = cfg->rows;
    pgl_result r = {0, 1, 0, 0.0};
    double t0 = now_us();
    uint32_t pos = cfg->start_pos;
    pss_status st;
    pss_enqueue_opts o = {NULL, NULL, NULL, 0, NULL, 0, NULL, 0, 0};

    /* prefill-final pass: slot 0, no position increment (generate.c:642) */
    uint32_t posv[256];
    for (uint32_t i = 0; i < rows; ++i) posv[i] = pos;
    st = pss_set_position(s, 0, rows, posv);
    if (st != PSS_OK) return st;
    pinned_host[0] = 0xFFFFFFFFu;
    __atomic_thread_fence(__ATOMIC_SEQ_CST);
    o.host_tokens = pinned_dev;
    st = pss_enqueue_ex(s, logits(lctx, pos), cfg->dtype, cfg->row_stride, rows, cfg->mode, 0, 0,
                        cfg->rng_mode, &o);
    if (st != PSS_OK) return st;
    st = wait_token(s, rows, &pinned_host[0]);
    if (st != PSS_OK) return st;
    uint32_t tok = pinned_host[0];
    r.emitted = 1;
    int stop = emit(ectx, tok);
    if (tok == cfg->eos || stop) {
        r.finish_reason = 0;
        r.wall_us = now_us() - t0;
        *out = r;
        return pss_read_results(s, rows, NULL, NULL);
    }

    uint32_t remaining = cfg->max_new - 1;
    while (remaining > 0) {
        uint32_t cur = remaining < PGL_DECODE_GROUP ? remaining : PGL_DECODE_GROUP;
        for (uint32_t p = 0; p < cur; ++p) pinned_host[p * rows] = 0xFFFFFFFFu;
        __atomic_thread_fence(__ATOMIC_SEQ_CST);
        for (uint32_t p = 0; p < cur; ++p) {
            o.host_tokens = pinned_dev + p * rows;
            st = pss_enqueue_ex(s, logits(lctx, pos + p), cfg->dtype, cfg->row_stride, rows, cfg->mode, 1,
                                p, cfg->rng_mode, &o);
            if (st != PSS_OK) return st;
        }
        r.groups++;
        st = wait_token(s, rows, &pinned_host[(cur - 1) * rows]);
        if (st != PSS_OK) return st;
        pos += cur;
        for (uint32_t j = 0; j < cur; ++j) {
            tok = pinned_host[j * rows]; /* row 0, pass j */
            r.emitted++;
            remaining--;
            stop = emit(ectx, tok);
            if (tok == cfg->eos || stop) {
                r.finish_reason = 0;
                remaining = 0;
                break;
            }
        }
    }
    r.wall_us = now_us() - t0;
    *out = r;
    /* the state writes of the last passes are stream-ordered: wait for them */
    return pss_read_results(s, rows, NULL, NULL);
}

pss_status pgl_score(pss_sampler* s, pgl_logits_fn logits, void* lctx, uint32_t dtype, uint64_t row_stride,
                     const uint32_t* ids, uint32_t n, uint32_t start_pos, double* loss_sum, uint64_t* count) {
    if (!s || !logits || (!ids && n) || !loss_sum || !count) return PSS_ERR_INVALID_ARG;
    double sum = 0.0;
    uint64_t cnt = 0;
    uint32_t posv[1] = {start_pos};
    pss_status st = pss_set_position(s, 0, 1, posv);
    if (st != PSS_OK) return st;
    uint32_t results[PSS_RESULT_SLOTS];
    for (uint32_t j = 0; j < n; j += PGL_DECODE_GROUP) {
        const uint32_t cur = n - j < PGL_DECODE_GROUP ? n - j : PGL_DECODE_GROUP;
        st = pss_set_score_targets(s, 0, 1, cur, ids + j);
        if (st != PSS_OK) return st;
        for (uint32_t p = 0; p < cur; ++p) {
            st = pss_enqueue(s, logits(lctx, start_pos + j + p), dtype, row_stride, 1, PSS_MODE_SCORE, 1, p,
                             PSS_RNG_XORSHIFT32);
            if (st != PSS_OK) return st;
        }
        st = pss_read_results(s, 1, results, NULL);
        if (st != PSS_OK) return st;
        for (uint32_t p = 0; p < cur; ++p) {
            float loss;
            memcpy(&loss, &results[p], sizeof loss);
            sum += (double)loss;
            cnt++;
        }
    }
    *loss_sum = sum;
    *count = cnt;
    return PSS_OK;
}

pss_status pgl_step_latency(pss_sampler* s, pgl_logits_fn logits, void* lctx, uint32_t dtype,
                            uint64_t row_stride, uint32_t rng_mode, uint32_t steps,
                            uint32_t* pinned_dev, volatile uint32_t* pinned_host, double* lat_us,
                            uint32_t* tokens) {
    if (!s || !logits || !pinned_dev || !pinned_host || !lat_us) return PSS_ERR_INVALID_ARG;
    pss_enqueue_opts o = {NULL, NULL, NULL, 0, pinned_dev, 0, NULL, 0, 0};
    for (uint32_t i = 0; i < steps; ++i) {
        const void* x = logits(lctx, i);
        pinned_host[0] = 0xFFFFFFFFu;
        __atomic_thread_fence(__ATOMIC_SEQ_CST);
        double t0 = now_us();
        pss_status st = pss_enqueue_ex(s, x, dtype, row_stride, 1, PSS_MODE_SAMPLE, 1, 0, rng_mode, &o);
        if (st != PSS_OK) return st;
        uint32_t v;
        /* The kernel stores a token < vocab <= 2^18; the sentinel is never a token. */
        while ((v = __atomic_load_n(pinned_host, __ATOMIC_ACQUIRE)) == 0xFFFFFFFFu) {
        }
        lat_us[i] = now_us() - t0;
        if (tokens) tokens[i] = v;
    }
    /* The kernel's remaining state writes are stream-ordered; wait for them. */
    return pss_read_results(s, 1, NULL, NULL);
}

/* One decode group of the pipelined loop: `cur` gated passes with sequence
 * number `seq`, tokens into the pinned region `reg` (pass p at p * rows). */
static pss_status pipelined_group(pss_sampler* s, const pgl_config* cfg, pgl_logits_fn logits, void* lctx,
                                  uint32_t pos0, uint32_t cur, uint32_t seq, uint32_t* reg_dev,
                                  volatile uint32_t* reg_host) {
    const uint32_t rows = cfg->rows;
    for (uint32_t p = 0; p < cur; ++p) reg_host[p * rows] = 0xFFFFFFFFu;
    __atomic_thread_fence(__ATOMIC_SEQ_CST);
    pss_enqueue_opts o;
    memset(&o, 0, sizeof o);
    o.flags = PSS_ENQ_GATED;
    o.gate_seq = seq;
    o.eos = cfg->eos;
    for (uint32_t p = 0; p < cur; ++p) {
        o.host_tokens = reg_dev + p * rows;
        const pss_status st = pss_enqueue_ex(s, logits(lctx, pos0 + p), cfg->dtype, cfg->row_stride, rows,
                                             cfg->mode, 1, p, cfg->rng_mode, &o);
        if (st != PSS_OK) return st;
    }
    return PSS_OK;
}

pss_status pgl_generate_pipelined(pss_sampler* s, const pgl_config* cfg, pgl_logits_fn logits, void* lctx,
                                  pgl_emit_fn emit, void* ectx, uint32_t* pinned_dev,
                                  volatile uint32_t* pinned_host, pgl_result* out) {
    if (!s || !cfg || !logits || !emit || !out || !pinned_dev || !pinned_host || cfg->max_new == 0 ||
        cfg->rows == 0 || cfg->rows > 256)
        return PSS_ERR_INVALID_ARG;
    const uint32_t rows = cfg->rows;
    pgl_result r = {0, 1, 0, 0.0};
    double t0 = now_us();
    pss_status st = pss_reset_gate(s);
    if (st != PSS_OK) return st;
    uint32_t posv[256];
    for (uint32_t i = 0; i < rows; ++i) posv[i] = cfg->start_pos;
    st = pss_set_position(s, 0, rows, posv);
    if (st != PSS_OK) return st;

    /* prefill-final pass: slot 0, no increment, sequence number 1 */
    pinned_host[0] = 0xFFFFFFFFu;
    __atomic_thread_fence(__ATOMIC_SEQ_CST);
    pss_enqueue_opts o;
    memset(&o, 0, sizeof o);
    o.flags = PSS_ENQ_GATED;
    o.gate_seq = 1u;
    o.eos = cfg->eos;
    o.host_tokens = pinned_dev;
    st = pss_enqueue_ex(s, logits(lctx, cfg->start_pos), cfg->dtype, cfg->row_stride, rows, cfg->mode, 0, 0,
                        cfg->rng_mode, &o);
    if (st != PSS_OK) return st;

    const uint32_t decode = cfg->max_new - 1u;
    const uint32_t ngroups = (decode + PGL_DECODE_GROUP - 1u) / PGL_DECODE_GROUP;
    uint32_t queued = 0;
    /* group g: passes at positions start + 4g + p, region g % 2, sequence 2 + g */
#define PGL_GROUP_CUR(g) (decode - (g) * PGL_DECODE_GROUP < PGL_DECODE_GROUP ? decode - (g) * PGL_DECODE_GROUP \
                                                                              : PGL_DECODE_GROUP)
#define PGL_REGION(g) (rows + ((g) & 1u) * PGL_DECODE_GROUP * rows)
    while (queued < ngroups && queued < 2u) {
        st = pipelined_group(s, cfg, logits, lctx, cfg->start_pos + queued * PGL_DECODE_GROUP, PGL_GROUP_CUR(queued),
                             2u + queued, pinned_dev + PGL_REGION(queued), pinned_host + PGL_REGION(queued));
        if (st != PSS_OK) return st;
        queued++;
    }

    st = wait_token(s, rows, &pinned_host[0]);
    if (st != PSS_OK) return st;
    uint32_t tok = pinned_host[0];
    r.emitted = 1;
    int stop = emit(ectx, tok);
    if (tok == cfg->eos || stop) {
        r.finish_reason = 0;
        r.wall_us = now_us() - t0;
        *out = r;
        return pss_read_results(s, rows, NULL, NULL);
    }
    for (uint32_t g = 0; g < ngroups; ++g) {
        const uint32_t cur = PGL_GROUP_CUR(g);
        volatile uint32_t* reg = pinned_host + PGL_REGION(g);
        st = wait_token(s, rows, &reg[(cur - 1u) * rows]);
        if (st != PSS_OK) return st;
        uint32_t toks[PGL_DECODE_GROUP];
        int eos_seen = 0;
        for (uint32_t j = 0; j < cur; ++j) {
            toks[j] = reg[j * rows]; /* row 0, pass j */
            if (toks[j] == cfg->eos) eos_seen = 1;
        }
        r.groups++;
        if (!eos_seen && queued < ngroups) { /* region g % 2 is free again */
            st = pipelined_group(s, cfg, logits, lctx, cfg->start_pos + queued * PGL_DECODE_GROUP,
                                 PGL_GROUP_CUR(queued), 2u + queued, pinned_dev + PGL_REGION(queued),
                                 pinned_host + PGL_REGION(queued));
            if (st != PSS_OK) return st;
            queued++;
        }
        for (uint32_t j = 0; j < cur; ++j) {
            r.emitted++;
            stop = emit(ectx, toks[j]);
            if (toks[j] == cfg->eos || stop) {
                r.finish_reason = 0;
                r.wall_us = now_us() - t0;
                *out = r;
                return pss_read_results(s, rows, NULL, NULL);
            }
        }
    }
#undef PGL_GROUP_CUR
#undef PGL_REGION
    r.wall_us = now_us() - t0;
    *out = r;
    return pss_read_results(s, rows, NULL, NULL);
}
