/*
 * pumice_generate.h - C generate-loop call site of the sampler: the token
 * consumption side of src/generate.c (generateTokens :1027-1159 and the
 * prefill-final pass of runPrefill :1000-1016), driving the sampler C ABI
 * instead of the Vulkan ArgMax-Reduce operation.  The model forward that
 * produces logits is outside this path; a callback supplies the device logits
 * of each pass (the LM-head GEMV output in the reference).
 */
#ifndef PUMICE_GENERATE_H
#define PUMICE_GENERATE_H

#include <stdint.h>

#include "pumice_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PGL_DECODE_GROUP 4u /* include/generate.h:12 DECODE_GROUP */

/* Device logits (one row per sampler row) for the pass at `position`. */
typedef const void* (*pgl_logits_fn)(void* ctx, uint32_t position);
/* A ready-made logits source: ctx is a pgl_logits_table, the pass at
 * `position` reads rows[position % count] (synthetic logits resident on the
 * device, standing in for the LM head). */
typedef struct {
    const void* const* rows;
    uint32_t count;
} pgl_logits_table;
const void* pgl_table_logits(void* ctx, uint32_t position);

/* Called per emitted token of row 0, in order; non-zero asks the loop to stop
 * (generatorRequestStop, src/generate.c:1019-1021). */
typedef int (*pgl_emit_fn)(void* ctx, uint32_t token);

typedef struct {
    uint32_t max_new;    /* maxNewTokens, >= 1                                */
    uint32_t eos;        /* EOS id (0xFFFFFFFF: none)                         */
    uint32_t rows;       /* sampler rows stepped together (row 0 is emitted)  */
    uint32_t dtype;      /* pss_dtype of the logits                           */
    uint64_t row_stride; /* elements between logit rows                       */
    uint32_t mode;       /* pss_mode                                          */
    uint32_t rng_mode;   /* pss_rng_mode                                      */
    uint32_t start_pos;  /* position after the prompt (stateSetPosition)      */
} pgl_config;

typedef struct {
    uint32_t emitted;       /* tokens passed to emit                          */
    uint32_t finish_reason; /* 0 = EOS or stop request, 1 = length            */
    uint32_t groups;        /* decode groups submitted                         */
    double wall_us;         /* host wall time of the whole loop               */
} pgl_result;

/*
 * generateTokens: one prefill-final pass (do_increment 0, slot 0), then decode
 * groups of PGL_DECODE_GROUP passes (do_increment 1, slots 0..3); after each
 * group the host reads the result slots (the reference's readBuffer(result))
 * and emits them, stopping at EOS, at max_new, or when emit asks to stop.
 */
pss_status pgl_generate(pss_sampler* s, const pgl_config* cfg, pgl_logits_fn logits, void* lctx,
                        pgl_emit_fn emit, void* ectx, pgl_result* out);

/*
 * pgl_generate with the tokens delivered through device-visible pinned host
 * memory instead of a copy of the result slots: pass p of a group also
 * stores its rows' tokens at pinned_dev[p * rows + row] (host view
 * pinned_host, at least rows * PGL_DECODE_GROUP u32), and after enqueueing a
 * group the host spins until the last pass's row-0 token lands (passes are
 * stream-ordered, so the earlier ones have landed too).  The result slots are
 * still written on the device.  Same tokens and state as pgl_generate; the
 * group turnaround has no copy and no stream synchronization.  A token that
 * has not landed after 2 s ends the loop with the stream's status (or
 * PSS_ERR_HIP).
 */
pss_status pgl_generate_pinned(pss_sampler* s, const pgl_config* cfg, pgl_logits_fn logits, void* lctx,
                               pgl_emit_fn emit, void* ectx, uint32_t* pinned_dev,
                               volatile uint32_t* pinned_host, pgl_result* out);

/*
 * The decode loop with the next group queued before the current one is read
 * (no counterpart in the reference, which waits for each group before it
 * submits the next, src/generate.c:1139-1149): the prefill-final pass and the
 * first two decode groups are queued at once, and each time the host has read
 * a group's tokens (pinned memory, as pgl_generate_pinned) it queues the group
 * after the next, so the GPU never waits for the host.  The passes are
 * PSS_ENQ_GATED with the group's sequence number and cfg->eos: a group queued
 * after the one whose row 0 drew EOS does nothing, so tokens, result slots and
 * the final state equal pgl_generate's.  A stop asked by `emit` (not EOS, not
 * max_new) comes after up to two groups have been queued beyond it: those
 * groups run and advance the state.  pinned_dev / pinned_host: at least
 * 9 * rows u32 (prefill slot, two group regions).  out->groups counts the
 * groups whose tokens were read.
 */
pss_status pgl_generate_pipelined(pss_sampler* s, const pgl_config* cfg, pgl_logits_fn logits, void* lctx,
                                  pgl_emit_fn emit, void* ectx, uint32_t* pinned_dev,
                                  volatile uint32_t* pinned_host, pgl_result* out);

/*
 * Scoring consumption of generateScore (src/generate.c:1198-1228) for row 0:
 * ids[0..n) are scored in groups of PGL_DECODE_GROUP passes; per group the
 * targets go to the pass slots (pss_set_score_targets, the reference's
 * tokenIds[1 + p] writes), pass p reads the logits at position
 * start_pos + j (j = the id's index) with PSS_MODE_SCORE and do_increment 1,
 * and the group's result slots are read back as float losses and summed in
 * binary64 in id order.  *loss_sum and *count as generateScore's outLoss and
 * outCount.
 */
pss_status pgl_score(pss_sampler* s, pgl_logits_fn logits, void* lctx, uint32_t dtype, uint64_t row_stride,
                     const uint32_t* ids, uint32_t n, uint32_t start_pos, double* loss_sum, uint64_t* count);

/*
 * Launch-to-token latency: `steps` single-row passes; each enqueues with the
 * token also stored into device-visible pinned host memory (`pinned_dev`, whose
 * host view is `pinned_host`) and spins on the host until it lands.
 * lat_us[i] = host time from just before pss_enqueue_ex to the token being
 * visible; tokens[i] = the token.  Row 0 only.
 */
pss_status pgl_step_latency(pss_sampler* s, pgl_logits_fn logits, void* lctx, uint32_t dtype,
                            uint64_t row_stride, uint32_t rng_mode, uint32_t steps,
                            uint32_t* pinned_dev, volatile uint32_t* pinned_host, double* lat_us,
                            uint32_t* tokens);

#ifdef __cplusplus
}
#endif

#endif /* PUMICE_GENERATE_H */
