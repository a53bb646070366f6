/*
 * pumice_sampler.h - C ABI of the MI355X (gfx950) token sampler.
 *
 * Drop-in for the reference's on-GPU sampler path:
 *   - sample_params            include/state.h:8-16 (byte-identical layout)
 *   - pss_set_params           generatorSetSampling, src/generate.c:1411-1430
 *   - pss_reset_history        resetGenerator's history reset, src/generate.c:1238-1252
 *   - pss_set_position         stateSetPosition, src/generate.c:993
 *   - pss_enqueue              the "ArgMax-Reduce.spv" operation built by
 *                              buildLmHead, src/generate.c:545-547, executed by
 *                              executeRecord/SubmitNow (src/dispatch.c:272-351)
 *   - pss_read_results         readBuffer(st->result), src/generate.c:1131 /
 *                              src/buffer.c:253-311
 *
 * Conventions
 *   - Every entry point returns a pss_status; nothing calls exit().
 *   - One pss_sampler is used from one host thread.  Work is stream-ordered
 *     and asynchronous: pss_enqueue never synchronizes the device, so step n+1
 *     can be enqueued before the tokens of step n are read.
 *   - The caller owns the logits (device memory, read-only to the sampler).
 *     The sampler owns its per-row state: params, rng, history ring, position,
 *     result slots, token ids.  No device allocation happens after pss_create.
 *   - Rows are independent: row r has its own params, rng stream, history ring
 *     of PSS_MAX_PENALTY_LEN ids, position and result slots.
 */
#ifndef PUMICE_SAMPLER_H
#define PUMICE_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* include/state.h:8-16 — 28 bytes, field order and types unchanged. */
typedef struct {
    float temperature;      /* <= 0 (or NaN): greedy argmax for the row   */
    float repPenalty;       /* CTRL scaling of ids in the window, 1 = off  */
    uint32_t penaltyLength; /* window length, clamped to 1024, 0 = off     */
    uint32_t topK;          /* keep the k largest (ties kept), 0 = off      */
    float topP;             /* nucleus mass, applied iff 0 < topP < 1       */
    float minP;             /* drop p < minP (p relative to the max), <=0 off */
    float presencePenalty;  /* flat subtract for ids in the window, 0 = off */
} sample_params;

#define PSS_MAX_PENALTY_LEN 1024u   /* include/model.h:9 MAX_PENALTY_LEN */
#define PSS_RESULT_SLOTS 4u         /* include/generate.h:12 DECODE_GROUP */
#define PSS_MAX_VOCAB 262144u       /* ArgMax-Reduce.comp:6 PEN_WORDS * 32 */

typedef enum {
    PSS_OK = 0,
    PSS_ERR_INVALID_ARG = 1,  /* bad size, null pointer, out-of-range param */
    PSS_ERR_ALLOC = 2,        /* device or pinned allocation failed */
    PSS_ERR_HIP = 3,          /* a HIP runtime call failed */
    PSS_ERR_UNSUPPORTED = 4,  /* e.g. vocab above PSS_MAX_VOCAB */
    PSS_ERR_NO_DEVICE = 5     /* no usable gfx950 device */
} pss_status;

typedef enum { PSS_DTYPE_F32 = 0, PSS_DTYPE_F16 = 1 } pss_dtype;

/* ArgMax-Reduce.comp push constant `mode` (0 greedy, 1 sample).  SAMPLE picks
 * greedy per row when that row's temperature is not > 0 (generate.c:1418). */
/* PSS_MODE_SCORE: ArgMax-Reduce.comp mode 2 (:169-214), the negative
 * log-likelihood of a given target (pss_set_score_targets) as float bits in
 * the result slot; generateScore, src/generate.c:1161-1236. */
typedef enum { PSS_MODE_GREEDY = 0, PSS_MODE_SAMPLE = 1, PSS_MODE_SCORE = 2 } pss_mode;

/* Uniform source of the draw.
 *   XORSHIFT32: the reference stream: s = rng (0 -> 0x9E3779B9), u = (s>>8)/2^24,
 *               then rng = xorshift32(s)  (ArgMax-Reduce.comp:349-351, :381-383).
 *   PHILOX:     u = (philox4x32_10({step, row, 0, 0}, {seed, 0}).x >> 8) / 2^24,
 *               then step += 1; seed and step are per row. */
typedef enum { PSS_RNG_XORSHIFT32 = 0, PSS_RNG_PHILOX = 1 } pss_rng_mode;

/* Per-row diagnostics, filled when pss_enqueue_opts.row_info is set. */
typedef struct {
    uint32_t token;       /* drawn / argmax id                                 */
    uint32_t kept_count;  /* size of the surviving-candidate set              */
    uint32_t tau_key;     /* order-preserving key of the final value cutoff   */
    uint32_t tmax_key;    /* key of the row maximum of the transformed logits */
    uint64_t z_kept;      /* kept mass, fixed point 2^-45                      */
    uint64_t z_topk;      /* mass of the top-k set, fixed point 2^-45         */
    uint64_t target;      /* draw target: first id with cumulative mass > it  */
    uint32_t u24;         /* 24-bit uniform used by the draw                  */
    uint32_t flags;       /* PSS_INFO_* bits                                   */
} pss_row_info;

#define PSS_INFO_GREEDY 1u     /* row was decoded greedily                    */
#define PSS_INFO_FALLBACK 2u   /* no id crossed the target; last kept id used */
#define PSS_INFO_SCORE 4u      /* scoring pass: z_kept = Zq of all ids, tmax_key = key(gmax) */

typedef struct pss_sampler pss_sampler;

/* Optional outputs for verification (device pointers, each may be NULL). */
typedef struct {
    pss_row_info* row_info;   /* [rows]                                          */
    uint32_t* kept_mask;      /* [rows][mask_words], bit j of row r = id j kept  */
    float* probs;             /* [rows][probs_stride], p_j / Z for kept ids, else 0 */
    uint64_t probs_stride;    /* elements between rows of probs (>= vocab)       */
    uint32_t* host_tokens;    /* device-visible pinned host memory [rows]:
                                 the token of each row is also stored here      */
    uint32_t flags;           /* PSS_ENQ_* bits                                  */
    void* split_event;        /* hipEvent_t recorded on the sampler's stream after
                                 the first kernel of the step (with PSS_ENQ_SPLIT:
                                 per-kernel timing); NULL: none                  */
    uint32_t gate_seq;        /* with PSS_ENQ_GATED: sequence number of the pass's
                                 decode group (> 0, increasing group by group)   */
    uint32_t eos;             /* with PSS_ENQ_GATED: the id that closes the gate */
} pss_enqueue_opts;

/* Run the one-workgroup-per-row general kernel instead of the streaming kernel
 * (both compute identical results; used to cross-check them). */
#define PSS_ENQ_GENERAL 1u
/* The streaming path picks its form by batch size: each row spread over a
 * few workgroups of one round, finished by the last of them to arrive (small
 * batches), or one workgroup per row (large).  These force a form (identical
 * results; used to cross-check them): two kernels (segment kernel over all
 * rows, then a finisher kernel per row), the one-workgroup-per-row kernel, or
 * the small-batch kernel. */
#define PSS_ENQ_SPLIT 2u
#define PSS_ENQ_FUSED 4u
#define PSS_ENQ_SMALL 8u
/* Gated pass (no counterpart in the reference, whose host waits for each
 * decode group before it submits the next): the sampler keeps one device word
 * eos_at (reset by pss_reset_gate).  A gated pass does nothing at all (no
 * output, no state change) if eos_at < opts.gate_seq; when row 0 draws
 * opts.eos it lowers eos_at to opts.gate_seq.  Passes of one decode group
 * share gate_seq, so the rest of the group that drew EOS still runs and every
 * later group is skipped: a caller can queue group n + 1 before it has read
 * group n's tokens and still end in the state of the unpipelined loop. */
#define PSS_ENQ_GATED 16u
/* Force the register-resident form (one workgroup per row holding the whole
 * row in registers; rows of 16-byte aligned fp32 up to 102,400 ids or fp16 up
 * to 106,496 ids, the fused form otherwise).  The automatic choice takes it
 * for batches above the small-batch form's range.  Identical results. */
#define PSS_ENQ_RESIDENT 32u

/* Words per row of kept_mask. */
uint32_t pss_mask_words(uint32_t vocab);

/*
 * Create a sampler for `vocab` ids (<= PSS_MAX_VOCAB) and up to `max_rows` rows
 * on the current HIP device.  `hip_stream` is a hipStream_t; NULL makes the
 * sampler create (and later destroy) its own non-blocking stream.  Histories are filled with the sentinel 0xFFFFFFFF (state.c:101-103),
 * positions, rng states and params are zero.
 */
pss_status pss_create(pss_sampler** out, uint32_t vocab, uint32_t max_rows, void* hip_stream);
pss_status pss_destroy(pss_sampler* s);

/*
 * generatorSetSampling for rows [row0, row0+rows): copies params and seeds.
 * seeds[i] becomes the row's xorshift state and Philox key; the Philox step
 * restarts at 0.  seeds may be NULL (seed 0).  Rejected (PSS_ERR_INVALID_ARG):
 * NaN topP / minP / repPenalty / presencePenalty, and minP > 1 (nothing could be
 * kept).  All other values follow the reference semantics (topK clamped to
 * vocab, penaltyLength clamped to 1024, topP outside (0,1) disables top-p).
 * Stream-ordered.
 */
pss_status pss_set_params(pss_sampler* s, uint32_t row0, uint32_t rows,
                          const sample_params* params, const uint32_t* seeds);

/* Fill the history ring of rows [row0, row0+rows) with `fill`
 * (0xFFFFFFFF = empty; the reference's resetGenerator fills 0). */
pss_status pss_reset_history(pss_sampler* s, uint32_t row0, uint32_t rows, uint32_t fill);

/* Load explicit history windows: hist is [rows][len], len <= 1024; slots at and
 * beyond len are set to the sentinel. */
pss_status pss_set_history(pss_sampler* s, uint32_t row0, uint32_t rows,
                           const uint32_t* hist, uint32_t len);

/*
 * Targets of scoring passes (PSS_MODE_SCORE): ids[r * slots + k] is the token
 * scored by pass slot k (pass_idx = k, 0 <= k < slots <= PSS_RESULT_SLOTS) of
 * row row0 + r.  Replaces the host writes of tokenIds[1 + p] before each
 * group in generateScore (src/generate.c:1190, :1208) and the shader's read
 * of tokenIds[1 + passIdx] (ArgMax-Reduce.comp:196).  Synchronous with the
 * sampler's stream (the caller's array may be reused on return).  Ids >= V
 * score against a logit of 0, as the shader does.
 */
pss_status pss_set_score_targets(pss_sampler* s, uint32_t row0, uint32_t rows, uint32_t slots,
                                 const uint32_t* ids);

pss_status pss_set_position(pss_sampler* s, uint32_t row0, uint32_t rows, const uint32_t* pos);

/*
 * One sampler step over `rows` logit rows (state rows 0..rows-1).
 *   logits      device pointer, row r at logits + r*row_stride elements
 *   dtype       PSS_DTYPE_F32 or PSS_DTYPE_F16
 *   mode        PSS_MODE_SAMPLE (per-row greedy when T <= 0), PSS_MODE_GREEDY, or
 *               PSS_MODE_SCORE (result slot = float bits of the target's NLL,
 *               token = the target; history, rng and step untouched)
 *   do_increment  1: position += 1 after the step (ArgMax-Reduce.comp:384)
 *   pass_idx    result slot 0..3 written (ArgMax-Reduce.comp:377)
 *   rng_mode    pss_rng_mode
 * Per row the step writes result[pass_idx], token_ids, the history ring slot
 * position % W (W = min(penaltyLength, 1024) > 0, sampled rows only), advances
 * the rng (sampled rows only) and the position.
 */
pss_status pss_enqueue(pss_sampler* s, const void* logits, uint32_t dtype, uint64_t row_stride,
                       uint32_t rows, uint32_t mode, uint32_t do_increment, uint32_t pass_idx,
                       uint32_t rng_mode);

pss_status pss_enqueue_ex(pss_sampler* s, const void* logits, uint32_t dtype, uint64_t row_stride,
                          uint32_t rows, uint32_t mode, uint32_t do_increment, uint32_t pass_idx,
                          uint32_t rng_mode, const pss_enqueue_opts* opts);

/* Synchronize the sampler's stream and copy result slots [rows][4] and/or the
 * last token of each row [rows] to host memory (either may be NULL). */
pss_status pss_read_results(pss_sampler* s, uint32_t rows, uint32_t* results, uint32_t* tokens);

/* Re-open the gate of PSS_ENQ_GATED passes (eos_at = 0xFFFFFFFF), stream-ordered. */
pss_status pss_reset_gate(pss_sampler* s);

/* Synchronize and copy per-row state to host (any pointer may be NULL):
 * history [rows][1024], position [rows], rng [rows], philox step [rows]. */
pss_status pss_read_state(pss_sampler* s, uint32_t rows, uint32_t* history, uint32_t* position,
                          uint32_t* rng, uint32_t* step);

/* Device pointers of the state buffers, for consumers on the same stream
 * (e.g. an embedding gather reading token_ids). */
typedef struct {
    uint32_t* result;     /* [max_rows][4]    */
    uint32_t* token_ids;  /* [max_rows]       */
    uint32_t* position;   /* [max_rows]       */
    uint32_t* rng;        /* [max_rows]       */
    uint32_t* step;       /* [max_rows]       */
    uint32_t* history;    /* [max_rows][1024] */
} pss_state_ptrs;

pss_status pss_get_state_ptrs(pss_sampler* s, pss_state_ptrs* out);

/* One sampling or greedy step that allocates nothing (no counterpart in the
 * reference).  For callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * It is pss_enqueue_ex without a sampler object: the caller passes every
 * input and output as device pointers (params [rows], the state buffers of
 * `state` laid out as pss_state_ptrs describes for `rows` rows, logits with
 * `row_stride` elements between rows) and the stream; the workspace of the
 * small-batch form is a per-GPU array inside the library, set up on the first
 * call on each device (the device current at the call).
 *   - rows <= PSS_NOALLOC_MAX_ROWS, else PSS_ERR_INVALID_ARG; modes
 *     PSS_MODE_GREEDY and PSS_MODE_SAMPLE; opts may carry row_info,
 *     kept_mask, probs and host_tokens, but no flags or split_event.
 *   - max_topk / max_window: upper bounds of the rows' topK and
 *     penaltyLength, used only to choose the kernel form (any values give the
 *     same results).
 *   - Calls on one GPU share its workspace: calls that overlap in time on one
 *     GPU (different streams, no ordering between them) race.
 * Same results as pss_enqueue_ex on the same inputs. */
#define PSS_NOALLOC_MAX_ROWS 16u
pss_status pss_enqueue_noalloc(const sample_params* params, const pss_state_ptrs* state, uint32_t vocab,
                               const void* logits, uint32_t dtype, uint64_t row_stride, uint32_t rows,
                               uint32_t mode, uint32_t do_increment, uint32_t pass_idx, uint32_t rng_mode,
                               uint32_t max_topk, uint32_t max_window, const pss_enqueue_opts* opts,
                               void* hip_stream);

/* Host-side request sanitization of the reference's stdin server
 * (src/compute.c:113-114): penaltyLength clamped to 1024, seed 0 -> 1. */
pss_status pss_sanitize_request(sample_params* params, uint32_t* seed);

/* Measurement helper (no counterpart in the reference): the plain read of
 * `bytes` (a multiple of 16, 16-byte aligned) with the resident sampler
 * kernel's access pattern and nothing else -- 1,024-thread workgroups over
 * 400 KiB chunks, 16-byte nontemporal loads -- writing one word per
 * workgroup to out[pss_read_ceiling_blocks(bytes)].  Its rate is the read
 * ceiling the sampler's roofline fraction is set beside. */
uint32_t pss_read_ceiling_blocks(uint64_t bytes);
pss_status pss_read_ceiling(const void* src, uint64_t bytes, uint32_t* out, void* hip_stream);

/* Stream the sampler enqueues on (hipStream_t). */
void* pss_stream(pss_sampler* s);

const char* pss_status_string(pss_status st);

#ifdef __cplusplus
}
#endif

#endif /* PUMICE_SAMPLER_H */
