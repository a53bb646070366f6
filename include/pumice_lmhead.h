/*
 * pumice_lmhead.h - C ABI of the gfx950 LM head: the final RMSNorm fused with
 * the fp16 GEMV over the vocabulary, the step right before the sampler.
 *
 * The reference builds it in buildLmHead (src/generate.c:532-547) as one of two
 * operations over the same weights:
 *   - sampling: "LMHead-GEMV-Q16.spv" (shader/Utility/Q16/LMHead-GEMV-Q16.comp:28-72)
 *     writes raw logits[V] for ArgMax-Reduce mode 1  -> plh_logits;
 *   - greedy:   "LMHead-GEMV-ArgMax-Q16.spv" (LMHead-GEMV-ArgMax-Q16.comp) writes
 *     per-workgroup {maxValue, maxIndex} and ArgMax-Reduce mode 0
 *     (ArgMax-Reduce.comp:135-166) reduces them to the token  -> plh_greedy.
 *
 * Data (as the reference uploads them):
 *   x        fp32 [rows][x_stride]: the final hidden state, K values per row
 *   gamma    fp32 [K]: the final norm's weight
 *   weight   fp16 block-transposed head (src/data.c:305 transpose_block16, FP16):
 *            16-byte block (kb, n) at byte offset (kb * V + n) * 16 holds the 8
 *            halves w[8 kb + j][n], j = 0..7 (the shader's uvec4 B[kb * N + n]);
 *            plh_transpose_block16 builds it from a row-major [K][V] matrix.
 *   logits   fp32 [rows][logits_stride]
 *
 * Arithmetic (identical on every call, so results are reproducible bit for
 * bit):
 *   ss      = sum over k of x[k]^2 in binary64, then rounded to binary32
 *   inv_rms = 1 / sqrtf(ss / K + 1e-6f)                      (binary32, IEEE)
 *   a[k]    = (x[k] * gamma[k]) * inv_rms                     (binary32)
 *   logit   = ((p0 + p1) + p2) + p3, p_s = fmaf chain over the 8-row blocks
 *             kb in [s KB / 4, (s + 1) KB / 4), KB = K / 8, k ascending.
 * The reference accumulates in binary32 in its own order (one chain per column
 * on the GPU, src/validation.c:157-163 / :3898-3910 on the CPU); both are
 * within binary32 rounding of the exact sum.
 *
 * rows > 1 evaluates each row independently (the reference dispatches M = 1).
 * All calls are asynchronous on the head's stream; allocation happens only in
 * plh_create.
 */
#ifndef PUMICE_LMHEAD_H
#define PUMICE_LMHEAD_H

#include <stdint.h>

#include "pumice_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct plh_head plh_head;

/* Columns per workgroup tile and K-slices of the GEMV (fixed: they define the
 * summation order above). */
#define PLH_TILE 64u
#define PLH_SLICES 4u
#define PLH_MAX_K 65536u

/* The head over device-resident weights (not copied; they must outlive the
 * head).  K % 8 == 0, 8 <= K <= PLH_MAX_K, 1 <= V <= PSS_MAX_VOCAB; the
 * workspace holds max_rows normalized rows and the greedy form's per-tile
 * winners.  hip_stream NULL: the head creates its own stream.  Replaces the
 * lmHead / gammaFinal bindings of buildLmHead (src/generate.c:536-542). */
pss_status plh_create(plh_head** out, const void* weight_bt, const float* gamma, uint32_t K, uint32_t V,
                      uint32_t max_rows, void* hip_stream);
pss_status plh_destroy(plh_head* h);

/* RMSNorm + GEMV into logits (LMHead-GEMV-Q16.comp:28-72, dispatched by
 * src/generate.c:536-538); x_stride >= K, logits_stride >= V (elements). */
pss_status plh_logits(plh_head* h, const float* x, uint64_t x_stride, uint32_t rows, float* logits,
                      uint64_t logits_stride);

/* RMSNorm + GEMV + argmax without a logits buffer (LMHead-GEMV-ArgMax-Q16.comp
 * + ArgMax-Reduce.comp mode 0, src/generate.c:540-546): the largest logit's id,
 * lowest id among equal values, NaN never chosen (as pss_enqueue with
 * PSS_MODE_GREEDY on plh_logits' output), written into the sampler's state:
 * result[row][pass_idx] = token, token_ids[row] = token, position[row] +=
 * do_increment.  The sampler must have the head's vocabulary and stream. */
pss_status plh_greedy(plh_head* h, pss_sampler* s, const float* x, uint64_t x_stride, uint32_t rows,
                      uint32_t do_increment, uint32_t pass_idx);

/* Host: block-transpose a row-major fp16 [K][V] head into the layout above
 * (src/data.c:305-331 transpose_block16 with QUANT_FP16). */
pss_status plh_transpose_block16(const uint16_t* w_kv, uint16_t* w_bt, uint32_t K, uint32_t V);

void* plh_stream(plh_head* h);

/* Source row formats of plh_pack_head. */
#define PLH_SRC_BF16 0u
#define PLH_SRC_FP16 1u

/* Host: read a pruned-vocabulary map, pruned-vocab/mapping.npy (int32[V],
 * pruned id -> original id), into out[expected]: NumPy format version 1,
 * dtype '<i4', one dimension of length `expected`, as src/prune.c:32-57
 * loadMapping requires.  PSS_ERR_INVALID_ARG on any mismatch (the reference
 * exits). */
pss_status plh_load_vocab_map(const char* path, uint32_t expected, int32_t* out);

/* Device: build the block-transposed fp16 head from the model's lm_head rows
 * src[src_rows][K] (bf16 or fp16, row-major, device memory) as the reference
 * builds it at load time: row n of the head is source row mapping[n]
 * (mapping: host int32[V], every entry in [0, src_rows); NULL: n, the
 * unpruned vocabulary, src_rows = V).  Values pass through the reference's
 * conversions: the pruning gather re-encodes fp16 rows as bf16
 * (src/prune.c:128-146, float_to_bf16), the loader converts bf16 (or fp16)
 * to fp16 with the truncating float_to_fp16 (src/weights.c:520-566) and
 * block-transposes (src/data.c:305-331).  Synchronous; allocates a temporary
 * copy of the map.  w_bt: K * V halves. */
pss_status plh_pack_head(const void* src, uint32_t src_dtype, uint32_t src_rows, uint32_t K,
                         const int32_t* mapping, uint32_t V, uint16_t* w_bt, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* PUMICE_LMHEAD_H */
