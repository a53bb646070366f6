/*
 * pss_oracle.h - CPU restatements of the reference sampler.  TEST
 * INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker.  Never linked into the product.
 */
#ifndef PSS_ORACLE_H
#define PSS_ORACLE_H

#include <stdint.h>
#include "pumice_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Per-row mutable sampler state, as the GPU sampler keeps it. */
typedef struct {
    uint32_t* history;  /* [1024] ring */
    uint32_t position;
    uint32_t rng;       /* xorshift state / Philox key */
    uint32_t step;      /* Philox counter */
} oracle_row_state;

/* O1: the exact build contract (sort-based).  Returns the token.
 * kept (V bytes), p_out (V floats: unnormalized p, or NaN-free raw t for greedy
 * rows), probs (V floats: p/Z for kept), probs64 (V doubles: fp64
 * exp-normalized over the kept set) may each be NULL. */
uint32_t oracle_o1_row(const float* logits, uint32_t V, const sample_params* sp,
                       oracle_row_state* st, uint32_t row, uint32_t mode, uint32_t rng_mode,
                       uint32_t do_increment, pss_row_info* info, uint8_t* kept, float* p_out,
                       float* probs, double* probs64);

/* Batched O1 over rows with per-row params/state; logits in f32 or f16 bits.
 * threads <= 1 runs on the calling thread. */
void oracle_o1_batch(const void* logits, uint32_t dtype, uint64_t row_stride, uint32_t rows,
                     uint32_t V, const sample_params* params, uint32_t* history, uint32_t* position,
                     uint32_t* rng, uint32_t* step, uint32_t mode, uint32_t rng_mode,
                     uint32_t do_increment, uint32_t* tokens, pss_row_info* infos, int threads);

/* The CPU baseline: O1 (no diagnostics) or O3 over rows, thread i pinned
 * to cpus[i] (cpus may be NULL: no pinning).  O3 runs on a private copy of
 * each row, without the tolerance acceptance test. */
void oracle_o1_batch_pinned(const void* logits, uint32_t dtype, uint64_t row_stride, uint32_t rows,
                            uint32_t V, const sample_params* params, uint32_t* history, uint32_t* position,
                            uint32_t* rng, uint32_t* step, uint32_t mode, uint32_t rng_mode,
                            uint32_t do_increment, uint32_t* tokens, int threads, const int* cpus);
void oracle_o3_batch_pinned(const float* logits, uint64_t row_stride, uint32_t rows, uint32_t V,
                            const sample_params* params, uint32_t* history, uint32_t* position,
                            uint32_t* rng, uint32_t* tokens, int threads, const int* cpus);

/* O2: literal restatement of ArgMax-Reduce.comp mode 1 (TS=1024 partition,
 * 28+28 bisection, fp32, libm expf, a fixed reduction association).
 * Mutates `logits` in place like the shader.  V must be a multiple of 4. */
uint32_t oracle_o2_shader_row(float* logits, uint32_t V, const sample_params* sp,
                              uint32_t* history, uint32_t* pos, uint32_t* rng,
                              uint32_t do_increment, float* thr_out);

/* O3: restatement of the reference's fp64 sort-based oracle sampler_ref
 * (src/validation.c:4974-5092), including its tolerance acceptance.
 * Mutates `logits` in place (logits[j] = (float)p[j]) like the original. */
uint32_t oracle_o3_sampler_ref(float* logits, int V, const sample_params* sp, uint32_t* history,
                               uint32_t* pos, uint32_t* rng, uint32_t acceptTok, double tol,
                               int* tolOut);

/* Greedy: argmax of raw logits, smallest id on ties (NaN never wins). */
uint32_t oracle_greedy_row(const float* logits, uint32_t V);

/* Two-stage greedy as the reference runs it: per-256-column winners
 * (LMHead-GEMV-ArgMax-Q16.comp:75-96) then a 1024-thread tree reduce
 * (ArgMax-Reduce.comp:135-167). */
uint32_t oracle_greedy_two_stage(const float* logits, uint32_t V);

/* src/data.c:8-28 */
float oracle_get_pseudo_random(int i, int j, int seed);
void oracle_get_data(int seed, int M, int N, float* out);

/* src/data.c:30-52 float_to_fp16 (truncating), :54-81 fp16_to_float,
 * :83-93 getDataFP16. */
uint16_t oracle_float_to_fp16(float f);
float oracle_fp16_to_float(uint16_t h);
void oracle_get_data_fp16(int seed, int M, int N, uint16_t* out);
void oracle_float_to_fp16_many(const float* f, uint16_t* h, uint64_t n);
void oracle_fp16_to_float_many(const uint16_t* h, float* f, uint64_t n);

/* LM head (LMHead-GEMV-Q16.comp:28-72): src/data.c:305-331 transpose_block16
 * for FP16; the RMSNorm with the GPU's summation order (returns inv_rms,
 * writes a[K]); the GEMV over the block-transposed head with the GPU's
 * K-slice order (nslices slices, fmaf chains, partials added in slice order);
 * and the same GEMV in binary64 with sum |a w| for error bounds. */
void oracle_transpose_block16_fp16(const uint16_t* w_kv, uint16_t* w_bt, uint32_t K, uint32_t V);
/* src/data.c:187-200 bf16 conversions. */
float oracle_bf16_to_float(uint16_t b);
uint16_t oracle_float_to_bf16(float f);
void oracle_float_to_bf16_many(const float* f, uint16_t* b, uint64_t n);
/* The reference's load-time build of the fp16 head from lm_head rows
 * src[src_rows][K] (src_dtype 0 bf16 / 1 fp16): src/prune.c:128-146 gather
 * (fp16 rows re-encoded as bf16) when map is not NULL, src/weights.c:520-566
 * conversion to fp16 and transpose into [K][V], src/data.c:305-331. */
void oracle_pack_head(const uint16_t* src, uint32_t src_dtype, uint32_t K, const int32_t* map, uint32_t V,
                      uint16_t* w_bt);
float oracle_lmhead_norm(const float* x, const float* gamma, uint32_t K, float* a);
void oracle_lmhead_logits(const float* a, const uint16_t* w_bt, uint32_t K, uint32_t V, uint32_t nslices,
                          float* out);
void oracle_lmhead_logits64(const float* a, const uint16_t* w_bt, uint32_t K, uint32_t V, double* out,
                            double* absdot);

/* exp checks over every binary32 x in [lo, hi], hi <= 0.  Returns the number of
 * monotonicity violations (pss_exp(x') > pss_exp(x) for x' < x); writes the max
 * error, in ulps of the exact result, against the fp64 libm exp, sampled at every
 * acc_stride-th bit pattern. */
uint64_t oracle_exp_scan(float lo, float hi, uint32_t acc_stride, double* max_ulp,
                        float* worst_x);

float oracle_pss_exp(float x);
void oracle_exp_many(const float* x, float* y, uint64_t n);
/* Scoring mode on one fp32 row; returns the NLL, Zq and key(gmax) optional. */
float oracle_o1_score_row(const float* logits, uint32_t V, uint32_t target, uint64_t* zq_out,
                          uint32_t* gmax_key_out);
double oracle_log64(double x);
void oracle_prob_many(const float* t, float tmax, float* y, uint64_t n);
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
uint32_t oracle_xorshift32(uint32_t x);
uint64_t oracle_topp_need(float topP, uint64_t zk);
uint64_t oracle_draw_target(uint32_t u24, uint64_t z);
uint32_t oracle_key(float t);
float oracle_unkey(uint32_t k);
float oracle_canon(float t);
uint64_t oracle_fixq(float p);
float oracle_h2f(uint16_t h);

#ifdef __cplusplus
}
#endif

#endif
