/*
 * pss_oracle.c - CPU restatements of the reference's logits -> token sampler.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load this library, and only as the checker (or
 * as the timed CPU baseline).  The product (pumice_amd/) never calls it.
 *
 * O1  oracle_o1_row         the exact build contract, written as a full sort
 *                           like the reference's own oracle sampler_ref
 *                           (src/validation.c:4974-5092) but with the shader's
 *                           fp32 transform (shader/Utility/ArgMax-Reduce.comp:
 *                           222-269), exact order statistics for top-k/top-p,
 *                           fixed-point masses and an exact draw predicate.
 * O2  oracle_o2_shader_row  ArgMax-Reduce.comp mode 1 restated literally
 *                           (bisection, fp32 sums, libm expf).
 * O3  oracle_o3_sampler_ref src/validation.c:4974-5092 restated (fp64).
 * greedy                    LMHead-GEMV-ArgMax-Q16.comp:75-96 +
 *                           ArgMax-Reduce.comp:135-167.
 * get_pseudo_random         src/data.c:8-28.
 * fp16 data, LM head        src/data.c:30-93, :305-331; LMHead-GEMV-Q16.comp:28-72
 *                           in the GPU's summation order (plh_lmhead.hip).
 *
 * Built with -ffp-contract=off; pss_exp and the integer helpers come from the
 * shared deterministic math header, pinned by tests against libm and
 * published known-answer vectors.
 */
#define _GNU_SOURCE /* pthread_setaffinity_np: the CPU baseline pins one thread per core */
#include "pss_oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>

#include "pss_math.h"

#define O_MAX_PEN 1024u

static int cmp_u64_desc(const void* a, const void* b) {
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return (x < y) ? 1 : (x > y ? -1 : 0);
}

float oracle_pss_exp(float x) { return pss_exp(x); }

/* ------------------------------------------------------------------------ */
/* Greedy                                                                   */
/* ------------------------------------------------------------------------ */

uint32_t oracle_greedy_row(const float* logits, uint32_t V) {
    uint32_t best = 0, bestKey = 0;
    for (uint32_t j = 0; j < V; ++j) {
        uint32_t k = pss_key(pss_canon(logits[j]));
        if (j == 0 || k > bestKey) {
            bestKey = k;
            best = j;
        }
    }
    return best;
}

/* Stage 1: 256-column groups, -inf beyond V, tree reduce with smaller-index
 * tie-break (LMHead-GEMV-ArgMax-Q16.comp:75-96).  Stage 2: 1024 threads each
 * scan groups i = tid, tid+1024, ... then a tree reduce
 * (ArgMax-Reduce.comp:136-160).  Values compared as canonical binary32. */
static int beats(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

uint32_t oracle_greedy_two_stage(const float* logits, uint32_t V) {
    uint32_t groups = (V + 255u) / 256u;
    float* gv = (float*)malloc(sizeof(float) * groups);
    uint32_t* gi = (uint32_t*)malloc(sizeof(uint32_t) * groups);
    float rv[1024];
    uint32_t ri[1024];
    for (uint32_t g = 0; g < groups; ++g) {
        float v[256];
        uint32_t id[256];
        for (uint32_t c = 0; c < 256; ++c) {
            uint32_t col = g * 256u + c;
            v[c] = col < V ? pss_canon(logits[col]) : pss_u2f(0xFF800000u);
            id[c] = col;
        }
        for (uint32_t stride = 128; stride > 0; stride >>= 1)
            for (uint32_t c = 0; c < stride; ++c)
                if (beats(v[c + stride], id[c + stride], v[c], id[c])) {
                    v[c] = v[c + stride];
                    id[c] = id[c + stride];
                }
        gv[g] = v[0];
        gi[g] = id[0];
    }
    for (uint32_t t = 0; t < 1024; ++t) {
        float bv = pss_u2f(0xFF800000u);
        uint32_t bi = 0;
        for (uint32_t g = t; g < groups; g += 1024)
            if (beats(gv[g], gi[g], bv, bi)) {
                bv = gv[g];
                bi = gi[g];
            }
        rv[t] = bv;
        ri[t] = bi;
    }
    for (uint32_t stride = 512; stride > 0; stride >>= 1)
        for (uint32_t t = 0; t < stride; ++t)
            if (beats(rv[t + stride], ri[t + stride], rv[t], ri[t])) {
                rv[t] = rv[t + stride];
                ri[t] = ri[t + stride];
            }
    free(gv);
    free(gi);
    return ri[0];
}

/* ------------------------------------------------------------------------ */
/* O1                                                                       */
/* ------------------------------------------------------------------------ */

uint32_t oracle_o1_row(const float* logits, uint32_t V, const sample_params* sp,
                       oracle_row_state* st, uint32_t row, uint32_t mode, uint32_t rng_mode,
                       uint32_t do_increment, pss_row_info* info, uint8_t* kept_out, float* p_out,
                       float* probs, double* probs64) {
    pss_row_info inf;
    memset(&inf, 0, sizeof inf);
    int greedy = (mode == PSS_MODE_GREEDY) || !(sp->temperature > 0.0f);
    if (greedy) {
        uint32_t tok = oracle_greedy_row(logits, V);
        uint32_t tmaxKey = pss_key(pss_canon(logits[tok]));
        if (do_increment) st->position += 1u;
        inf.token = tok;
        inf.kept_count = 1;
        inf.tau_key = tmaxKey;
        inf.tmax_key = tmaxKey;
        inf.flags = PSS_INFO_GREEDY;
        if (info) *info = inf;
        if (kept_out) {
            memset(kept_out, 0, V);
            kept_out[tok] = 1;
        }
        if (p_out)
            for (uint32_t j = 0; j < V; ++j) p_out[j] = logits[j];
        if (probs) {
            for (uint32_t j = 0; j < V; ++j) probs[j] = 0.0f;
            probs[tok] = 1.0f;
        }
        if (probs64) {
            for (uint32_t j = 0; j < V; ++j) probs64[j] = 0.0;
            probs64[tok] = 1.0;
        }
        return tok;
    }

    /* S1/S2: fp32 transform exactly as ArgMax-Reduce.comp:222-265. */
    uint32_t W = sp->penaltyLength < O_MAX_PEN ? sp->penaltyLength : O_MAX_PEN;
    float invT = 1.0f / sp->temperature;
    float pres = sp->presencePenalty * invT;
    float rep = sp->repPenalty;
    int doPen = (W > 0u) && (rep != 1.0f || pres != 0.0f);
    uint8_t* member = (uint8_t*)calloc(V, 1);
    if (doPen)
        for (uint32_t h = 0; h < W; ++h) {
            uint32_t id = st->history[h];
            if (id < V) member[id] = 1;
        }
    float* t = (float*)malloc(sizeof(float) * V);
    uint32_t* key = (uint32_t*)malloc(sizeof(uint32_t) * V);
    float* p = (float*)malloc(sizeof(float) * V);
    uint64_t* q = (uint64_t*)malloc(sizeof(uint64_t) * V);
    uint64_t* order = (uint64_t*)malloc(sizeof(uint64_t) * V);
    uint8_t* kept = (uint8_t*)malloc(V);

    uint32_t tmaxKey = 0;
    for (uint32_t j = 0; j < V; ++j) {
        float v = logits[j] * invT;
        if (doPen && member[j]) {
            if (rep != 1.0f) v = (v > 0.0f) ? (v / rep) : (v * rep);
            v = v - pres;
        }
        v = pss_canon(v);
        t[j] = v;
        key[j] = pss_key(v);
        if (key[j] > tmaxKey) tmaxKey = key[j];
    }
    float tmax = pss_unkey(tmaxKey);

    /* S4: probabilities and fixed-point masses. */
    for (uint32_t j = 0; j < V; ++j) {
        p[j] = pss_prob(t[j], tmax);
        q[j] = pss_fixq(p[j]);
        order[j] = ((uint64_t)key[j] << 32) | (uint64_t)(0xFFFFFFFFu - j);
    }
    qsort(order, V, sizeof(uint64_t), cmp_u64_desc);

    /* S5: top-k, K-th largest value, ties kept. */
    uint32_t K = sp->topK < V ? sp->topK : V;
    uint32_t tauK = K > 0 ? (uint32_t)(order[K - 1] >> 32) : 0u;
    uint64_t zk = 0;
    for (uint32_t j = 0; j < V; ++j)
        if (key[j] >= tauK) zk += q[j];
    uint32_t tau = tauK;

    /* S6: top-p, largest value v with mass(t >= v) >= topP * Zk. */
    if (sp->topP > 0.0f && sp->topP < 1.0f) {
        uint64_t need = pss_topp_need(sp->topP, zk);
        uint64_t acc = 0;
        for (uint32_t i = 0; i < V; ++i) {
            uint32_t j = 0xFFFFFFFFu - (uint32_t)order[i];
            acc += q[j];
            if (acc >= need) {
                uint32_t tp = (uint32_t)(order[i] >> 32);
                if (tp > tau) tau = tp;
                break;
            }
        }
    }

    /* S7: min-p in probability space (p_max = 1). */
    int useMinP = sp->minP > 0.0f;
    uint64_t z = 0;
    uint32_t keptCount = 0;
    for (uint32_t j = 0; j < V; ++j) {
        kept[j] = key[j] >= tau && (!useMinP || p[j] >= sp->minP);
        if (kept[j]) {
            z += q[j];
            keptCount++;
        }
    }

    /* S8: uniform, target, ascending-id inverse CDF with integer masses. */
    uint32_t u24;
    uint32_t s = st->rng;
    if (rng_mode == PSS_RNG_PHILOX) {
        pss_u32x4 c = {{st->step, row, 0u, 0u}};
        u24 = pss_philox4x32_10(c, st->rng, 0u).v[0] >> 8;
    } else {
        if (s == 0u) s = PSS_XORSHIFT_ZERO_SEED;
        u24 = s >> 8;
    }
    uint64_t target = pss_draw_target(u24, z);
    uint64_t acc = 0;
    uint32_t tok = 0;
    int found = 0;
    for (uint32_t j = 0; j < V; ++j) {
        if (!kept[j]) continue;
        acc += q[j];
        if (acc > target) {
            tok = j;
            found = 1;
            break;
        }
    }
    if (!found) {
        inf.flags |= PSS_INFO_FALLBACK;
        for (uint32_t j = V; j-- > 0;)
            if (kept[j]) {
                tok = j;
                break;
            }
    }

    /* S9: epilogue (ArgMax-Reduce.comp:376-385). */
    if (W > 0u) st->history[st->position % W] = tok;
    if (rng_mode == PSS_RNG_PHILOX)
        st->step += 1u;
    else
        st->rng = pss_xorshift32(s);
    if (do_increment) st->position += 1u;

    inf.token = tok;
    inf.kept_count = keptCount;
    inf.tau_key = tau;
    inf.tmax_key = tmaxKey;
    inf.z_kept = z;
    inf.z_topk = zk;
    inf.target = target;
    inf.u24 = u24;
    if (info) *info = inf;
    if (kept_out) memcpy(kept_out, kept, V);
    if (p_out) memcpy(p_out, p, sizeof(float) * V);
    if (probs) {
        float zf = (float)z * 0x1.0p-45f;
        for (uint32_t j = 0; j < V; ++j) probs[j] = kept[j] ? p[j] / zf : 0.0f;
    }
    if (probs64) {
        double tm = (double)tmax, sum = 0.0;
        for (uint32_t j = 0; j < V; ++j) {
            double e = 0.0;
            if (kept[j]) e = (t[j] == tmax) ? 1.0 : exp((double)t[j] - tm);
            probs64[j] = e;
            sum += e;
        }
        for (uint32_t j = 0; j < V; ++j) probs64[j] /= sum;
    }
    free(member);
    free(t);
    free(key);
    free(p);
    free(q);
    free(order);
    free(kept);
    return tok;
}

typedef struct {
    const void* logits;
    uint32_t dtype;
    uint64_t stride;
    uint32_t V;
    const sample_params* params;
    uint32_t* history;
    uint32_t* position;
    uint32_t* rng;
    uint32_t* step;
    uint32_t mode, rng_mode, do_increment;
    uint32_t* tokens;
    pss_row_info* infos;
    uint32_t r0, r1;
    int cpu;  /* >= 0: pin the worker to this CPU */
    int o3;   /* run O3 (sampler_ref) instead of O1 */
} batch_job;

static void pin_self(int cpu) {
    if (cpu < 0) return;
    cpu_set_t set;
    CPU_ZERO(&set);
    CPU_SET(cpu, &set);
    (void)pthread_setaffinity_np(pthread_self(), sizeof set, &set);
}

static void* batch_worker(void* arg) {
    batch_job* b = (batch_job*)arg;
    pin_self(b->cpu);
    float* row = NULL;
    if (b->o3) {
        /* O3 mutates its row: a private copy per row */
        row = (float*)malloc(sizeof(float) * b->V);
        for (uint32_t r = b->r0; r < b->r1; ++r) {
            memcpy(row, (const float*)b->logits + (uint64_t)r * b->stride, sizeof(float) * b->V);
            int tol = 0;
            uint32_t tok = oracle_o3_sampler_ref(row, (int)b->V, &b->params[r], b->history + (uint64_t)r * O_MAX_PEN,
                                                 &b->position[r], &b->rng[r], 0xFFFFFFFFu, 5e-4, &tol);
            if (b->tokens) b->tokens[r] = tok;
        }
        free(row);
        return NULL;
    }
    if (b->dtype == PSS_DTYPE_F16) row = (float*)malloc(sizeof(float) * b->V);
    for (uint32_t r = b->r0; r < b->r1; ++r) {
        const float* l;
        if (b->dtype == PSS_DTYPE_F16) {
            const uint16_t* h = (const uint16_t*)b->logits + (uint64_t)r * b->stride;
            for (uint32_t j = 0; j < b->V; ++j) row[j] = pss_h2f(h[j]);
            l = row;
        } else {
            l = (const float*)b->logits + (uint64_t)r * b->stride;
        }
        oracle_row_state st;
        st.history = b->history + (uint64_t)r * O_MAX_PEN;
        st.position = b->position[r];
        st.rng = b->rng[r];
        st.step = b->step[r];
        uint32_t tok = oracle_o1_row(l, b->V, &b->params[r], &st, r, b->mode, b->rng_mode,
                                     b->do_increment, b->infos ? &b->infos[r] : NULL, NULL, NULL,
                                     NULL, NULL);
        b->position[r] = st.position;
        b->rng[r] = st.rng;
        b->step[r] = st.step;
        if (b->tokens) b->tokens[r] = tok;
    }
    free(row);
    return NULL;
}

static void run_batch(const void* logits, uint32_t dtype, uint64_t row_stride, uint32_t rows, uint32_t V,
                      const sample_params* params, uint32_t* history, uint32_t* position, uint32_t* rng,
                      uint32_t* step, uint32_t mode, uint32_t rng_mode, uint32_t do_increment,
                      uint32_t* tokens, pss_row_info* infos, int threads, const int* cpus, int o3);

void oracle_o1_batch(const void* logits, uint32_t dtype, uint64_t row_stride, uint32_t rows,
                     uint32_t V, const sample_params* params, uint32_t* history, uint32_t* position,
                     uint32_t* rng, uint32_t* step, uint32_t mode, uint32_t rng_mode,
                     uint32_t do_increment, uint32_t* tokens, pss_row_info* infos, int threads) {
    run_batch(logits, dtype, row_stride, rows, V, params, history, position, rng, step, mode, rng_mode,
              do_increment, tokens, infos, threads, NULL, 0);
}

void oracle_o1_batch_pinned(const void* logits, uint32_t dtype, uint64_t row_stride, uint32_t rows,
                            uint32_t V, const sample_params* params, uint32_t* history, uint32_t* position,
                            uint32_t* rng, uint32_t* step, uint32_t mode, uint32_t rng_mode,
                            uint32_t do_increment, uint32_t* tokens, int threads, const int* cpus) {
    run_batch(logits, dtype, row_stride, rows, V, params, history, position, rng, step, mode, rng_mode,
              do_increment, tokens, NULL, threads, cpus, 0);
}

void oracle_o3_batch_pinned(const float* logits, uint64_t row_stride, uint32_t rows, uint32_t V,
                            const sample_params* params, uint32_t* history, uint32_t* position,
                            uint32_t* rng, uint32_t* tokens, int threads, const int* cpus) {
    run_batch(logits, PSS_DTYPE_F32, row_stride, rows, V, params, history, position, rng, NULL, 1, 0, 1,
              tokens, NULL, threads, cpus, 1);
}

static void run_batch(const void* logits, uint32_t dtype, uint64_t row_stride, uint32_t rows, uint32_t V,
                      const sample_params* params, uint32_t* history, uint32_t* position, uint32_t* rng,
                      uint32_t* step, uint32_t mode, uint32_t rng_mode, uint32_t do_increment,
                      uint32_t* tokens, pss_row_info* infos, int threads, const int* cpus, int o3) {
    if (threads < 1) threads = 1;
    if ((uint32_t)threads > rows) threads = (int)rows;
    batch_job jobs[256];
    pthread_t tids[256];
    if (threads > 256) threads = 256;
    for (int i = 0; i < threads; ++i) {
        batch_job* b = &jobs[i];
        b->logits = logits;
        b->dtype = dtype;
        b->stride = row_stride;
        b->V = V;
        b->params = params;
        b->history = history;
        b->position = position;
        b->rng = rng;
        b->step = step;
        b->mode = mode;
        b->rng_mode = rng_mode;
        b->do_increment = do_increment;
        b->tokens = tokens;
        b->infos = infos;
        b->r0 = (uint32_t)((uint64_t)rows * i / threads);
        b->r1 = (uint32_t)((uint64_t)rows * (i + 1) / threads);
        b->cpu = cpus ? cpus[i] : -1;
        b->o3 = o3;
    }
    if (threads == 1 && !cpus) { /* pinning happens on a worker thread, never the caller's */
        batch_worker(&jobs[0]);
        return;
    }
    for (int i = 0; i < threads; ++i) pthread_create(&tids[i], NULL, batch_worker, &jobs[i]);
    for (int i = 0; i < threads; ++i) pthread_join(tids[i], NULL);
}

/* ------------------------------------------------------------------------ */
/* O2: ArgMax-Reduce.comp mode 1, literally                                 */
/* ------------------------------------------------------------------------ */

#define O2_TS 1024u
#define O2_SG 64u /* wave64 subgroups */
#define O2_BISECT 28

/* subgroupAdd over 64 lanes, associated as an adjacent-pairs tree. */
static float o2_subgroup_add(const float* lane) {
    float v[O2_SG];
    memcpy(v, lane, sizeof v);
    for (uint32_t stride = 1; stride < O2_SG; stride <<= 1)
        for (uint32_t i = 0; i + stride < O2_SG; i += 2 * stride) v[i] = v[i] + v[i + stride];
    return v[0];
}

/* sumAll (ArgMax-Reduce.comp:91-103): subgroupAdd, then thread 0 adds the 16
 * subgroup sums in order starting from 0. */
static float o2_sum_all(const float* per_thread) {
    float t = 0.0f;
    for (uint32_t sg = 0; sg < O2_TS / O2_SG; ++sg) t += o2_subgroup_add(per_thread + sg * O2_SG);
    return t;
}

static float o2_mass_above(const float* lg, uint32_t base4, uint32_t cnt4, float mySum,
                           float myMax, float myMin, float thr) {
    if (myMax < thr) return 0.0f;
    if (myMin >= thr) return mySum;
    float s = 0.0f;
    for (uint32_t k = 0; k < cnt4; ++k) {
        const float* p = lg + 4u * (base4 + k);
        s += (p[0] >= thr ? p[0] : 0.0f) + (p[1] >= thr ? p[1] : 0.0f);
        s += (p[2] >= thr ? p[2] : 0.0f) + (p[3] >= thr ? p[3] : 0.0f);
    }
    return s;
}

uint32_t oracle_o2_shader_row(float* lg, uint32_t V, const sample_params* sp, uint32_t* history,
                              uint32_t* pos, uint32_t* rng, uint32_t do_increment,
                              float* thr_out) {
    const uint32_t TS = O2_TS;
    uint32_t V4 = (V + 3u) / 4u;
    uint32_t E4 = (V4 + TS - 1u) / TS;
    static uint32_t base4[O2_TS], cnt4[O2_TS];
    static float mySum[O2_TS], myMax[O2_TS], myMin[O2_TS], tmp[O2_TS];
    static float blockSum[O2_TS], cumBase[O2_TS];
    for (uint32_t tid = 0; tid < TS; ++tid) {
        base4[tid] = tid * E4;
        cnt4[tid] = base4[tid] < V4 ? (E4 < V4 - base4[tid] ? E4 : V4 - base4[tid]) : 0u;
    }
    float penalty = sp->repPenalty;
    float pres = sp->presencePenalty * (1.0f / sp->temperature);
    uint32_t penLen = sp->penaltyLength > 1024u ? 1024u : sp->penaltyLength;
    uint32_t topK = sp->topK > V ? V : sp->topK;
    float topP = sp->topP;
    int doPen = (penLen > 0u) && (penalty != 1.0f || pres != 0.0f);
    float invT = 1.0f / sp->temperature;
    uint8_t* bits = (uint8_t*)calloc(262144u, 1);
    if (doPen)
        for (uint32_t h = 0; h < penLen; ++h)
            if (history[h] < 262144u) bits[history[h]] = 1;

    float gMax = -3.4e38f, gMin = 3.4e38f;
    for (uint32_t tid = 0; tid < TS; ++tid) {
        float lmax = -3.4e38f, lmin = 3.4e38f;
        for (uint32_t k = 0; k < cnt4[tid]; ++k) {
            uint32_t j = base4[tid] * 4u + k * 4u;
            float* t = lg + 4u * (base4[tid] + k);
            for (int c = 0; c < 4; ++c) {
                t[c] = t[c] * invT;
                if (doPen && bits[j + c]) {
                    if (penalty != 1.0f) t[c] = (t[c] > 0.0f) ? (t[c] / penalty) : (t[c] * penalty);
                    t[c] -= pres;
                }
            }
            if (j + 1u >= V) t[1] = -3.4e38f;
            if (j + 2u >= V) t[2] = -3.4e38f;
            if (j + 3u >= V) t[3] = -3.4e38f;
            for (int c = 0; c < 4; ++c) {
                lmax = fmaxf(lmax, t[c]);
                lmin = fminf(lmin, t[c]);
            }
        }
        gMax = fmaxf(gMax, lmax);
        gMin = fminf(gMin, lmin);
    }
    free(bits);

    for (uint32_t tid = 0; tid < TS; ++tid) {
        mySum[tid] = 0.0f;
        myMax[tid] = 0.0f;
        myMin[tid] = 1.0f;
        for (uint32_t k = 0; k < cnt4[tid]; ++k) {
            float* p = lg + 4u * (base4[tid] + k);
            for (int c = 0; c < 4; ++c) p[c] = expf(p[c] - gMax);
            mySum[tid] += (p[0] + p[1]) + (p[2] + p[3]);
            myMax[tid] = fmaxf(myMax[tid], fmaxf(fmaxf(p[0], p[1]), fmaxf(p[2], p[3])));
            myMin[tid] = fminf(myMin[tid], fminf(fminf(p[0], p[1]), fminf(p[2], p[3])));
        }
    }
    float Zall = o2_sum_all(mySum);
    float gThrP = 0.0f;

    if (topK > 0u) {
        float gLo = gMin, gHi = gMax;
        for (int it = 0; it < O2_BISECT; ++it) {
            gThrP = expf(0.5f * (gLo + gHi) - gMax);
            uint32_t total = 0;
            for (uint32_t tid = 0; tid < TS; ++tid) {
                if (!(myMax[tid] >= gThrP)) continue;
                for (uint32_t k = 0; k < cnt4[tid]; ++k) {
                    const float* p = lg + 4u * (base4[tid] + k);
                    for (int c = 0; c < 4; ++c) total += p[c] >= gThrP ? 1u : 0u;
                }
            }
            float mid = 0.5f * (gLo + gHi);
            if (total >= topK)
                gLo = mid;
            else
                gHi = mid;
        }
        gThrP = expf(gLo - gMax);
    }

    if (topP < 1.0f && topP > 0.0f) {
        float Zk = Zall, gLo = gMin, gHi = gMax;
        if (topK > 0u) {
            for (uint32_t tid = 0; tid < TS; ++tid)
                tmp[tid] = o2_mass_above(lg, base4[tid], cnt4[tid], mySum[tid], myMax[tid],
                                         myMin[tid], gThrP);
            Zk = o2_sum_all(tmp);
        }
        float target = topP * Zk;
        for (int it = 0; it < O2_BISECT; ++it) {
            gThrP = expf(0.5f * (gLo + gHi) - gMax);
            for (uint32_t tid = 0; tid < TS; ++tid)
                tmp[tid] = o2_mass_above(lg, base4[tid], cnt4[tid], mySum[tid], myMax[tid],
                                         myMin[tid], gThrP);
            float s = o2_sum_all(tmp);
            float mid = 0.5f * (gLo + gHi);
            if (s >= target)
                gLo = mid;
            else
                gHi = mid;
        }
        gThrP = expf(gLo - gMax);
    }

    if (sp->minP > 0.0f && gThrP < sp->minP) gThrP = sp->minP;

    for (uint32_t tid = 0; tid < TS; ++tid)
        blockSum[tid] = o2_mass_above(lg, base4[tid], cnt4[tid], mySum[tid], myMax[tid],
                                      myMin[tid], gThrP);
    float acc = 0.0f;
    for (uint32_t i = 0; i < TS; ++i) {
        cumBase[i] = acc;
        acc += blockSum[i];
    }
    uint32_t s = *rng;
    if (s == 0u) s = PSS_XORSHIFT_ZERO_SEED;
    float u = (float)(s >> 8) * (1.0f / 16777216.0f);
    float gTarget = u * acc;
    uint32_t win = TS - 1u;
    for (uint32_t i = 0; i < TS; ++i)
        if (gTarget < cumBase[i] + blockSum[i]) {
            win = i;
            break;
        }
    float a = cumBase[win];
    uint32_t chosen = base4[win] * 4u;
    int found = 0;
    for (uint32_t k = 0; k < cnt4[win]; ++k) {
        const float* p = lg + 4u * (base4[win] + k);
        uint32_t j = base4[win] * 4u + k * 4u;
        for (uint32_t c = 0; c < 4; ++c)
            if (!found && j + c < V && p[c] >= gThrP) {
                a += p[c];
                chosen = j + c;
                if (gTarget < a) found = 1;
            }
    }
    if (penLen > 0u) history[*pos % penLen] = chosen;
    *rng = pss_xorshift32(s);
    if (do_increment) *pos += 1u;
    if (thr_out) *thr_out = gThrP;
    return chosen;
}

/* ------------------------------------------------------------------------ */
/* O3: sampler_ref (src/validation.c:4974-5092), fp64                       */
/* ------------------------------------------------------------------------ */

typedef struct {
    double a, p;
} o3_pair;

static int o3_desc(const void* x, const void* y) {
    double a = ((const o3_pair*)x)->a, b = ((const o3_pair*)y)->a;
    return a > b ? -1 : (a < b ? 1 : 0);
}

uint32_t oracle_o3_sampler_ref(float* logits, int V, const sample_params* sp, uint32_t* history,
                               uint32_t* pos, uint32_t* rng, uint32_t acceptTok, double tol,
                               int* tolOut) {
    int W = (int)(sp->penaltyLength > 1024u ? 1024u : sp->penaltyLength);
    double* a = (double*)malloc(sizeof(double) * V);
    double* p = (double*)malloc(sizeof(double) * V);
    uint8_t* seen = (uint8_t*)calloc((size_t)V, 1);
    o3_pair* arr = (o3_pair*)malloc(sizeof(o3_pair) * V);
    for (int j = 0; j < V; ++j) a[j] = (double)logits[j] / (double)sp->temperature;
    if (W > 0 && (sp->repPenalty != 1.0f || sp->presencePenalty != 0.0f))
        for (int h = 0; h < W; ++h) {
            uint32_t id = history[h];
            if (id >= (uint32_t)V || seen[id]) continue;
            seen[id] = 1;
            if (sp->repPenalty != 1.0f)
                a[id] = a[id] > 0.0 ? a[id] / (double)sp->repPenalty : a[id] * (double)sp->repPenalty;
            a[id] -= (double)sp->presencePenalty / (double)sp->temperature;
        }
    double mx = -1e300;
    for (int j = 0; j < V; ++j)
        if (a[j] > mx) mx = a[j];
    for (int j = 0; j < V; ++j) {
        p[j] = exp(a[j] - mx);
        logits[j] = (float)p[j];
        arr[j].a = a[j];
        arr[j].p = p[j];
    }
    qsort(arr, (size_t)V, sizeof(o3_pair), o3_desc);
    int topK = (int)sp->topK > V ? V : (int)sp->topK;
    double thr = -1e300;
    int kept = V;
    if (topK > 0) {
        thr = arr[topK - 1].a;
        kept = 0;
        while (kept < V && arr[kept].a >= thr) kept++;
    }
    if (sp->topP < 1.0f && sp->topP > 0.0f) {
        double zk = 0.0;
        for (int i = 0; i < kept; ++i) zk += arr[i].p;
        double tgt = (double)sp->topP * zk, acc = 0.0;
        int i = 0;
        for (; i < kept; ++i) {
            acc += arr[i].p;
            if (acc >= tgt) break;
        }
        if (i >= kept) i = kept - 1;
        thr = arr[i].a;
        kept = 0;
        while (kept < V && arr[kept].a >= thr) kept++;
    }
    if (sp->minP > 0.0f) {
        double tm = mx + log((double)sp->minP);
        if (tm > thr) {
            thr = tm;
            kept = 0;
            while (kept < V && arr[kept].a >= thr) kept++;
        }
    }
    double zkept = 0.0;
    for (int i = 0; i < kept; ++i) zkept += arr[i].p;
    uint32_t s = *rng;
    if (s == 0u) s = PSS_XORSHIFT_ZERO_SEED;
    double u = (double)(s >> 8) / 16777216.0;
    double target = u * zkept, acc = 0.0, qLo = -1.0, qHi = -1.0;
    uint32_t chosen = 0;
    int found = 0;
    for (int j = 0; j < V; ++j) {
        if (!(a[j] >= thr)) continue;
        if ((uint32_t)j == acceptTok) {
            qLo = acc;
            qHi = acc + p[j];
        }
        acc += p[j];
        if (!found) {
            chosen = (uint32_t)j;
            if (target < acc) found = 1;
        }
        if (found && (uint32_t)j >= acceptTok) break;
    }
    if (!found)
        for (int j = V - 1; j >= 0; --j)
            if (a[j] >= thr) {
                chosen = (uint32_t)j;
                break;
            }
    if (tolOut) *tolOut = 0;
    if (acceptTok != 0xFFFFFFFFu && acceptTok != chosen && qLo >= 0.0) {
        double dist = target > qHi ? target - qHi : (target < qLo ? qLo - target : 0.0);
        if (dist <= tol * zkept) {
            chosen = acceptTok;
            if (tolOut) *tolOut = 1;
        }
    }
    if (W > 0) history[*pos % (uint32_t)W] = chosen;
    *rng = pss_xorshift32(s);
    *pos += 1u;
    free(a);
    free(p);
    free(seen);
    free(arr);
    return chosen;
}

/* ------------------------------------------------------------------------ */
/* src/data.c:8-28                                                          */
/* ------------------------------------------------------------------------ */

/*
 * Scoring mode (ArgMax-Reduce.comp:169-214), build contract: raw logits made
 * canonical (NaN -> -inf, -0 -> +0), gmax their maximum, Zq the exact
 * fixed-point sum of exp(t - gmax), lt the target's value (0 when target >=
 * V, as the shader's sumAll over no match), nll = log(Z) + gmax - lt
 * (pss_score_nll).  Plain loops in id order.
 */
float oracle_o1_score_row(const float* logits, uint32_t V, uint32_t target, uint64_t* zq_out,
                          uint32_t* gmax_key_out) {
    float gmax = pss_u2f(0xFF800000u);
    for (uint32_t j = 0; j < V; ++j) {
        const float t = pss_canon(logits[j]);
        if (pss_key(t) > pss_key(gmax)) gmax = t;
    }
    uint64_t zq = 0;
    for (uint32_t j = 0; j < V; ++j) zq += pss_fixq(pss_prob(pss_canon(logits[j]), gmax));
    const float lt = target < V ? pss_canon(logits[target]) : 0.0f;
    if (zq_out) *zq_out = zq;
    if (gmax_key_out) *gmax_key_out = pss_key(gmax);
    return pss_score_nll(zq, gmax, lt);
}

double oracle_log64(double x) { return pss_log64(x); }

float oracle_get_pseudo_random(int i, int j, int seed) {
    /* The original forms i*73129 + j*95121 + seed*15473 in int and converts to
     * unsigned; done here in uint32_t so the wrap is defined. */
    uint32_t h = (uint32_t)i * 73129u + (uint32_t)j * 95121u + (uint32_t)seed * 15473u;
    h = (h ^ 61u) ^ (h >> 16);
    h += h << 3;
    h ^= h >> 4;
    h *= 0x27d4eb2du;
    h ^= h >> 15;
    return ((float)(h % 2000001u) / 1000000.0f) - 1.0f;
}

void oracle_get_data(int seed, int M, int N, float* out) {
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) out[(size_t)i * N + j] = oracle_get_pseudo_random(i, j, seed);
}

/* ------------------------------------------------------------------------ */
/* fp16 data and the LM head                                                */
/* ------------------------------------------------------------------------ */

/* src/data.c:30-52: sign, then the binary32 exponent e: e < -24 -> signed
 * zero, e <= -15 -> subnormal with the mantissa (hidden bit included) shifted
 * right by -1 - e, e >= 16 -> signed infinity, else the exponent rebiased
 * and the mantissa truncated to 10 bits.  No rounding anywhere. */
uint16_t oracle_float_to_fp16(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    const int e = (int)((b >> 23) & 0xFFu) - 127;
    const uint32_t m = b & 0x7FFFFFu;
    if (e < -24) return sign;
    if (e <= -15) return (uint16_t)(sign | ((m | 0x800000u) >> (-1 - e)));
    if (e >= 16) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)(e + 15) << 10) | (m >> 13));
}

/* IEEE binary16 -> binary32 (exact): value = (-1)^s 2^(E-15) (1 + m/1024),
 * subnormals m 2^-24, E = 31 infinities / NaNs (payload kept). */
float oracle_fp16_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16, E = (h >> 10) & 31u, m = h & 1023u;
    uint32_t b;
    if (E == 31u) {
        b = s | 0x7F800000u | (m << 13);
    } else if (E == 0u) {
        const float v = ldexpf((float)m, -24);
        memcpy(&b, &v, 4);
        b |= s;
    } else {
        b = s | ((E + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &b, 4);
    return f;
}

void oracle_float_to_fp16_many(const float* f, uint16_t* h, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) h[i] = oracle_float_to_fp16(f[i]);
}

void oracle_fp16_to_float_many(const uint16_t* h, float* f, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) f[i] = oracle_fp16_to_float(h[i]);
}

void oracle_get_data_fp16(int seed, int M, int N, uint16_t* out) {
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j)
            out[(size_t)i * N + j] = oracle_float_to_fp16(oracle_get_pseudo_random(i, j, seed));
}

/* src/data.c:305-331 with 16-bit data: output block (kb, n) = the 8 halves
 * w[8 kb + j][n], j = 0..7, at halves offset (kb V + n) 8 + j. */
void oracle_transpose_block16_fp16(const uint16_t* w_kv, uint16_t* w_bt, uint32_t K, uint32_t V) {
    for (uint32_t kb = 0; kb < K / 8u; ++kb)
        for (uint32_t n = 0; n < V; ++n)
            for (uint32_t j = 0; j < 8u; ++j)
                w_bt[((size_t)kb * V + n) * 8u + j] = w_kv[(size_t)(8u * kb + j) * V + n];
}

/* src/data.c:187-192: the bf16 bits are the high half of the binary32. */
float oracle_bf16_to_float(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* src/data.c:194-200: round to nearest, ties to even, by adding 0x7FFF plus
 * the lowest kept bit before dropping the low half (no NaN special case). */
uint16_t oracle_float_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void oracle_float_to_bf16_many(const float* f, uint16_t* b, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) b[i] = oracle_float_to_bf16(f[i]);
}

/* Pruned (map given): gatherRows copies row map[v] (bf16 as is, fp16 through
 * float_to_bf16(fp16_to_float)) into a bf16 tensor, which loadEmbedLike turns
 * into float_to_fp16(bf16_to_float(.)).  Unpruned: loadEmbedLike reads the
 * shard tensor directly (bf16 as above, fp16 through float_to_fp16 of its
 * float value).  Both then transpose_block16 the [K][V] fp16 matrix. */
void oracle_pack_head(const uint16_t* src, uint32_t src_dtype, uint32_t K, const int32_t* map, uint32_t V,
                      uint16_t* w_bt) {
    uint16_t* eng = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)K * V);
    for (uint32_t v = 0; v < V; ++v) {
        const uint16_t* row = src + (size_t)(map ? (uint32_t)map[v] : v) * K;
        for (uint32_t k = 0; k < K; ++k) {
            uint16_t raw = row[k];
            float x;
            if (src_dtype == 0u) {
                x = oracle_bf16_to_float(raw);
            } else if (map) {
                x = oracle_bf16_to_float(oracle_float_to_bf16(oracle_fp16_to_float(raw)));
            } else {
                x = oracle_fp16_to_float(raw);
            }
            eng[(size_t)k * V + v] = oracle_float_to_fp16(x);
        }
    }
    oracle_transpose_block16_fp16(eng, w_bt, K, V);
    free(eng);
}

/* RMSNorm of LMHead-GEMV-Q16.comp:34-58 (src/validation.c:157-163 on the
 * CPU): rms = sqrt(sum x^2 / K + 1e-6), a = x gamma / rms.  The sum of squares
 * in the GPU's order: 256 strided binary64 partials (thread t: k = t, t + 256,
 * ...), a xor butterfly over each group of 64, the four group sums in order;
 * then binary32 for the rest, as the shader. */
float oracle_lmhead_norm(const float* x, const float* gamma, uint32_t K, float* a) {
    double p[256];
    for (uint32_t t = 0; t < 256u; ++t) {
        double s = 0.0;
        for (uint32_t k = t; k < K; k += 256u) {
            const double v = (double)x[k];
            s = s + v * v;
        }
        p[t] = s;
    }
    for (uint32_t w = 0; w < 4u; ++w) {
        double* q = p + 64u * w;
        for (uint32_t off = 32u; off >= 1u; off >>= 1) {
            double nq[64];
            for (uint32_t l = 0; l < 64u; ++l) nq[l] = q[l] + q[l ^ off];
            memcpy(q, nq, sizeof(nq));
        }
    }
    double tot = p[0];
    for (uint32_t w = 1; w < 4u; ++w) tot = tot + p[64u * w];
    const float inv = 1.0f / sqrtf((float)tot / (float)K + 1e-6f);
    for (uint32_t k = 0; k < K; ++k) a[k] = (x[k] * gamma[k]) * inv;
    return inv;
}

/* The GEMV of LMHead-GEMV-Q16.comp:60-70 (acc += a[k] w[k][n] over k) in the
 * GPU's order: slice s covers the 8-row blocks [s KB / S, (s + 1) KB / S),
 * KB = K / 8, each an fmaf chain from 0 in ascending k; the slice partials
 * are added in slice order. */
void oracle_lmhead_logits(const float* a, const uint16_t* w_bt, uint32_t K, uint32_t V, uint32_t nslices,
                          float* out) {
    const uint32_t KB = K / 8u;
    for (uint32_t n = 0; n < V; ++n) {
        float tot = 0.0f;
        for (uint32_t s = 0; s < nslices; ++s) {
            float acc = 0.0f;
            for (uint32_t kb = s * KB / nslices; kb < (s + 1u) * KB / nslices; ++kb) {
                const uint16_t* blk = w_bt + ((size_t)kb * V + n) * 8u;
                for (uint32_t j = 0; j < 8u; ++j) acc = fmaf(a[8u * kb + j], oracle_fp16_to_float(blk[j]), acc);
            }
            tot = s == 0u ? acc : tot + acc;
        }
        out[n] = tot;
    }
}

void oracle_lmhead_logits64(const float* a, const uint16_t* w_bt, uint32_t K, uint32_t V, double* out,
                            double* absdot) {
    for (uint32_t n = 0; n < V; ++n) {
        double s = 0.0, m = 0.0;
        for (uint32_t k = 0; k < K; ++k) {
            const double t = (double)a[k] * (double)oracle_fp16_to_float(w_bt[((size_t)(k / 8u) * V + n) * 8u + k % 8u]);
            s += t;
            m += fabs(t);
        }
        out[n] = s;
        if (absdot) absdot[n] = m;
    }
}

/* ------------------------------------------------------------------------ */
/* exp scan                                                                 */
/* ------------------------------------------------------------------------ */

static double ulp_of(float y) {
    if (y == 0.0f) return 0x1.0p-149;
    int e;
    frexpf(y, &e);
    double u = ldexp(1.0, e - 24);
    return u < 0x1.0p-149 ? 0x1.0p-149 : u;
}

uint64_t oracle_exp_scan(float lo, float hi, uint32_t acc_stride, double* max_ulp,
                        float* worst_x) {
    /* x <= 0: walk every bit pattern from hi (closest to 0) down to lo for the
     * monotonicity check; every acc_stride-th one for the error against libm. */
    uint64_t viol = 0;
    double mu = 0.0;
    float wx = 0.0f;
    uint32_t bh = pss_f2u(hi), bl = pss_f2u(lo);
    float prev = 0.0f;
    int have = 0;
    /* Negative floats: bit pattern increases as value decreases. */
    if (hi == 0.0f) bh = 0x80000000u;
    for (uint64_t b = bh; b <= bl; ++b) {
        float x = pss_u2f((uint32_t)b);
        float y = pss_exp(x);
        if (have && y > prev) viol++; /* x decreased, exp must not increase */
        prev = y;
        have = 1;
        if (acc_stride > 1 && (b % acc_stride) != 0) continue;
        double ref = exp((double)x);
        double err = fabs((double)y - ref) / ulp_of((float)ref);
        if (err > mu) {
            mu = err;
            wx = x;
        }
    }
    if (max_ulp) *max_ulp = mu;
    if (worst_x) *worst_x = wx;
    return viol;
}

/* ------------------------------------------------------------------------ */
/* Exported views of the shared deterministic helpers, for known-answer tests */
/* ------------------------------------------------------------------------ */

void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    pss_u32x4 c = {{ctr[0], ctr[1], ctr[2], ctr[3]}};
    pss_u32x4 r = pss_philox4x32_10(c, key[0], key[1]);
    for (int i = 0; i < 4; ++i) out[i] = r.v[i];
}
uint32_t oracle_xorshift32(uint32_t x) { return pss_xorshift32(x); }
uint64_t oracle_topp_need(float topP, uint64_t zk) { return pss_topp_need(topP, zk); }
uint64_t oracle_draw_target(uint32_t u24, uint64_t z) { return pss_draw_target(u24, z); }
uint32_t oracle_key(float t) { return pss_key(t); }
float oracle_unkey(uint32_t k) { return pss_unkey(k); }
float oracle_canon(float t) { return pss_canon(t); }
uint64_t oracle_fixq(float p) { return pss_fixq(p); }
float oracle_h2f(uint16_t h) { return pss_h2f(h); }
void oracle_exp_many(const float* x, float* y, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) y[i] = pss_exp(x[i]);
}
void oracle_prob_many(const float* t, float tmax, float* y, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) y[i] = pss_prob(t[i], tmax);
}
